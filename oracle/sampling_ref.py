"""Oracle: a numpy restatement of goethe_engine/sampling.py (test infrastructure; parity checker and CPU baseline).

Every function follows the reference line by line in numpy, with the same numpy primitives (fp32 division, stable
argsort, fp64 exp, pairwise sum, sequential cumsum), so on the same numpy build it reproduces the reference's bits:

  mix / uniform       sampling.py:42-51   splitmix64 of (seed, i); uniform = (mix >> 11) / 2**53
  _sorted_p           sampling.py:59-65   z = x / float32(t); stable descending order; fp64 softmax in that order
  sample              sampling.py:68-85   NaN row / all-masked row -> -1; greedy first argmax of nan_to_num;
                                          top-k AND top-p over the unfiltered q; draw = count(c < u * c[-1])
  dist                sampling.py:88-97   fp64 distribution in vocabulary order
  draw                sampling.py:100-104 inverse CDF in vocabulary order

Extensions the reference does not have (serve.py:24,133-135 and api.py:85-87 refuse them), defined here once and used
by both this oracle and the HIP path. Their parity is pinned by closed forms and brute force, not by the reference:

  penalties   c_t = occurrences of token t in the row's history (ids outside [0, V) ignored). If c_t > 0:
              repetition x = x * rp if x < 0 else x / rp (HF RepetitionPenaltyLogitsProcessor), then frequency
              x = x - fp * float32(c_t), then presence x = x - pp (vLLM apply_penalties order). Every step is a separately
              rounded fp32 operation. Penalties act before the NaN test, the mask and the temperature.
  min_p       keep_i &= q_i >= min_p * q_0 (fp64, q the unfiltered sorted distribution), AND-ed like top-k and top-p.
  logprobs    top-N of fp64 log_softmax(z) = (z - z_max) - log(sum(exp(z - z_max))) over the full row in the stable
              descending order, cast to fp32, with their token ids. z = x / float32(T) for T > 0 and z = x for T == 0.
  bf16        logits are upcast exactly to fp32 first (sampling.py:70 casts any dtype to fp32).
  uniforms    sample(..., uniforms=u) replaces uniform(seeds[r], idxs[r]) by u[r] (shared per-row draws).
"""
import numpy as np

M64 = (1 << 64) - 1
_G = 0x9E3779B97F4A7C15
_C1 = 0xBF58476D1CE4E5B9
_C2 = 0x94D049BB133111EB


def mix(seed, i):
    """splitmix64 finaliser of seed + (i + 1) * golden (sampling.py:42-47), Python big ints masked to 64 bits."""
    z = (seed + (i + 1) * _G) & M64
    z = ((z ^ (z >> 30)) * _C1) & M64
    z = ((z ^ (z >> 27)) * _C2) & M64
    return z ^ (z >> 31)


def uniform(seed, idx):
    """(mix >> 11) / 2**53 in [0, 1) (sampling.py:50-51)."""
    return (mix(seed, idx) >> 11) / float(1 << 53)


def mix_np(seed, i):
    """Vectorised mix over uint64 arrays (wrapping arithmetic), equal to mix() elementwise."""
    s = np.asarray(seed, dtype=np.uint64)
    i = np.asarray(i, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = s + (i + np.uint64(1)) * np.uint64(_G)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(_C1)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(_C2)
    return z ^ (z >> np.uint64(31))


def uniform_np(seed, idx):
    return (mix_np(seed, idx) >> np.uint64(11)).astype(np.float64) / float(1 << 53)


def _p(p, name, default):
    return getattr(p, name, default)


def as_f32(x):
    """Any logits row/batch as fp32 numpy (bf16 torch tensors are upcast exactly; sampling.py:54-56,70)."""
    if hasattr(x, "detach"):
        import torch
        t = x.detach().cpu()
        if t.dtype == torch.bfloat16:
            t = t.float()
        return np.array(t.numpy(), dtype=np.float32)
    return np.array(x, dtype=np.float32)


def as_bool(m):
    if hasattr(m, "detach"):
        m = m.detach().cpu().numpy()
    return np.asarray(m).astype(bool)


def apply_penalties(x, hist, rp=1.0, fp=0.0, pp=0.0):
    """In place on one fp32 row: repetition, then frequency, then presence, each separately rounded in fp32."""
    if hist is None:
        return x
    h = np.asarray(hist, dtype=np.int64).reshape(-1)
    v = x.shape[0]
    h = h[(h >= 0) & (h < v)]
    if h.size == 0:
        return x
    c = np.bincount(h, minlength=v)
    sel = np.nonzero(c)[0]
    xs = x[sel]
    rp32, fp32, pp32 = np.float32(rp), np.float32(fp), np.float32(pp)
    xs = np.where(xs < 0, xs * rp32, xs / rp32).astype(np.float32)
    xs = (xs - fp32 * c[sel].astype(np.float32)).astype(np.float32)
    xs = (xs - pp32).astype(np.float32)
    x[sel] = xs
    return x


def sorted_p(x, t):
    """sampling.py:59-65: (order, q) with z = x / float32(t), stable descending order, fp64 softmax in that order."""
    z = x / np.float32(t)
    order = np.argsort(-z, kind="stable")
    zs = z[order].astype(np.float64)
    e = np.exp(zs - zs[0])
    return order, e / e.sum()


def keep_mask(q, p):
    """sampling.py:80 plus min-p: prefix conditions over the unfiltered sorted q."""
    n = len(q)
    keep = (np.arange(n) < (_p(p, "top_k", 0) or n)) & (np.cumsum(q) - q < _p(p, "top_p", 1.0))
    mp = _p(p, "min_p", 0.0)
    if mp:
        keep &= q >= mp * q[0]
    return keep


def process_row(x, p, mask=None, hist=None):
    """Penalties then mask on one fp32 row; returns (x, bad) as sampling.py:70-75 computes them."""
    apply_penalties(x, hist, _p(p, "repetition_penalty", 1.0), _p(p, "frequency_penalty", 0.0),
                    _p(p, "presence_penalty", 0.0))
    bad = bool(np.isnan(x).any())
    if mask is not None:
        x[~as_bool(mask)[:x.shape[0]]] = -np.inf
    bad |= not np.isfinite(x).any()
    return x, bad


def sample(logits, params, seeds, idxs, masks, history=None, uniforms=None):
    """sampling.py:68-85, extended with per-row history (penalties), min_p and shared uniforms."""
    return [r["token"] for r in sample_full(logits, params, seeds, idxs, masks, history, uniforms)]


def sample_full(logits, params, seeds, idxs, masks, history=None, uniforms=None):
    """Per row: token, processed logits (after penalties and mask, before temperature) and top-N logprobs."""
    x = as_f32(logits)
    if x.ndim == 1:
        x = x[None]
    out = []
    for r in range(x.shape[0]):
        p = params[r]
        row = x[r].copy()
        row, bad = process_row(row, p, masks[r] if masks is not None else None,
                               history[r] if history is not None else None)
        res = dict(processed=row.copy())
        tok = -1 if bad else int(np.nan_to_num(row, nan=-np.inf).argmax())
        t = p.temperature
        if t > 0 and not bad:
            order, q = sorted_p(row, t)
            keep = keep_mask(q, p)
            c = np.cumsum(q * keep)
            u = uniforms[r] if uniforms is not None else uniform(seeds[r], idxs[r])
            j = max(min(int((c < u * c[-1]).sum()), int(keep.sum()) - 1), 0)
            tok = int(order[j])
        res["token"] = -1 if bad else tok
        n = _p(p, "logprobs", None)
        if n:
            z = row / np.float32(t) if t > 0 else row.copy()
            order = np.argsort(-z, kind="stable")
            zs = z[order].astype(np.float64)
            lp = (zs - zs[0]) - np.log(np.exp(zs - zs[0]).sum())
            k = min(n, len(order))
            res["logprob_ids"] = order[:k].astype(np.int64)
            res["logprobs"] = lp[:k].astype(np.float32)
        out.append(res)
    return out


def dist(logits, p, mask=None, history=None):
    """sampling.py:88-97 (plus penalties and min-p): fp64 probabilities in vocabulary order."""
    x = as_f32(logits).reshape(-1).copy()
    if history is not None:
        apply_penalties(x, history, _p(p, "repetition_penalty", 1.0), _p(p, "frequency_penalty", 0.0),
                        _p(p, "presence_penalty", 0.0))
    if mask is not None:
        x[~as_bool(mask)[:x.shape[0]]] = -np.inf
    order, q = sorted_p(x, p.temperature)
    q = q * keep_mask(q, p)
    out = np.zeros_like(q)
    out[order] = q / q.sum()
    return out


def draw(q, u):
    """sampling.py:100-104: min(count(cumsum(q) < u * sum), last index with q > 0), vocabulary order."""
    if hasattr(q, "detach"):
        q = q.detach().cpu().numpy()
    q = np.asarray(q)
    c = np.cumsum(q)
    return int(min(int((c < u * c[-1]).sum()), int(np.nonzero(q > 0)[0][-1])))


def unpack_mask(words, v):
    """grammar.py:44-45: token t allowed iff bit t % 32 of word t // 32 is set (LSB first), truncated to v."""
    w = np.asarray(words).astype(np.uint32)
    bits = (w[:, None] >> np.arange(32, dtype=np.uint32)) & 1
    return bits.reshape(-1)[:v].astype(bool)


def pack_mask(m):
    """Inverse of unpack_mask: bool [v] -> int32 [ceil(v / 32)] (bits past v are zero)."""
    m = np.asarray(m).astype(bool)
    v = m.shape[0]
    n = (v + 31) // 32
    b = np.zeros(n * 32, dtype=np.uint64)
    b[:v] = m
    w = (b.reshape(n, 32) << np.arange(32, dtype=np.uint64)).sum(1)
    return w.astype(np.uint32).view(np.int32)
