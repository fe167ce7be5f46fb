"""Seeded synthetic inputs for the five selection workloads (host numpy; no np.random, so any numpy gives the same
integer streams). Every draw comes from a splitmix64 stream (the same mix as goethe_engine/sampling.py:42-47), indexed
so that any row can be generated on its own: stream position = row * width + column.

  c1  B=8 V=32000 fp32 N(0, 2^2); T 0.8, top-k 40, top-p 0.95, repetition 1.1; 64-id uniform history; u_r = uniform(0, r)
  c2  B=64 V=128256 fp32 N(0, 3^2); packed mask of 20 runs (length U[200,420]) + 200 scattered ids; greedy
  c3  B=256 V=151936 fp32 N(0, 2.5^2) - 1.1 ln(1 + pi(t)) (pi a per-row permutation: the rank of token t), re-centred;
      2048-id history with ranks ~ Zipf(1.2) mapped through pi; per-row penalties, T, top-k, top-p, min-p;
      4748-word mask (rows r % 4 == 0 the c2 recipe, others all ones); u_r = uniform(1, r)
  c4  32 requests, tree parents [0,1,2,3,0,5,6,7]; target N(0, 2^2) rows for the anchor and 8 nodes; draft logits of
      the 7 nodes with kids = target row + N(0, 0.5^2); kids drawn from softmax(draft) with the SALT_DRAFT stream
  c5  B=1024 V=262144 bf16 1.5 * Gumbel(0,1) (RNE to bf16); T 1, top-p 0.9, top-20 logprobs; u_r = uniform(3, r)
"""
from dataclasses import dataclass, field

import numpy as np

from .sampling import SamplingParams, mix

_G, _C1, _C2 = 0x9E3779B97F4A7C15, 0xBF58476D1CE4E5B9, 0x94D049BB133111EB
M64 = (1 << 64) - 1


def mix_array(seed, idx):
    """splitmix64(seed, idx) elementwise over uint64 arrays (wrapping arithmetic)."""
    s = np.uint64(seed & M64)
    i = np.asarray(idx, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = s + (i + np.uint64(1)) * np.uint64(_G)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(_C1)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(_C2)
    return z ^ (z >> np.uint64(31))


def uniforms(seed, idx):
    """uniform(seed, idx) = (mix >> 11) / 2^53 for an array of indices (fp64, exact)."""
    return (mix_array(seed, idx) >> np.uint64(11)).astype(np.float64) * (1.0 / float(1 << 53))


def normals(seed, idx):
    """Box-Muller normals from two interleaved streams (2k, 2k + 1) of one seed, fp64."""
    i = np.asarray(idx, dtype=np.uint64) * np.uint64(2)
    u1 = 1.0 - uniforms(seed, i)
    u2 = uniforms(seed, i + np.uint64(1))
    return np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)


def to_bf16_bits(x):
    """fp32 -> bf16 bits, round to nearest even (finite inputs)."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    b = (b + np.uint64(0x7FFF) + ((b >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    return b.astype(np.uint16)


def bf16_bits_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def pack_bits(m):
    """bool [rows, V] -> int32 [rows, ceil(V / 32)], token t is bit t % 32 of word t // 32."""
    m = np.asarray(m, dtype=bool)
    rows, v = m.shape
    n = (v + 31) // 32
    b = np.zeros((rows, n * 32), dtype=np.uint32)
    b[:, :v] = m
    w = (b.reshape(rows, n, 32) << np.arange(32, dtype=np.uint32)).sum(2, dtype=np.uint64)
    return w.astype(np.uint32).view(np.int32)


def grammar_mask(seed, r, v, runs=20, lo=200, hi=420, scattered=200):
    """One row of the grammar-mask recipe: `runs` contiguous runs of length U[lo, hi] plus scattered ids."""
    u = uniforms(seed, np.arange(r * 4096, r * 4096 + 2 * runs + scattered, dtype=np.uint64))
    m = np.zeros(v, dtype=bool)
    for k in range(runs):
        ln = lo + int(u[2 * k] * (hi - lo + 1))
        st = int(u[2 * k + 1] * max(1, v - ln))
        m[st:st + ln] = True
    m[(u[2 * runs:] * v).astype(np.int64)] = True
    if not m.any():
        m[0] = True
    return m


@dataclass
class Batch:
    """A selection batch: logits (fp32 numpy, or bf16 bits as uint16), per-row params, masks, histories, uniforms."""
    name: str
    logits: np.ndarray
    params: list
    uniforms: np.ndarray
    masks: np.ndarray = None          # int32 [B, words] packed, or None
    history: list = None              # per row int32 ids or None
    bf16: bool = False
    extra: dict = field(default_factory=dict)

    @property
    def rows(self):
        return self.logits.shape[0]

    @property
    def vocab(self):
        return self.logits.shape[1]

    def logits_f32(self):
        return bf16_bits_to_f32(self.logits) if self.bf16 else self.logits

    def bytes_per_row(self):
        """Algorithmic bytes of one row: one read of the logits, mask words, history ids; 4 B token out, 8 B per logprob."""
        s = 2 if self.bf16 else 4
        v = self.vocab
        b = s * v + 4
        if self.masks is not None:
            b += 4 * ((v + 31) // 32)
        if self.history is not None:
            b += 4 * int(np.mean([len(h) for h in self.history]))
        n = self.params[0].logprobs or 0
        return b + 8 * n


def c1(rows=None):
    b, v = 8, 32000
    rows = range(b) if rows is None else rows
    x = np.stack([(2.0 * normals(0, np.arange(r * v, (r + 1) * v, dtype=np.uint64))).astype(np.float32) for r in rows])
    hist = [(uniforms(0x51, np.arange(r * 64, (r + 1) * 64, dtype=np.uint64)) * v).astype(np.int32) for r in rows]
    p = [SamplingParams(temperature=0.8, top_k=40, top_p=0.95, repetition_penalty=1.1) for _ in rows]
    return Batch("c1", x, p, uniforms(0, np.array(list(rows), dtype=np.uint64)), None, hist)


def c2(rows=None, b=64, v=128256):
    rows = range(b) if rows is None else rows
    x = np.stack([(3.0 * normals(1000, np.arange(r * v, (r + 1) * v, dtype=np.uint64))).astype(np.float32) for r in rows])
    m = pack_bits(np.stack([grammar_mask(1001, r, v) for r in rows]))
    p = [SamplingParams() for _ in rows]
    return Batch("c2", x, p, np.zeros(len(rows)), m, None)


def _perm(seed, r, v):
    """A seeded permutation: pi[t] = rank of token t (argsort of a uniform stream), and its inverse."""
    u = mix_array(seed, np.arange(r * v, (r + 1) * v, dtype=np.uint64))
    inv = np.argsort(u, kind="stable")          # inv[rank] = token
    pi = np.empty(v, dtype=np.int64)
    pi[inv] = np.arange(v)
    return pi, inv


def zipf_ranks(seed, n, v, s, offset=0):
    cdf = np.cumsum(np.power(np.arange(1, v + 1, dtype=np.float64), -s))
    u = uniforms(seed, np.arange(offset, offset + n, dtype=np.uint64)) * cdf[-1]
    return np.minimum(np.searchsorted(cdf, u, side="right"), v - 1)


C3_TOPK = (0, 20, 50, 200)


def c3_params(r):
    u = uniforms(2000, np.arange(r * 8, r * 8 + 8, dtype=np.uint64))
    return SamplingParams(temperature=float(0.5 + u[0]), top_k=C3_TOPK[int(u[1] * 4)], top_p=float(0.8 + 0.2 * u[2]),
                          min_p=(0.0, 0.05)[int(u[3] * 2)], frequency_penalty=float(u[4]),
                          presence_penalty=float(u[5]), repetition_penalty=float(1.0 + 0.3 * u[6]))


def c3(rows=None, b=256, v=151936, h=2048):
    rows = range(b) if rows is None else rows
    xs, hist, ms = [], [], []
    for r in rows:
        pi, inv = _perm(3000, r, v)
        x = 2.5 * normals(3001, np.arange(r * v, (r + 1) * v, dtype=np.uint64)) - 1.1 * np.log1p(pi)
        xs.append((x - x.mean()).astype(np.float32))
        hist.append(inv[zipf_ranks(3002, h, v, 1.2, offset=r * h)].astype(np.int32))
        ms.append(grammar_mask(3003, r, v) if r % 4 == 0 else np.ones(v, dtype=bool))
    p = [c3_params(r) for r in rows]
    return Batch("c3", np.stack(xs), p, uniforms(1, np.array(list(rows), dtype=np.uint64)), pack_bits(np.stack(ms)), hist)


C4_PARENTS = [0, 1, 2, 3, 0, 5, 6, 7]
SALT_DRAFT = 1 << 42


def c4(requests=None, n_req=32, v=128256):
    """Per request: target fp32 [9, V], draft fp32 [9, V] (rows of nodes with kids filled, others zero), tokens [8],
    seed. Kids of node u are drawn from softmax(draft[u]) (fp64) at uniform(mix(seed, SALT_DRAFT + k), depth(u))."""
    requests = range(n_req) if requests is None else requests
    kids = [[] for _ in range(9)]
    for j, par in enumerate(C4_PARENTS):
        kids[par].append(j + 1)
    depth = [0] * 9
    for j, par in enumerate(C4_PARENTS):
        depth[j + 1] = depth[par] + 1
    out = []
    for q in requests:
        base = q * 9 * v
        tgt = (2.0 * normals(4000, np.arange(base, base + 9 * v, dtype=np.uint64))).astype(np.float32).reshape(9, v)
        noise = (0.5 * normals(4001, np.arange(base, base + 9 * v, dtype=np.uint64))).astype(np.float32).reshape(9, v)
        drf = np.zeros_like(tgt)
        seed = mix(2, q)
        toks = [0] * 8
        for u in range(9):
            if not kids[u]:
                continue
            drf[u] = tgt[u] + noise[u]
            z = drf[u].astype(np.float64)
            e = np.exp(z - z.max())
            qd = e / e.sum()
            c = np.cumsum(qd)
            for k, node in enumerate(kids[u]):
                uu = (mix(mix(seed, SALT_DRAFT + k), depth[u]) >> 11) / float(1 << 53)
                toks[node - 1] = int(min(int((c < uu * c[-1]).sum()), int(np.nonzero(qd > 0)[0][-1])))
        out.append(dict(target=tgt, draft=drf, tokens=toks, parents=list(C4_PARENTS), seed=seed,
                        params=SamplingParams(temperature=1.0, accept="rejection")))
    return out


def c5(rows=None, b=1024, v=262144):
    rows = range(b) if rows is None else rows
    xs = []
    for r in rows:
        k = mix_array(5000, np.arange(r * v, (r + 1) * v, dtype=np.uint64)) >> np.uint64(11)
        u = (k.astype(np.float64) + 0.5) * (1.0 / float(1 << 53))      # open interval (0, 1)
        xs.append(to_bf16_bits((1.5 * -np.log(-np.log(u))).astype(np.float32)))
    p = [SamplingParams(temperature=1.0, top_p=0.9, logprobs=20) for _ in rows]
    return Batch("c5", np.stack(xs), p, uniforms(3, np.array(list(rows), dtype=np.uint64)), None, None, bf16=True)


CONFIGS = dict(c1=c1, c2=c2, c3=c3, c5=c5)
