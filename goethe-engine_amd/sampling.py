"""MI355X drop-in for goethe_engine/sampling.py: the same call surface, the arithmetic in libgse.so (HIP, gfx950).

  SamplingParams / validate   sampling.py:8-39, extended with neutral-default fields: repetition_penalty=1.0,
                              frequency_penalty=0.0, presence_penalty=0.0, min_p=0.0, logprobs=None
  mix / uniform / host        sampling.py:42-56 (host integer helpers the engine also calls, engine.py:208)
  sample                      sampling.py:68-85  -> gse_sample (one fused pass; token -1 for a row without a finite
                              choice); keyword additions: history= (per-row token ids for the penalties),
                              uniforms= (shared per-row draws instead of uniform(seed, idx)), exact= (finish every row
                              on the exact radix-select path)
  dist                        sampling.py:88-97  -> gse_dist
  draw                        sampling.py:100-104 -> gse_draw

Logits may be torch tensors on the GPU (used in place, fp32 or bf16, any row stride), CPU tensors or numpy arrays
(copied to the GPU first). There is no CPU path: without a HIP device every call raises RuntimeError.
"""
import ctypes as C
import weakref
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib

M64 = (1 << 64) - 1


@dataclass(frozen=True)
class SamplingParams:
    temperature: float = 0.0
    top_p: float = 1.0
    top_k: int = 0
    seed: int | None = None
    max_tokens: int = 16
    stop_token_ids: tuple = ()
    stop_sequences: tuple = ()
    ignore_eos: bool = False
    n: int = 1
    grammar: tuple | None = None  # (kind, spec), see grammar.py
    priority: int = 0
    accept: str = "exact"  # speculative acceptance at temperature > 0: exact (seeded sample match) | rejection
    repetition_penalty: float = 1.0
    frequency_penalty: float = 0.0
    presence_penalty: float = 0.0
    min_p: float = 0.0
    logprobs: int | None = None

    def validate(self):
        if not (self.temperature >= 0 and self.temperature < float("inf")):
            raise ValueError("temperature must be finite and >= 0")
        if not 0 < self.top_p <= 1:
            raise ValueError("top_p must be in (0, 1]")
        if self.top_k < 0:
            raise ValueError("top_k must be >= 0")
        if self.max_tokens < 1:
            raise ValueError("max_tokens must be >= 1")
        if self.n < 1:
            raise ValueError("n must be >= 1")
        if self.n > 1 and self.temperature == 0:
            raise ValueError("n > 1 needs temperature > 0")
        if any(len(s) == 0 for s in self.stop_sequences):
            raise ValueError("empty stop sequence")
        if self.accept not in ("exact", "rejection"):
            raise ValueError("accept must be exact or rejection")
        if not (self.repetition_penalty > 0 and self.repetition_penalty < float("inf")):
            raise ValueError("repetition_penalty must be finite and > 0")
        if not (abs(self.frequency_penalty) < float("inf") and abs(self.presence_penalty) < float("inf")):
            raise ValueError("frequency_penalty and presence_penalty must be finite")
        if not 0 <= self.min_p <= 1:
            raise ValueError("min_p must be in [0, 1]")
        if self.logprobs is not None and not 0 <= self.logprobs <= _lib.MAX_LOGPROBS:
            raise ValueError(f"logprobs must be in [0, {_lib.MAX_LOGPROBS}]")


def mix(seed, i):
    """splitmix64 of (seed, i): the child seed or the uniform stream of a request."""
    z = (seed + (i + 1) * 0x9E3779B97F4A7C15) & M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


def uniform(seed, idx):
    return (mix(seed, idx) >> 11) / float(1 << 53)


def host(x):
    """A numpy view of logits / masks / probabilities from any backend (numpy, or a torch tensor)."""
    return x.detach().cpu().numpy() if hasattr(x, "detach") else np.asarray(x)


# ---- device plumbing ----------------------------------------------------------------------------------------------------

def _device():
    if not torch.cuda.is_available():
        raise RuntimeError("goethe-engine_amd needs a HIP device (torch.cuda.is_available() is False)")
    return torch.device("cuda", torch.cuda.current_device())


def _logits(x):
    """[B, V] logits on the GPU with unit column stride: (tensor, dtype code)."""
    if not isinstance(x, torch.Tensor):
        x = torch.from_numpy(np.ascontiguousarray(np.asarray(x, dtype=np.float32)))
    if x.dim() == 1:
        x = x.unsqueeze(0)
    if x.device.type != "cuda":
        x = x.to(_device(), non_blocking=False)
    if x.dtype == torch.bfloat16:
        code = _lib.BF16
    else:
        if x.dtype != torch.float32:
            x = x.float()
        code = _lib.F32
    if x.stride(1) != 1 or x.stride(0) < x.shape[1] or x.storage_offset() < 0:
        x = x.contiguous()
    return x, code


def _get(p, name, default):
    v = getattr(p, name, default)
    return default if v is None else v


# Row templates: the 72-byte gse_row of a params object's fields (seed, idx and history range left zero, mask_row -1),
# kept per live frozen params object. A request's SamplingParams is one frozen object for its whole life (the engine
# passes s.params every step), so a step's rows are a join of cached templates and a few vectorised columns.
_tmpl = {}


def _template(p):
    e = _tmpl.get(id(p))
    if e is not None and e[0]() is p:
        return e[1]
    r = np.zeros(1, dtype=_lib.ROW)
    t = float(p.temperature)
    t32 = np.float32(t)
    r["temperature"] = t32
    r["flags"] = _lib.ROW_TEMP_UNDERFLOW if t > 0 and t32 == 0 else 0
    r["top_k"] = min(int(_get(p, "top_k", 0)), 0x7FFFFFFF)
    r["top_p"] = float(_get(p, "top_p", 1.0))
    r["min_p"] = float(_get(p, "min_p", 0.0))
    r["repetition_penalty"] = np.float32(_get(p, "repetition_penalty", 1.0))
    r["frequency_penalty"] = np.float32(_get(p, "frequency_penalty", 0.0))
    r["presence_penalty"] = np.float32(_get(p, "presence_penalty", 0.0))
    r["logprobs"] = int(_get(p, "logprobs", 0))
    r["mask_row"] = -1
    b = r.tobytes()
    dp = getattr(p, "__dataclass_params__", None)
    if dp is not None and dp.frozen:  # (a mutable params object is read afresh every call)
        try:
            ref = weakref.ref(p, lambda _, k=id(p): _tmpl.pop(k, None))
        except TypeError:
            return b
        _tmpl[id(p)] = (ref, b)
    return b


def _u64_col(vals, n):
    """A uint64 column from per-row Python ints (taken mod 2^64) or None (0)."""
    if vals is None:
        return np.zeros(n, np.uint64)
    try:
        return np.fromiter(vals, np.uint64, n)
    except (TypeError, OverflowError, ValueError):
        return np.array([(int(v) & M64) if v is not None else 0 for v in vals], np.uint64)


def _rows(params, seeds, idxs, hist_range):
    """gse_row records of the rows: params fields, seeds and idxs (mod 2^64, None -> 0), mask_row -1, and the history
    range of each row: hist_range is None, CSR offsets [n + 1], or (begin [n], end [n])."""
    n = len(params)
    r = np.frombuffer(b"".join([_template(p) for p in params]), dtype=_lib.ROW).copy() if n else \
        np.zeros(0, dtype=_lib.ROW)
    r["seed"] = _u64_col(seeds, n)
    r["idx"] = _u64_col(idxs, n)
    if hist_range is not None:
        if isinstance(hist_range, tuple):
            r["hist_begin"], r["hist_end"] = hist_range
        else:
            r["hist_begin"] = hist_range[:-1]
            r["hist_end"] = hist_range[1:]
    return r


def _masks(h, masks, n, v, dev, rows):
    """Per-row masks (None, bool [V] or packed int32 [>= ceil(V / 32)], torch or numpy), or a grammar.MaskBatch ->
    device words [k, W] and rows' mask_row. Packed rows go to the device in one copy, bool rows in one copy and one
    pack launch."""
    if masks is None:
        return None, 0
    words = (v + 31) // 32
    if getattr(masks, "is_mask_batch", False):  # grammar.MaskBatch: every row's words in one host buffer, one copy
        if masks.rows < n or masks.vocab != v:
            raise ValueError(f"mask batch of {masks.rows} x {masks.vocab}, the logits are {n} x {v}")
        if not masks.filled[:n].any():
            return None, 0
        idx = np.nonzero(masks.filled[:n])[0]
        rows["mask_row"][idx] = idx
        return masks.device_words(dev, n), masks.words
    pk_i, pk, bo_i, bo = [], [], [], []
    for i in range(n):
        m = masks[i] if i < len(masks) else None
        if m is None:
            continue
        if not isinstance(m, torch.Tensor):
            m = torch.from_numpy(np.asarray(m))
        size = m.numel()
        if m.dtype in _PACKED and words <= size < v:
            pk_i.append(i)
            pk.append(m if size == words and m.dim() == 1 else m.reshape(-1)[:words])
        elif size == v:
            bo_i.append(i)
            bo.append(m if m.dim() == 1 else m.reshape(-1))
        else:
            raise ValueError(f"mask of row {i} has {size} entries, the row has {v} tokens")
    if not pk and not bo:
        return None, 0
    out = torch.empty((len(pk) + len(bo), words), dtype=torch.int32, device=dev)
    if pk:
        out[:len(pk)].copy_(_stack(pk, dev).view(torch.int32))
        rows["mask_row"][pk_i] = np.arange(len(pk), dtype=np.int32)
    if bo:
        t = _stack(bo, dev)
        b = t.view(torch.uint8) if t.dtype == torch.bool else (t != 0).to(torch.uint8)
        h.call("gse_pack_mask", _lib.ptr(b), b.stride(0), len(bo), v, _lib.ptr(out[len(pk):]), words,
               _lib.stream_of(dev.index))
        rows["mask_row"][bo_i] = len(pk) + np.arange(len(bo), dtype=np.int32)
    return out, words


_PACKED = (torch.int32, torch.uint32)


def _stack(rows, dev):
    """Equal-length 1-D tensors as one [k, n] tensor on dev: stacked where they are, then one copy."""
    t = torch.stack(rows) if len({r.device for r in rows}) == 1 else torch.stack([r.cpu() for r in rows])
    return t.to(dev, non_blocking=True)


class History:
    """Penalty histories resident on the device: row r's token ids are ids[r, :length[r]] of an int32 [rows, capacity]
    device tensor. sample(..., history=h) reads them in place (each row's range in the buffer, no copy); append() adds
    one token per row on the device, as an engine does after each step. For the engine's own layout (a list of per-row
    token sequences) sample() builds the same ranges from one concatenation."""

    is_history = True

    def __init__(self, rows, capacity, device=None):
        dev = device if device is not None else _device()
        self.ids = torch.full((int(rows), int(capacity)), -1, dtype=torch.int32, device=dev)
        self.length = np.zeros(int(rows), np.int64)

    def set(self, row, ids):
        """Row `row`'s history (its first capacity ids kept)."""
        t = ids if isinstance(ids, torch.Tensor) else torch.from_numpy(np.asarray(ids, dtype=np.int64))
        t = t.reshape(-1)[:self.ids.shape[1]]
        self.ids[row, :t.numel()].copy_(t.to(self.ids.device, torch.int32), non_blocking=True)
        self.length[row] = t.numel()

    def append(self, tokens):
        """One token more for each of the first len(tokens) rows (device tensor or list); rows at capacity keep theirs."""
        n = len(tokens)
        room = np.nonzero(self.length[:n] < self.ids.shape[1])[0]
        if not len(room):
            return
        t = tokens if isinstance(tokens, torch.Tensor) else torch.tensor(list(tokens), dtype=torch.int32)
        t = t.to(self.ids.device, torch.int32)
        ri = torch.from_numpy(room).to(self.ids.device)
        ci = torch.from_numpy(self.length[room]).to(self.ids.device)
        self.ids[ri, ci] = t[ri]
        self.length[room] += 1

    def ranges(self, n):
        """(begin, end) of the first n rows in the flattened buffer."""
        cap = self.ids.shape[1]
        begin = np.arange(n, dtype=np.int64) * cap
        return begin, begin + self.length[:n]


def _history(history, n, dev):
    """The rows' penalty histories as a device id buffer and each row's (begin, end) in it: None; a History (used in
    place); a CSR pair (ids, offsets [n + 1]); or per-row id sequences (None: no history), concatenated on the host, or on
    the device when every row is a device tensor. Ids outside [0, vocab) are ignored by the library."""
    if history is None:
        return None, None
    if getattr(history, "is_history", False):
        if history.ids.shape[0] < n:
            raise ValueError(f"history of {history.ids.shape[0]} rows for {n} rows")
        return history.ids.reshape(-1), history.ranges(n)
    if isinstance(history, tuple) and len(history) == 2:
        ids, offs = history
        offs = np.asarray(offs, dtype=np.int64)
        if offs.shape != (n + 1,):
            raise ValueError(f"history offsets must have {n + 1} entries")
        if offs[-1] == 0:
            return None, None
        t = ids if isinstance(ids, torch.Tensor) else torch.from_numpy(np.asarray(ids))
        return t.to(dev, torch.int32, non_blocking=True).reshape(-1), offs
    rows = [history[i] if i < len(history) else None for i in range(n)]
    lens = np.array([0 if h is None else (h.numel() if isinstance(h, torch.Tensor) else len(h)) for h in rows],
                    np.int64)
    if lens.sum() == 0:
        return None, None
    offs = np.zeros(n + 1, np.int64)
    np.cumsum(lens, out=offs[1:])
    live = [h for h, k in zip(rows, lens) if k]
    if all(isinstance(h, torch.Tensor) and h.device.type == "cuda" for h in live):
        ids = torch.cat([h.reshape(-1) for h in live]).to(dev)
        if ids.dtype != torch.int32:
            ids = torch.where((ids >= 0) & (ids < 0x7FFFFFFF), ids, torch.full_like(ids, -1)).to(torch.int32)
        return ids, offs
    a = np.concatenate([h.detach().cpu().numpy().reshape(-1) if isinstance(h, torch.Tensor) else
                        np.asarray(h).reshape(-1) for h in live])
    if a.dtype != np.int32:
        a = a.astype(np.int64)
        a = np.where((a >= 0) & (a < 0x7FFFFFFF), a, -1).astype(np.int32)
    return torch.from_numpy(a).to(dev, non_blocking=True), offs


class Selection:
    """Device results of one gse_sample call: tokens [B] int32, optional logprob ids / values [B, N], processed [B, V]."""

    def __init__(self, tokens, logprob_ids=None, logprobs=None, processed=None):
        self.tokens, self.logprob_ids, self.logprobs, self.processed = tokens, logprob_ids, logprobs, processed

    def tolist(self):
        return [int(t) for t in self.tokens.cpu().tolist()]


def _batch(x, code, rows_dev, mask_dev, mask_ld, hist_dev, uni_dev, dev, flags=0):
    b = _lib.Batch()
    b.size = C.sizeof(_lib.Batch)
    b.dtype = code
    b.rows, b.vocab = x.shape[0], x.shape[1]
    b.ld = x.stride(0)
    b.logits = x.data_ptr()
    b.params = rows_dev.data_ptr()
    b.mask = mask_dev.data_ptr() if mask_dev is not None else None
    b.mask_ld = mask_ld
    b.hist = hist_dev.data_ptr() if hist_dev is not None else None
    b.uniforms = uni_dev.data_ptr() if uni_dev is not None else None
    b.stream = torch.cuda.current_stream(dev).cuda_stream
    b.flags = flags
    return b


def _prepare(logits, params, seeds, idxs, masks, history, uniforms):
    x, code = _logits(logits)
    n, v = x.shape
    if len(params) != n:
        raise ValueError(f"{len(params)} params for {n} rows")
    dev = x.device
    h = _lib.handle(dev.index, n, v)
    hist_dev, hrange = _history(history, n, dev)
    rows = _rows(params, seeds, idxs, hrange)
    mask_dev, mask_ld = _masks(h, masks, n, v, dev, rows)
    rows_dev = torch.from_numpy(rows.view(np.uint8)).to(dev, non_blocking=True)
    uni_dev = None
    if uniforms is not None:
        u = uniforms if isinstance(uniforms, torch.Tensor) else torch.from_numpy(np.asarray(uniforms, np.float64))
        uni_dev = u.to(dev, torch.float64).reshape(-1).contiguous()
    keep = (x, rows_dev, mask_dev, hist_dev, uni_dev, rows)
    return h, x, code, dev, _batch(x, code, rows_dev, mask_dev, mask_ld, hist_dev, uni_dev, dev), keep


def _sample_flags(params, rows=None):
    """GSE_BATCH_* bits the drop-in adds to a gse_sample call: NO_SPLIT when every row is greedy (temperature 0 as
    float32, as the device decides), since greedy rows never take the split-row finish and its launch is saved."""
    if rows is not None:
        greedy = (rows["temperature"] == 0) & ((rows["flags"] & _lib.ROW_TEMP_UNDERFLOW) == 0)
        return _lib.BATCH_NO_SPLIT if len(rows) and bool(greedy.all()) else 0
    return _lib.BATCH_NO_SPLIT if params and all(float(p.temperature) == 0.0 for p in params) else 0


def sample_ex(logits, params, seeds, idxs, masks, history=None, uniforms=None, exact=False, processed=False,
              flags=0):
    """gse_sample on the current stream, asynchronously: a Selection of device tensors. flags adds GSE_BATCH_* bits
    (testing: BATCH_NO_PLAN_WAIT)."""
    x, _ = _logits(logits)
    n, v = x.shape
    dev = x.device if n else None
    if n == 0:
        return Selection(torch.zeros(0, dtype=torch.int32))
    h, x, code, dev, b, keep = _prepare(x, params, seeds, idxs, masks, history, uniforms)
    if exact:
        b.flags |= _lib.BATCH_EXACT
    rows = keep[5]
    b.flags |= int(flags) | _sample_flags(params, rows)
    nlp = min(int(rows["logprobs"].max()), _lib.MAX_LOGPROBS) if n else 0
    toks = torch.empty(n, dtype=torch.int32, device=dev)
    o = _lib.Out()
    o.size = C.sizeof(_lib.Out)
    o.tokens = toks.data_ptr()
    lp_ids = lps = proc = None
    if nlp:
        lp_ids = torch.empty((n, nlp), dtype=torch.int32, device=dev)
        lps = torch.empty((n, nlp), dtype=torch.float32, device=dev)
        o.logprob_ids, o.logprobs, o.logprobs_ld = lp_ids.data_ptr(), lps.data_ptr(), nlp
    if processed:
        proc = torch.empty((n, v), dtype=torch.float32, device=dev)
        o.processed, o.processed_ld = proc.data_ptr(), v
    h.call("gse_sample", C.byref(b), C.byref(o))
    sel = Selection(toks, lp_ids, lps, proc)
    sel._keep = keep
    return sel


def sample(logits, params, seeds, idxs, masks, history=None, uniforms=None, exact=False):
    """Token per row, -1 for a row without a finite choice. A row depends only on its logits, params, seed and token
    index (and, with the extensions, its history and shared uniform)."""
    return sample_ex(logits, params, seeds, idxs, masks, history, uniforms, exact).tolist()


def dist_batch(logits, params, masks=None, history=None):
    """fp64 [B, V] device tensor: dist() of every row."""
    x, code = _logits(logits)
    n, v = x.shape
    h, x, code, dev, b, keep = _prepare(x, params, None, None, masks, history, None)
    out = torch.empty((n, v), dtype=torch.float64, device=dev)
    h.call("gse_dist", C.byref(b), out.data_ptr(), v)
    return out


def dist(logits, p, mask=None, history=None):
    """float64 probabilities over the vocabulary that sample() draws a temperature > 0 row from (top-k, top-p, mask).
    A GPU tensor in, a GPU tensor out; otherwise numpy out."""
    on_gpu = isinstance(logits, torch.Tensor) and logits.device.type == "cuda"
    out = dist_batch(logits, [p], [mask] if mask is not None else None,
                     [history] if history is not None else None)[0]
    return out if on_gpu else out.cpu().numpy()


def draw(q, u):
    """Inverse CDF of probabilities q (vocabulary order) at u in [0, 1)."""
    qt = q if isinstance(q, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(np.asarray(q, np.float64)))
    if qt.device.type != "cuda":
        qt = qt.to(_device())
    qt = qt.to(torch.float64).reshape(-1).contiguous()
    dev = qt.device
    h = _lib.handle(dev.index, 1, qt.numel())
    ut = torch.tensor([float(u)], dtype=torch.float64, device=dev)
    out = torch.empty(1, dtype=torch.int32, device=dev)
    h.call("gse_draw", qt.data_ptr(), qt.numel(), 1, qt.numel(), ut.data_ptr(), out.data_ptr(),
                      _lib.stream_of(dev.index))
    j = int(out.item())
    if j < 0:
        raise IndexError("draw: no token has positive probability")
    return j
