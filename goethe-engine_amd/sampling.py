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


def _rows(params, seeds, idxs, hist_offsets):
    n = len(params)
    r = np.zeros(n, dtype=_lib.ROW)
    for i, p in enumerate(params):
        t = float(p.temperature)
        t32 = np.float32(t)
        r["temperature"][i] = t32
        if t > 0 and t32 == 0:
            r["flags"][i] = _lib.ROW_TEMP_UNDERFLOW
        r["top_k"][i] = min(int(_get(p, "top_k", 0)), 0x7FFFFFFF)
        r["top_p"][i] = float(_get(p, "top_p", 1.0))
        r["min_p"][i] = float(_get(p, "min_p", 0.0))
        r["repetition_penalty"][i] = np.float32(_get(p, "repetition_penalty", 1.0))
        r["frequency_penalty"][i] = np.float32(_get(p, "frequency_penalty", 0.0))
        r["presence_penalty"][i] = np.float32(_get(p, "presence_penalty", 0.0))
        r["logprobs"][i] = int(_get(p, "logprobs", 0))
        r["seed"][i] = (int(seeds[i]) & M64) if seeds is not None and seeds[i] is not None else 0
        r["idx"][i] = (int(idxs[i]) & M64) if idxs is not None and idxs[i] is not None else 0
    r["mask_row"] = -1
    if hist_offsets is not None:
        r["hist_begin"] = hist_offsets[:-1]
        r["hist_end"] = hist_offsets[1:]
    return r


def _masks(h, masks, n, v, dev, rows):
    """Per-row masks (None, bool [V] or packed int32 [>= ceil(V / 32)]), or a grammar.MaskBatch -> device words [k, W]
    and rows' mask_row."""
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
    packed, bools, where = [], [], []
    for i in range(n):
        m = masks[i]
        if m is None:
            continue
        mt = m if isinstance(m, torch.Tensor) else torch.from_numpy(np.asarray(m))
        if mt.dtype in (torch.int32, torch.uint32) and mt.numel() >= words and mt.numel() < v:
            packed.append((i, mt.reshape(-1)[:words].view(torch.int32) if mt.dtype == torch.uint32 else
                           mt.reshape(-1)[:words]))
        else:
            if mt.numel() != v:
                raise ValueError(f"mask of row {i} has {mt.numel()} entries, the row has {v} tokens")
            bools.append((i, mt.reshape(-1).to(torch.bool)))
    if not packed and not bools:
        return None, 0
    out = torch.empty((len(packed) + len(bools), words), dtype=torch.int32, device=dev)
    k = 0
    for i, mt in packed:
        out[k].copy_(mt.to(dev, non_blocking=True))
        rows["mask_row"][i] = k
        k += 1
    if bools:
        b = torch.stack([mt for _, mt in bools]).to(dev, non_blocking=True).to(torch.uint8)
        h.ck(h.L.gse_pack_mask(h.h, _lib.ptr(b), b.stride(0), len(bools), v, _lib.ptr(out[k:]), words,
                               _lib.stream_of(dev.index)), "gse_pack_mask")
        for j, (i, _) in enumerate(bools):
            rows["mask_row"][i] = k + j
    return out, words


def _history(history, n, dev):
    if history is None:
        return None, None
    parts, offs = [], [0]
    for i in range(n):
        hi = history[i] if i < len(history) else None
        if hi is None:
            offs.append(offs[-1])
            continue
        a = hi.detach().cpu().numpy() if isinstance(hi, torch.Tensor) else np.asarray(hi)
        a = a.astype(np.int64).reshape(-1)
        a = a[(a >= 0) & (a < 0x7FFFFFFF)].astype(np.int32)
        parts.append(a)
        offs.append(offs[-1] + len(a))
    if offs[-1] == 0:
        return None, None
    ids = torch.from_numpy(np.concatenate(parts)).to(dev, non_blocking=True)
    return ids, np.asarray(offs, dtype=np.int64)


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
    hist_dev, offs = _history(history, n, dev)
    rows = _rows(params, seeds, idxs, offs)
    mask_dev, mask_ld = _masks(h, masks, n, v, dev, rows)
    rows_dev = torch.from_numpy(rows.view(np.uint8)).to(dev, non_blocking=True)
    uni_dev = None
    if uniforms is not None:
        u = uniforms if isinstance(uniforms, torch.Tensor) else torch.from_numpy(np.asarray(uniforms, np.float64))
        uni_dev = u.to(dev, torch.float64).reshape(-1).contiguous()
    keep = (x, rows_dev, mask_dev, hist_dev, uni_dev)
    return h, x, code, dev, _batch(x, code, rows_dev, mask_dev, mask_ld, hist_dev, uni_dev, dev), keep


def _sample_flags(params):
    """GSE_BATCH_* bits the drop-in adds to a gse_sample call: NO_SPLIT when every row is greedy (temperature 0 as
    float32, as the device decides), since greedy rows never take the split-row finish and its launch is saved."""
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
    b.flags |= int(flags) | _sample_flags(params)
    nlp = max([int(_get(p, "logprobs", 0)) for p in params] + [0])
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
    h.ck(h.L.gse_sample(h.h, C.byref(b), C.byref(o)), "gse_sample")
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
    h.ck(h.L.gse_dist(h.h, C.byref(b), out.data_ptr(), v), "gse_dist")
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
    h.ck(h.L.gse_draw(h.h, qt.data_ptr(), qt.numel(), 1, qt.numel(), ut.data_ptr(), out.data_ptr(),
                      _lib.stream_of(dev.index)), "gse_draw")
    j = int(out.item())
    if j < 0:
        raise IndexError("draw: no token has positive probability")
    return j
