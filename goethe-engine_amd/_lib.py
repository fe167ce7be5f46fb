"""ctypes binding of libgse.so (include/gse.h), in the style of goethe_engine/gc_c.py:58-77 (bind with an ABI check,
size-first structs) and gc_c.py:222-227 (a negative return code becomes RuntimeError with the library's last error).

torch is imported before the library is loaded so that libgse.so binds to the HIP runtime torch already mapped (both
carry the soname libamdhip64.so.7): one runtime, so torch's streams and device pointers are valid in libgse calls.
"""
import ctypes as C
import os
import threading
from collections import OrderedDict

import numpy as np
import torch

ABI_MAJOR, ABI_MINOR = 1, 4
PATH_MAIN, PATH_DEEP, PATH_EXACT = 0, 1, 2  # gse_row_paths codes
OK, E_ARG, E_DEVICE, E_UNSUPPORTED, E_CAPACITY = 0, -1, -4, -5, -7
F32, BF16 = 0, 1
ROW_TEMP_UNDERFLOW = 1
ROW_MSS = 2
Q_PROB, Q_LOGITS_F32, Q_LOGITS_BF16 = 0, 1, 2
WALK_OK, WALK_ERROR, WALK_TRUNCATED, WALK_KIDS = 0, 1, 2, 3
MAX_KIDS = 16
NOALLOC_ROWS, NOALLOC_VOCAB = 32, 163840
BATCH_EXACT = 1
BATCH_PROFILE = 2
BATCH_NO_PLAN_WAIT = 4
BATCH_NO_SPLIT = 8  # (ABI 1.3)
BATCH_SUBBIN_FINISH = 16  # (ABI 1.4, testing)
MAX_LOGPROBS = 64
P_ = C.POINTER

PATH = os.environ.get("GSE_LIB", os.path.join(os.path.dirname(os.path.abspath(__file__)), "libgse.so"))

# gse_row (72 bytes): the per-row parameter record, built as a numpy structured array and copied to the device.
ROW = np.dtype({
    "names": ["temperature", "top_k", "top_p", "min_p", "repetition_penalty", "frequency_penalty",
              "presence_penalty", "mask_row", "seed", "idx", "hist_begin", "hist_end", "logprobs", "flags"],
    "formats": [np.float32, np.int32, np.float64, np.float64, np.float32, np.float32, np.float32, np.int32,
                np.uint64, np.uint64, np.int32, np.int32, np.int32, np.uint32],
    "offsets": [0, 4, 8, 16, 24, 28, 32, 36, 40, 48, 56, 60, 64, 68],
    "itemsize": 72})


class OpenParams(C.Structure):
    _fields_ = [("size", C.c_uint32), ("device", C.c_int32), ("max_rows", C.c_uint32), ("max_vocab", C.c_uint32)]


class Batch(C.Structure):
    _fields_ = [("size", C.c_uint32), ("dtype", C.c_uint32), ("rows", C.c_uint32), ("vocab", C.c_uint32),
                ("ld", C.c_int64), ("logits", C.c_void_p), ("params", C.c_void_p), ("mask", C.c_void_p),
                ("mask_ld", C.c_int64), ("hist", C.c_void_p), ("uniforms", C.c_void_p), ("stream", C.c_void_p),
                ("flags", C.c_uint32), ("reserved", C.c_uint32)]


class Out(C.Structure):
    _fields_ = [("size", C.c_uint32), ("reserved", C.c_uint32), ("tokens", C.c_void_p), ("processed", C.c_void_p),
                ("processed_ld", C.c_int64), ("logprob_ids", C.c_void_p), ("logprobs", C.c_void_p),
                ("logprobs_ld", C.c_int64)]


class MssBatch(C.Structure):
    _fields_ = [("size", C.c_uint32), ("nodes", C.c_uint32), ("vocab", C.c_uint32), ("max_kids", C.c_uint32),
                ("p", C.c_void_p), ("p_ld", C.c_int64), ("q", C.c_void_p), ("q_ld", C.c_int64),
                ("kid_tok", C.c_void_p), ("kid_q", C.c_void_p), ("seed", C.c_void_p), ("idx", C.c_void_p),
                ("out_token", C.c_void_p), ("out_kid", C.c_void_p), ("stream", C.c_void_p)]


class QRows(C.Structure):
    _fields_ = [("size", C.c_uint32), ("kind", C.c_uint32), ("rows", C.c_uint32), ("reserved", C.c_uint32),
                ("q", C.c_void_p), ("ld", C.c_int64), ("temperature", C.c_void_p)]


class Tree(C.Structure):
    _fields_ = [("size", C.c_uint32), ("requests", C.c_uint32), ("anchor", C.c_void_p), ("parent", C.c_void_p),
                ("token", C.c_void_p), ("qrow", C.c_void_p), ("qrows", QRows), ("max_kids", C.c_uint32),
                ("reserved", C.c_uint32)]


class TreeOut(C.Structure):
    _fields_ = [("size", C.c_uint32), ("reserved", C.c_uint32), ("emit_len", C.c_void_p), ("emit_tokens", C.c_void_p),
                ("emit_nodes", C.c_void_p), ("emit_ld", C.c_int64), ("status", C.c_void_p),
                ("node_token", C.c_void_p), ("node_kid", C.c_void_p)]


class PickBatch(C.Structure):
    _fields_ = [("size", C.c_uint32), ("dtype", C.c_uint32), ("rows", C.c_uint32), ("vocab", C.c_uint32),
                ("x", C.c_void_p), ("ld", C.c_int64), ("temperature", C.c_void_p), ("n", C.c_void_p),
                ("seed", C.c_void_p), ("at", C.c_void_p), ("out_tokens", C.c_void_p), ("out_logq", C.c_void_p),
                ("out_ld", C.c_int64), ("stream", C.c_void_p)]


SIGNATURES = dict(
    gse_abi_version=(C.c_uint32, []),
    gse_open=(C.c_int, [P_(OpenParams), P_(C.c_void_p)]),
    gse_sample=(C.c_int, [C.c_void_p, P_(Batch), P_(Out)]),
    gse_dist=(C.c_int, [C.c_void_p, P_(Batch), C.c_void_p, C.c_int64]),
    gse_draw=(C.c_int, [C.c_void_p, C.c_void_p, C.c_int64, C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p,
                        C.c_void_p]),
    gse_qprob=(C.c_int, [C.c_void_p, P_(QRows), C.c_uint32, C.c_void_p, C.c_int64, C.c_void_p]),
    gse_mss=(C.c_int, [C.c_void_p, P_(MssBatch)]),
    gse_sample_noalloc=(C.c_int, [P_(Batch), P_(Out)]),
    gse_verify_tree=(C.c_int, [C.c_void_p, P_(Batch), P_(Tree), P_(TreeOut)]),
    gse_draft_pick=(C.c_int, [C.c_void_p, P_(PickBatch)]),
    gse_pack_mask=(C.c_int, [C.c_void_p, C.c_void_p, C.c_int64, C.c_uint32, C.c_uint32, C.c_void_p, C.c_int64,
                             C.c_void_p]),
    gse_profile=(C.c_int, [C.c_void_p, P_(C.c_float), C.c_uint32, P_(C.c_uint32)]),
    gse_row_paths=(C.c_int, [C.c_void_p, C.c_uint32, C.c_void_p]),
    gse_last_error=(C.c_char_p, [C.c_void_p]),
    gse_close=(None, [C.c_void_p]),
)


def bind(path=PATH):
    """The library at path with its gse.h signatures; refuses a different ABI major or an older minor."""
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built: run __graft_entry__.build() (hipcc --offload-arch=gfx950)")
    L = C.CDLL(path)
    for n, (res, args) in SIGNATURES.items():
        f = getattr(L, n)
        f.restype, f.argtypes = res, args
    v = L.gse_abi_version()
    if v >> 16 != ABI_MAJOR or (v & 0xFFFF) < ABI_MINOR:
        raise RuntimeError(f"{path}: C ABI {v >> 16}.{v & 0xFFFF}, this module needs {ABI_MAJOR}.{ABI_MINOR}+")
    return L


_lock = threading.Lock()
_L = None
# Open handles, least recently used first, keyed by (device, stream). Each holds a device workspace (plan_layout in
# gse_int.h: about 47 MB for 256 rows x 151936 tokens, 278 MB for 1024 x 262144), so the cache is bounded: past
# MAX_HANDLES the least recently used one leaves it and is closed once nothing references it any more.
MAX_HANDLES = 8
_handles = OrderedDict()


def lib():
    global _L
    if _L is None:
        _L = bind()
    return _L


class Handle:
    """One gse handle on one device, for the calls of one stream. A handle is not thread safe (abi/gc.h:16-19): every
    library call goes through call(), which holds the handle's lock while the call is enqueued; the calls of two threads
    on one stream then run one after the other on the device, so they may share the workspace."""

    def __init__(self, device, rows, vocab):
        self.L = lib()
        self.device, self.rows, self.vocab = device, rows, vocab
        self.lock = threading.Lock()
        self.h = None
        h = C.c_void_p()
        p = OpenParams(C.sizeof(OpenParams), device, rows, vocab)
        rc = self.L.gse_open(C.byref(p), C.byref(h))
        if rc != OK:
            raise RuntimeError(f"gse_open failed ({rc}): {(self.L.gse_last_error(None) or b'').decode()}")
        self.h = h

    def ck(self, rc, what):
        if rc < 0:
            why = (self.L.gse_last_error(self.h) or b"").decode()
            raise RuntimeError(f"{what} failed ({rc}): {why}")
        return rc

    def call(self, name, *args):
        """gse_<name>(handle, *args) under the handle's lock; a negative code raises RuntimeError with the library's
        last error (gc_c.py:222-227)."""
        with self.lock:
            if not self.h:
                raise RuntimeError(f"{name}: the handle is closed")
            return self.ck(getattr(self.L, name)(self.h, *args), name)

    def row_paths(self, rows):
        """uint8 [rows]: which path finished each row of the last sample / dist call (PATH_MAIN, PATH_DEEP,
        PATH_EXACT). Waits for the device."""
        out = np.zeros(rows, np.uint8)
        self.call("gse_row_paths", rows, out.ctypes.data)
        return out

    def profile(self):
        """(calls, total milliseconds per kernel: main, deep, exact[, dist]) of the calls made with BATCH_PROFILE
        since the last read; clears the record."""
        ms = (C.c_float * 4)()
        calls = C.c_uint32()
        n = self.call("gse_profile", ms, 4, C.byref(calls))
        return calls.value, [float(ms[i]) for i in range(n)]

    def close(self):
        """Waits for the device (gse_close synchronizes) and frees the workspace."""
        with self.lock:
            if self.h:
                self.L.gse_close(self.h)
                self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # (interpreter shutdown)
            pass


def handle(device, rows, vocab):
    """The handle of (device, current stream) that fits rows x vocab, reopened larger on demand. Calls on two streams
    may overlap on the device, so each stream gets its own workspace; at most MAX_HANDLES stay cached."""
    if not torch.cuda.is_available():
        raise RuntimeError("goethe-engine_amd needs a HIP device (torch.cuda.is_available() is False)")
    key = (device, torch.cuda.current_stream(device).cuda_stream)
    with _lock:
        h = _handles.get(key)
        if h is None or h.rows < rows or h.vocab < vocab:
            # (a handle that is replaced or evicted is closed when its last user lets it go)
            h = Handle(device, max(rows, h.rows if h else 0, 64), max(vocab, h.vocab if h else 0))
            _handles[key] = h
            while len(_handles) > MAX_HANDLES:
                _handles.popitem(last=False)
        _handles.move_to_end(key)
        return h


def ptr(t):
    return C.c_void_p(t.data_ptr()) if t is not None else None


def stream_of(device):
    return C.c_void_p(torch.cuda.current_stream(device).cuda_stream)
