"""ctypes loader for the oracle's C restatement (oracle/c/oracle.c), built into oracle/_build/liboracle.so."""
import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
PATH = os.path.join(_HERE, "_build", "liboracle.so")
_L = None


def lib():
    global _L
    if _L is None:
        if not os.path.exists(PATH):
            raise RuntimeError(f"oracle C library not built: {PATH} (run __graft_entry__.build())")
        L = C.CDLL(PATH)
        L.ora_mix.restype, L.ora_mix.argtypes = C.c_uint64, [C.c_uint64, C.c_uint64]
        L.ora_uniform.restype, L.ora_uniform.argtypes = C.c_double, [C.c_uint64, C.c_uint64]
        L.ora_greedy.restype = None
        L.ora_greedy.argtypes = [C.c_void_p, C.c_int64, C.c_int32, C.c_int32, C.c_void_p, C.c_int32, C.c_void_p]
        L.ora_unpack.restype, L.ora_unpack.argtypes = None, [C.c_void_p, C.c_int32, C.c_void_p]
        _L = L
    return _L


def mix(seed, i):
    return int(lib().ora_mix(seed & ((1 << 64) - 1), i & ((1 << 64) - 1)))


def uniform(seed, idx):
    return float(lib().ora_uniform(seed & ((1 << 64) - 1), idx & ((1 << 64) - 1)))


def greedy(x, words=None):
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, v = x.shape
    out = np.empty(rows, dtype=np.int32)
    w = None if words is None else np.ascontiguousarray(words, dtype=np.int32)
    lib().ora_greedy(x.ctypes.data, v, rows, v, None if w is None else w.ctypes.data,
                     0 if w is None else w.shape[1], out.ctypes.data)
    return out


def unpack(words, v):
    w = np.ascontiguousarray(words, dtype=np.int32)
    out = np.empty(v, dtype=np.uint8)
    lib().ora_unpack(w.ctypes.data, v, out.ctypes.data)
    return out.astype(bool)
