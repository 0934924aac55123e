"""ctypes loader of the oracle's C restatement (oracle/_build/liboracle.so)."""
import ctypes
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_SO = _HERE / '_build' / 'liboracle.so'
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not _SO.exists():
            subprocess.run(['make', '-C', str(_HERE)], check=True, capture_output=True)
        h = ctypes.CDLL(str(_SO))
        p, i64 = ctypes.c_void_p, ctypes.c_int64
        h.oracle_topk.argtypes = [p, i64, i64, i64, ctypes.c_int, ctypes.c_int, p, p]
        h.oracle_topk.restype = ctypes.c_int
        h.oracle_choose_slot.argtypes = [i64, p, p, i64, p, p, i64]
        h.oracle_choose_slot.restype = i64
        h.oracle_plan_layer.argtypes = [i64, i64, p, i64, i64, p, p, i64, p, p, p, i64, p, p]
        h.oracle_plan_layer.restype = i64
        h.oracle_layer_slots.argtypes = [p, i64, i64, i64, p]
        h.oracle_layer_slots.restype = None
        h.oracle_softmax.argtypes = [p, i64, i64, p]
        h.oracle_softmax.restype = None
        h.oracle_weight_sum.argtypes = [p, i64, i64, p]
        h.oracle_weight_sum.restype = None
        h.oracle_expf.argtypes = [ctypes.c_float]
        h.oracle_expf.restype = ctypes.c_float
        _lib = h
    return _lib


def topk(values, k, largest=True, sorted=True):
    """torch CPU topk semantics (TopKImpl.h) on fp32 rows; returns (values, indices)."""
    v = np.ascontiguousarray(values, np.float32)
    rows, n = v.shape
    ov = np.empty((rows, k), np.float32)
    oi = np.empty((rows, k), np.int64)
    if lib().oracle_topk(v.ctypes.data, rows, n, k, int(largest), int(sorted), ov.ctypes.data,
                         oi.ctypes.data) != 0:
        raise ValueError('bad topk arguments')
    return ov, oi


def softmax(x):
    """torch's CPU softmax over the last dim of fp32 rows, restated (softmax.c)."""
    v = np.ascontiguousarray(x, np.float32)
    rows, n = v.shape
    out = np.empty_like(v)
    lib().oracle_softmax(v.ctypes.data, rows, n, out.ctypes.data)
    return out


def weight_sum(w):
    """torch's CPU sum over the last dim of fp32 rows of k <= 32, restated (softmax.c)."""
    v = np.ascontiguousarray(w, np.float32)
    rows, k = v.shape
    out = np.empty(rows, np.float32)
    lib().oracle_weight_sum(v.ctypes.data, rows, k, out.ctypes.data)
    return out
