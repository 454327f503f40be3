"""ctypes binding of oracle/_build/liboracle.so (the C restatement) -- TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, as the checker.
Build with `make -C oracle` (done by __graft_entry__.build()).
"""

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(f"{LIB_PATH} is not built (make -C oracle)")
        L = ctypes.CDLL(LIB_PATH)
        p, i64 = ctypes.c_void_p, ctypes.c_int64
        L.oracle_quant_rows.argtypes = [p, i64, i64, p, p]
        L.oracle_gemm_i32.argtypes = [p, p, p, i64, i64, i64]
        L.oracle_dequant.argtypes = [p, p, p, p, p, i64, i64]
        L.oracle_conv3x3_acc.argtypes = [p, p, p, i64, i64, i64, i64, i64]
        L.oracle_requant.argtypes = [p, i64, ctypes.c_int, ctypes.c_int, p]
        for f in (L.oracle_quant_rows, L.oracle_gemm_i32, L.oracle_dequant, L.oracle_conv3x3_acc,
                  L.oracle_requant):
            f.restype = None
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def quant_rows(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    r, k = x.shape
    q = np.empty((r, k), np.int8)
    s = np.empty(r, np.float32)
    lib().oracle_quant_rows(_p(x), r, k, _p(q), _p(s))
    return q, s


def gemm_i32(a, w):
    a = np.ascontiguousarray(a, dtype=np.int8)
    w = np.ascontiguousarray(w, dtype=np.int8)
    m, k = a.shape
    n = w.shape[0]
    c = np.empty((m, n), np.int32)
    lib().oracle_gemm_i32(_p(a), _p(w), _p(c), m, n, k)
    return c


def dequant(acc, sx, sw, bias=None):
    acc = np.ascontiguousarray(acc, dtype=np.int32)
    sx = np.ascontiguousarray(sx, dtype=np.float32)
    sw = np.ascontiguousarray(sw, dtype=np.float32)
    m, n = acc.shape
    y = np.empty((m, n), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    lib().oracle_dequant(_p(acc), _p(sx), _p(sw), None if b is None else _p(b), _p(y), m, n)
    return y


def conv3x3_acc(xq, wq):
    xq = np.ascontiguousarray(xq, dtype=np.int8)
    wq = np.ascontiguousarray(wq, dtype=np.int8)
    n, ci, h, w = xq.shape
    co = wq.shape[0]
    acc = np.empty((n, co, h, w), np.int32)
    lib().oracle_conv3x3_acc(_p(xq), _p(wq), _p(acc), n, ci, h, w, co)
    return acc


def requant(acc, shift, relu):
    acc = np.ascontiguousarray(acc, dtype=np.int32)
    out = np.empty(acc.shape, np.uint8 if relu else np.int8)
    lib().oracle_requant(_p(acc), acc.size, int(shift), int(bool(relu)), _p(out))
    return out
