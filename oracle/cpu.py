"""ctypes binding of the C oracle (oracle/cpu_mm.c -> oracle/libotpu_oracle.so).
TEST INFRASTRUCTURE ONLY: the fast checker at full sizes and the CPU baseline timer."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libotpu_oracle.so")
_lib = None
FMT = {"int8": 0, "int4": 1, "fp4": 2, "nvfp4": 3}


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built (make -C oracle)")
        _lib = C.CDLL(LIB_PATH)
        P, L, I = C.c_void_p, C.c_long, C.c_int
        _lib.otpu_cpu_qact.argtypes = [P, I, I, L, I, I, P, L, P, P, L]
        _lib.otpu_cpu_mm.argtypes = [P, L, P, P, L, I, I, P, L, P, L, I, I, I, I, P, P, L, P, P]
        _lib.otpu_cpu_argmax.argtypes = [P, L, P, P]
        _lib.otpu_cpu_threads.argtypes = [I]
        _lib.otpu_cpu_recip.argtypes = [P, L, P]
        _lib.otpu_cpu_recip.restype = None
    return _lib


def recip(x):
    """The C restatement's recip, elementwise (float32 in, float32 out)."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().otpu_cpu_recip(_p(x), x.size, _p(y))
    return y


def _p(a):
    return a.ctypes.data_as(C.c_void_p) if a is not None else None


def threads(n: int = 0) -> int:
    return lib().otpu_cpu_threads(n)


def qact(x, g: int = 32, row_mode: bool = False):
    x = np.ascontiguousarray(x, np.float32)
    M, K = x.shape
    q = np.empty((M, K), np.int8)
    S = np.empty(M, np.float32)
    d = np.empty((M, K // g), np.uint8)
    rc = lib().otpu_cpu_qact(_p(x), M, K, K, g, int(row_mode), _p(q), K, _p(S), _p(d), K // g)
    if rc:
        raise ValueError(f"otpu_cpu_qact: {rc}")
    return q, S, d


def mm(q, Sa, da, rows, srows, fmt: str, K: int, *, flags: int = 0, k0: int = 0, old=None,
       alpha=None, want_acc: bool = False):
    q = np.ascontiguousarray(q, np.int8)
    Sa = np.ascontiguousarray(Sa, np.float32)
    da = np.ascontiguousarray(da, np.uint8)
    rows = np.ascontiguousarray(rows, np.uint8)
    srows = np.ascontiguousarray(srows, np.uint8)
    M, N = q.shape[0], rows.shape[0]
    out = np.zeros((M, N), np.float32) if old is None else np.array(old, np.float32, copy=True)
    rmax = np.empty(M, np.float32)
    acc = np.empty((M, N), np.int64) if want_acc else None
    al = None if alpha is None else np.ascontiguousarray(alpha, np.float32)
    rc = lib().otpu_cpu_mm(_p(q), q.shape[1], _p(Sa), _p(da), da.shape[1], M, K, _p(rows),
                           rows.shape[1], _p(srows), srows.shape[1], N, FMT[fmt], flags, k0,
                           _p(al), _p(out), N, _p(rmax), _p(acc))
    if rc:
        raise ValueError(f"otpu_cpu_mm: {rc}")
    res = [out]
    if flags & 0x4:
        res.append(rmax)
    if want_acc:
        res.append(acc)
    return res[0] if len(res) == 1 else tuple(res)


def argmax(x):
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    best = np.zeros(1, np.uint64)
    tok = np.zeros(1, np.int32)
    lib().otpu_cpu_argmax(_p(x), x.shape[0], _p(best), _p(tok))
    return int(tok[0]), int(best[0])
