"""The activation quantizer on the GPU: `quantize_mx` and `quantize`, with the signatures and
outputs of the reference's `opentpu/fp32.py:295-343` (QACT's and QST's arithmetic), computed by
the HIP QACT kernel.

Inputs may be numpy arrays (copied to the device and the results back) or device tensors
(results stay on the device, on the current stream)."""
from __future__ import annotations

import numpy as np

from . import _lib as X


def quantize_mx(x, g: int, row_mode: bool = False, lo: bool = False):
    """Rows of x [rows, n] -> (q int8 [rows, n], S fp32 [rows], d uint8 [rows, n / g]):
    S = amax * f32(1/127), inv = 127 * recip(amax), d the largest offset <= 31 with the group's
    amax * 2^d <= amax (0 in row mode), q = q8(x * (inv * 2^d)) (`opentpu/fp32.py:321`)."""
    if lo:
        raise NotImplementedError("the split's lo part (SPLITQ) is not on this path")
    T = X.torch()
    numpy_in = X.is_numpy(x)
    xd = X.dev(x, np.float32)
    if xd.dim() != 2:
        raise ValueError("quantize_mx: x must be [rows, n]")
    M, K = xd.shape
    q = X.empty((M, K), np.int8)
    S = X.empty((M,), np.float32)
    d = X.empty((M, K // g), np.uint8)
    X.call("otpu_qact", X.ptr(xd), M, K, K, g, int(bool(row_mode)), X.ptr(q), K, X.ptr(S), X.ptr(d),
           K // g, X.stream())
    if numpy_in:
        return X.host(q), X.host(S), X.host(d)
    del T
    return q, S, d


def quantize(x, axis: int = -1):
    """One scale per row over the last axis (`opentpu/fp32.py:295`): (q int8, S fp32)."""
    if axis not in (-1, 1):
        raise ValueError("quantize: the rows' last axis")
    numpy_in = X.is_numpy(x)
    xd = X.dev(x, np.float32)
    M, K = xd.shape
    q = X.empty((M, K), np.int8)
    S = X.empty((M,), np.float32)
    g = 128 if K % 128 == 0 else (32 if K % 32 == 0 else 8)
    d = X.empty((M, K // g), np.uint8)
    X.call("otpu_qact", X.ptr(xd), M, K, K, g, 1, X.ptr(q), K, X.ptr(S), X.ptr(d), K // g, X.stream())
    return (X.host(q), X.host(S)) if numpy_in else (q, S)
