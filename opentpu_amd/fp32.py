"""The activation quantizer on the GPU: `quantize_mx` and `quantize`, with the signatures and
outputs of the reference's `opentpu/fp32.py:295-343` (QACT's and QST's arithmetic), and `qact`,
the QACT instruction's whole work (`opentpu/isasim.py:913-988`: the RSCALE / CSCALE
pre-multiplies, the split's LO / HL parts and ST's DRAM rows), computed by the HIP QACT kernel;
`lda` loads ST's rows back (`opentpu/isasim.py:990-1006`).

Inputs may be numpy arrays (copied to the device and the results back) or device tensors
(results stay on the device, on the current stream)."""
from __future__ import annotations

import numpy as np

from . import _lib as X

GROUPS = (8, 16, 32, 64, 128)


def _rows(x):
    xd = X.dev(x, np.float32)
    if xd.dim() != 2:
        raise ValueError("x must be [rows, n]")
    return xd


def quantize_mx(x, g: int, row_mode: bool = False, lo: bool = False):
    """Rows of x [rows, n] -> (q int8 [rows, n], S fp32 [rows], d uint8 [rows, n / g]):
    S = amax * f32(1/127), inv = 127 * recip(amax), d the largest offset <= 31 with the group's
    amax * 2^d <= amax (0 in row mode), q = q8(x * (inv * 2^d)) (`opentpu/fp32.py:321`).
    lo: the split's lo part instead, q8lo of the same products and the scale S * 2^-8
    (`opentpu/fp32.py:175-185`).  g in 8, 16, 32, 64, 128 and n a multiple of g."""
    return qact(x, g, row_mode, lo=lo)


def qact(x, g: int = 32, row_mode: bool = False, rscale=None, cscale=None, lo: bool = False,
         hl: bool = False, st: bool = False):
    """QACT of the rows of x [rows, n]: x' = (x * rscale[r]) * cscale[c] (each factor optional,
    two FTZ RNE products: RMSNorm's x * r * gamma), quantized as quantize_mx(x', g, row_mode, lo).
    hl: both parts of one read, (q, S, d, q_lo, S_lo).  st: also QACT ST's DRAM rows
    [rows, qrow_bytes] (each row's n bytes, then a block's 8-byte record: S, its 4 offsets; g 32,
    n a multiple of 128), appended to the result."""
    if lo and hl:
        raise ValueError("qact: HL with LO")
    if st and hl:
        raise ValueError("qact: ST with HL")
    if g not in GROUPS:
        raise ValueError(f"qact: groups of {g} (one of {GROUPS})")
    numpy_in = X.is_numpy(x)
    xd = _rows(x)
    M, K = xd.shape
    if K % g:
        raise ValueError(f"qact: {K} columns are not whole groups of {g}")
    rs = X.dev(np.asarray(rscale, np.float32).reshape(-1) if X.is_numpy(rscale) else rscale, np.float32) \
        if rscale is not None else None
    cs = X.dev(np.asarray(cscale, np.float32).reshape(-1) if X.is_numpy(cscale) else cscale, np.float32) \
        if cscale is not None else None
    if rs is not None and rs.numel() != M or cs is not None and cs.numel() != K:
        raise ValueError("qact: rscale [rows], cscale [n]")
    q = X.empty((M, 2 * K if hl else K), np.int8)
    S = X.empty((2 * M if hl else M,), np.float32)
    d = X.empty((M, K // g), np.uint8)
    stb = None
    qrs = 0
    if st:
        qrs = -(-(K + 8 * (K // 128)) // X.QALIGN) * X.QALIGN
        stb = X.empty((M, qrs), np.uint8)
    fl = (X.Q_ROW if row_mode else 0) | (X.Q_LO if lo else 0) | (X.Q_HL if hl else 0)
    X.call("otpu_qact", X.ptr(xd), M, K, K, g, fl, X.ptr(rs), X.ptr(cs), X.ptr(q), q.shape[1], X.ptr(S),
           X.ptr(d), K // g, X.ptr(stb), qrs, X.stream())
    if hl:
        out = (q[:, :K], S[:M], d, q[:, K:], S[M:])
    else:
        out = (q, S, d)
    if st:
        out = out + (stb[:, :K + 8 * (K // 128)],)
    if numpy_in:
        return tuple(np.ascontiguousarray(X.host(t)) for t in out)
    return out


def lda(qrows, KB: int):
    """LDA: QACT ST's rows [rows, >= KB * 136] back into an MM operand (q int8 [rows, KB*128],
    S fp32 [KB, rows] (block k's record scale), d uint8 [rows, 4 KB])."""
    numpy_in = X.is_numpy(qrows)
    b = X.dev(qrows, np.uint8)
    rows = b.shape[0]
    need = KB * 136
    if b.dim() != 2 or b.shape[1] < need:
        raise ValueError(f"lda: rows of {need} bytes")
    qrs = -(-need // X.QALIGN) * X.QALIGN
    if b.shape[1] != qrs or not b.is_contiguous():           # ST's stride: a multiple of QALIGN
        T = X.torch()
        nb = T.zeros((rows, qrs), dtype=T.uint8, device=b.device)
        nb[:, :need] = b[:, :need]
        b = nb
    q = X.empty((rows, KB * 128), np.int8)
    S = X.empty((KB, rows), np.float32)
    d = X.empty((rows, 4 * KB), np.uint8)
    X.call("otpu_lda", X.ptr(b), qrs, rows, KB, X.ptr(q), q.shape[1], X.ptr(S), X.ptr(d), d.shape[1], X.stream())
    return (X.host(q), X.host(S), X.host(d)) if numpy_in else (q, S, d)


def quantize(x, axis: int = -1):
    """One scale per group along `axis` (the whole axis is one group; `opentpu/fp32.py:295-307`),
    any shape: (q int8 of x's shape, S fp32 of x's shape without that axis)."""
    numpy_in = X.is_numpy(x)
    T = X.torch()
    xd = X.dev(np.asarray(x, np.float32) if numpy_in else x, np.float32)
    if xd.dim() == 0:
        raise ValueError("quantize: x needs an axis")
    ax = axis % xd.dim()
    moved = xd.movedim(ax, -1)
    lead = tuple(moved.shape[:-1])
    n = moved.shape[-1]
    rows = moved.reshape(-1, n)
    M = rows.shape[0]
    Kp = -(-n // 8) * 8                                  # zero columns change neither amax nor q
    xp = T.zeros((max(M, 1), Kp), dtype=T.float32, device=xd.device)
    if M:
        xp[:, :n] = rows
    q = X.empty((max(M, 1), Kp), np.int8)
    S = X.empty((max(M, 1),), np.float32)
    X.call("otpu_qact", X.ptr(xp), max(M, 1), Kp, Kp, 8, X.Q_ROW, None, None, X.ptr(q), Kp, X.ptr(S), None, 0,
           None, 0, X.stream())
    qo = q[:M, :n].reshape(lead + (n,)).movedim(-1, ax)
    So = S[:M].reshape(lead)
    return (np.ascontiguousarray(X.host(qo)), X.host(So)) if numpy_in else (qo, So)
