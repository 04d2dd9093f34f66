"""Oracle: MM (exact integer sums, one fp32 epilogue), ARGMAX and greedy (numpy).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

MM restated from `opentpu/isasim.py:749-910` (natural row layout, rows of one: WG = 1, no PAIR
or KT; SPL below) and `docs/isa.md:226-305`:

    for each output (j, n):  acc = sum over blocks k, groups g of B * c
        c  = sum_{i in g} q[j, i] * w[n, i]            exact; |c| < 2^19 (int8), 2^16 (4-bit)
        sh = W - dw[n, k0+k, g] - da[j, group]          W = 16 int8, 11 int4/fp4, 13 nvfp4
        B  = sh >= 0 ? m[n, k0+k, g] << sh : 0          the group drops where sh < 0
    y = mul(mul(i2f(acc), Sw[n]), mul(Sa[j], 2^-W))     three FTZ/RNE products
    ACC: y = add(old, y);  ASCALE: y = add(mul(old, alpha[j]), y);  RMAX: row max of the y.

SPL (split terms, `opentpu/isasim.py:757-770`, `:849-852`, `:872-873`; `docs/isa.md:414-441`):
one MM over a split operand's terms, one block (D = 128) of int8 RSC weights a part:

    KB 3: acc = sum_g [ c(hi, w_hi) << (16 - da)  +  c(lo, w_hi) << (8 - da)  +  c(hi, w_lo) << (8 - da) ]
    KB 2: acc = sum_g [ c(hi, w_hi) << (16 - da)  +  c(hi, w_lo) << (8 - da) ]
    (a term whose shift is negative adds nothing); y = (i2f(acc) * Sw) * (Sa_hi * 2^-16)

ARGMAX / greedy restated from `opentpu/isasim.py:1141-1152`, `opentpu/fp32.py:110-121`,
`opentpu/llm/generate.py:251-286`: the first index whose total-order key is largest.

Pinning (tests/test_oracle_mm.py):
SPL: a scalar Python-int model of the docs/isa.md pseudo-code with the advance table (KB 3:
ACT hi, lo, hi against rows hi, hi, lo; KB 2: hi, hi against hi, lo), and the closed form at
zero offsets acc = 2^16 hi.w_hi + 2^8 (lo.w_hi + hi.w_lo).
MM: a scalar Python-int model written from docs/isa.md (the
shape of the reference's `tests/test_mx.py:131-151` ref_mm) on the reference's CASES and
seeds; the reference's integer model with asserted drops (`tests/test_isa.py:85-118`); closed
forms (UNIT MM = plain integer dot; RSC + ROW activations: acc = 2^W * sum q w); the ARGMAX
KATs of `tests/test_autodecode.py:26-40`.
"""
from __future__ import annotations

import numpy as np

from . import fp32 as F
from .formats import D, NSUB, NVG, WINDOW, elements, unpack_scales

UNIT, ACC, RMAX, ASCALE, RSC = 0x1, 0x2, 0x4, 0x8, 0x80        # MM flag bits (isa.py:21,30)


def group_sums(q, w, gsize: int) -> np.ndarray:
    """c[j, n, t] = sum over group t (gsize elements) of q[j] * w[n], exact (int64).
    Each partial is < 2^53 in magnitude, so the float64 product is exact."""
    q = np.asarray(q, np.int64)
    w = np.asarray(w, np.int64)
    M, K = q.shape
    N = w.shape[0]
    T = K // gsize
    qf = q.reshape(M, T, gsize).transpose(1, 0, 2).astype(np.float64)   # [T, M, g]
    wf = w.reshape(N, T, gsize).transpose(1, 2, 0).astype(np.float64)   # [T, g, N]
    return np.matmul(qf, wf).transpose(1, 2, 0).astype(np.int64)        # [M, N, T]


def mm_acc(q, da, rows, srows, fmt: str, K: int, *, flags: int = 0, k0: int = 0):
    """The exact accumulators acc int64 [M, N] and (Sw [N]) of MM.

    q int8 [M, K]; da uint8 [M, K/32] (the activations' group offsets); rows / srows the
    element and scale rows (formats.py); k0 the MM's first block within the scale rows."""
    q = np.asarray(q)
    M = q.shape[0]
    KB = K // D
    w = elements(rows, fmt, K)
    Sw, dw, m = unpack_scales(srows, fmt, KB, k0, rsc=bool(flags & RSC), unit=bool(flags & UNIT))
    G = dw.shape[2]
    c = group_sums(q[:, :K], w, D // G).reshape(M, -1, KB, G)           # [M, N, KB, G]
    da = np.asarray(da, np.int64)[:, :KB * NSUB].reshape(M, KB, NSUB)
    da = np.repeat(da, G // NSUB, axis=2)                                # [M, KB, G]
    sh = WINDOW[fmt] - dw[None, :, :, :] - da[:, None, :, :]
    B = np.where(sh >= 0, m[None] << np.maximum(sh, 0), 0)
    return (B * c).sum(axis=(2, 3)), Sw


def epilogue(acc, Sw, Sa, fmt: str) -> np.ndarray:
    """y = (i2f(acc) * Sw[n]) * (Sa[j] * 2^-W), each product FTZ/RNE."""
    scale_a = F.mul(np.asarray(Sa, np.float32), F.pow2(-WINDOW[fmt]))
    return F.mul(F.mul(F.i2f(acc), np.asarray(Sw, np.float32)[None, :]), scale_a[:, None])


def mm(q, Sa, da, rows, srows, fmt: str, K: int, *, flags: int = 0, k0: int = 0,
       old=None, alpha=None):
    """MM's fp32 outputs [M, N] (and the row maxima [M] with RMAX)."""
    if flags & ASCALE and not (flags & UNIT and flags & ACC):
        raise ValueError("ASCALE needs UNIT and ACC")
    acc, Sw = mm_acc(q, da, rows, srows, fmt, K, flags=flags, k0=k0)
    y = epilogue(acc, Sw, Sa, fmt)
    if flags & ASCALE:
        y = F.add(F.mul(np.asarray(old, np.float32), np.asarray(alpha, np.float32)[:, None]), y)
    elif flags & ACC:
        y = F.add(np.asarray(old, np.float32), y)
    if flags & RMAX:
        return y, rowmax(y)
    return y


def mm_spl(q, Sa, da, w_hi, w_lo, Sw, nterms: int, *, old=None):
    """MM SPL's outputs [M, N]: q int8 [M, 128] (KB 2) or [M, 256] (KB 3: hi, then lo, as QACT HL
    writes them), Sa [M] (hi's), da uint8 [M, 4] (the hi part's offsets; lo shares them), w_hi /
    w_lo int8 [N, 128] (the weights' hi and lo rows), Sw [N] (hi's).  old: ACC."""
    if nterms not in (2, 3):
        raise ValueError("SPL takes 2 or 3 terms")
    q = np.asarray(q, np.int8)
    M = q.shape[0]
    hi = q[:, :D]
    lo = q[:, D:2 * D] if nterms == 3 else None
    wh = np.asarray(w_hi, np.uint8)[:, :D].view(np.int8)
    wl = np.asarray(w_lo, np.uint8)[:, :D].view(np.int8)
    terms = [(hi, wh, 0), (lo, wh, 8), (hi, wl, 8)] if nterms == 3 else [(hi, wh, 0), (hi, wl, 8)]
    da = np.asarray(da, np.int64)[:, :NSUB]                           # [M, 4]
    acc = np.zeros((M, wh.shape[0]), np.int64)
    for a, w, e in terms:
        c = group_sums(a, w, D // NSUB)                               # [M, N, 4]
        sh = WINDOW["int8"] - (da[:, None, :] + e)
        acc += np.where(sh >= 0, c << np.maximum(sh, 0), 0).sum(axis=2)
    y = epilogue(acc, np.asarray(Sw, np.float32), Sa, "int8")
    return F.add(np.asarray(old, np.float32), y) if old is not None else y


def rowmax(y) -> np.ndarray:
    """Row maxima in the total order (any evaluation order gives these bits)."""
    y = F.ftz(np.asarray(y, np.float32))
    return y[np.arange(y.shape[0]), np.argmax(F.key(y), axis=1)]


def argmax(y, base: int = 0):
    """VOP ARGMAX of each row: (max value, first index of it + base)."""
    y = F.ftz(np.atleast_2d(np.asarray(y, np.float32)))
    idx = np.argmax(F.key(y), axis=1)                  # numpy: the first maximal key
    return y[np.arange(y.shape[0]), idx], idx + base


def greedy(logits) -> int:
    """The token the LM head's greedy sampler picks: the smallest index of the largest key."""
    return int(argmax(np.asarray(logits).reshape(1, -1))[1][0])


def best_word(logits) -> int:
    """The 64-bit word (key << 32) | ~index whose unsigned max picks the greedy token."""
    k = F.key(np.asarray(logits, np.float32).reshape(-1)).astype(np.uint64)
    idx = np.arange(k.shape[0], dtype=np.uint64)
    return int(((k << np.uint64(32)) | (~idx & np.uint64(0xFFFFFFFF))).max())
