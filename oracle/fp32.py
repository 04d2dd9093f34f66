"""Oracle: the machine's fp32 arithmetic and its activation / weight-row quantizer (numpy).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Semantics restated from the reference:
  * IEEE binary32 round-to-nearest-even with flush-to-zero on operands and results, canonical
    NaN 0x7FC00000 from every arithmetic op: `opentpu/fp32.py:45-101`, `docs/isa.md:88-112`.
  * total-order key for max / argmax: `opentpu/fp32.py:104-121`.
  * `i2f` (int64 -> fp32, RNE): `opentpu/fp32.py:162-164`.
  * `q8` (rint half-even, saturate +-127, NaN -> 0): `opentpu/fp32.py:167-172`.
  * `recip` (magic seed, two Newton steps, correction step, exponent fix-up):
    `opentpu/fp32.py:242-261`, `docs/isa.md:124-135`.
  * `quantize` (one scale per row) and `quantize_mx` (row scale + power-of-two group offsets):
    `opentpu/fp32.py:295-343`, `docs/isa.md:163-178`.
  * `q8lo` and `quantize_mx(lo=True)`, the split quantizer's lo part (QACT / QST flag LO):
    `opentpu/fp32.py:175-185`, `:321-343`, `docs/isa.md:183-195`.
  * `qact` (QACT's RSCALE / CSCALE pre-multiplies, then the quantizer, its LO / HL parts):
    `opentpu/isasim.py:913-959`, `docs/isa.md:444-460`.
  * `qrows_store` / `lda` (QACT ST's DRAM rows of KB*D bytes and 8-byte records, and LDA back):
    `opentpu/isasim.py:962-1006`, `opentpu/isa.py:39-40`, `:577-580`, `docs/isa.md:468-486`.

How each function is pinned (tests/test_oracle_fp32.py):
  mul/add/sub   host IEEE binary32 (numpy float32) + the flush rule, the reference's zero-sign
                and subnormal-grid KATs (tests/test_fp.py:191-218 of the reference).
  key           KATs of the reference's ARGMAX tests (-0 < +0, denormal -> +0, NaN order).
  i2f           exact integers, ties at every power of two against Python's correctly rounded
                float conversion (fractions).
  recip         exact at every power of two, <= 1.2 ulp over all of [1, 2) and every exponent
                (the reference's bounds, tests/test_fp.py:221,324).
  q8            KATs (half-even, saturation, NaN).
  quantize_mx   a scalar model written from docs/isa.md (different formulation: float64 ratio
                search for d), driven like the reference's tests/test_mx.py:52-69.
  q8lo          a scalar model with exact rationals (round(256 (p - q8(p))) half to even, as
                docs/isa.md words it), brute force over every 2^-9 step of [-130, 130] and the
                half-ulp neighbours of each step, and the reconstruction bound the reference
                states (x ~ (q + lo / 256) within 2^-9; 2^-8 where lo saturates).
  qact          a per-element scalar model of the pre-multiplies in the documented order
                (x * r) * c, on inputs where (x * r) * c and x * (r * c) round differently.
  qrows_store   the record layout field by field (KB*D bytes, then per block: S little-endian
  / lda         and four offset bytes at KB*D + 8k), and lda(qrows_store(...)) = the operand.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32
U32 = np.uint32
TINY = F32(2.0 ** -126)             # smallest normal
QNAN = 0x7FC00000                   # the canonical NaN every arithmetic op returns
INV127 = F32(1.0 / 127.0)           # 0x3C010204
RECIP_MAGIC = 0x7EF311C3
MX_DMAX = 31                        # largest power-of-two group offset


def as_f32(x) -> np.ndarray:
    return np.asarray(x, dtype=F32)


def bits(x) -> np.ndarray:
    return as_f32(x).view(U32)


def from_bits(u) -> np.ndarray:
    return np.asarray(u, dtype=U32).view(F32)


def ftz(x) -> np.ndarray:
    """Denormals become zeros of the same sign; everything else (NaN too) keeps its bits."""
    u = bits(x).copy()
    den = ((u & U32(0x7F800000)) == 0) & ((u & U32(0x7FFFFF)) != 0)
    u[den] &= U32(0x80000000)
    return u.view(F32)


def _finish(r) -> np.ndarray:
    """An arithmetic result: flush a denormal result, replace any NaN by the canonical one."""
    r = ftz(r)
    u = r.view(U32).copy()
    u[np.isnan(r)] = U32(QNAN)
    return u.view(F32)


def _binary(op, a, b):
    a, b = np.broadcast_arrays(ftz(a), ftz(b))
    with np.errstate(all="ignore"):
        return _finish(op(a, b).astype(F32))


def mul(a, b):
    return _binary(np.multiply, a, b)


def add(a, b):
    return _binary(np.add, a, b)


def sub(a, b):
    return _binary(np.subtract, a, b)


def key(x) -> np.ndarray:
    """Total-order key (uint32) of flushed fp32 bits: -NaN < -inf < ... < -0 < +0 < ... < inf
    < NaN; the unsigned order of keys is that order."""
    u = bits(ftz(x)).astype(U32)
    neg = (u >> U32(31)).astype(bool)
    return np.where(neg, ~u, u | U32(0x80000000)).astype(U32)


def i2f(i) -> np.ndarray:
    """Signed int64 -> fp32, round to nearest even (the conversion is correctly rounded)."""
    return np.asarray(i, dtype=np.int64).astype(F32)


def q8(x) -> np.ndarray:
    x = ftz(x)
    x = np.where(np.isnan(x), F32(0), x)
    r = np.rint(x.astype(np.float64))               # half to even
    return np.clip(r, -127, 127).astype(np.int8)


def q8lo(x) -> np.ndarray:
    """The split's lo byte: sat127(rint(256 x) - 256 q8(x)), half to even, NaN -> 0
    (`opentpu/fp32.py:175-185`).  rint(256 x) is taken in float64 (exact for any fp32 x) and
    clipped to +-2^16 before the subtraction, where the result saturates either way."""
    x = ftz(x)
    nan = np.isnan(x)
    t = np.rint(np.where(nan, F32(0), x).astype(np.float64) * 256.0)
    t = np.clip(t, -65536.0, 65536.0)
    r = t - 256.0 * q8(x).astype(np.float64)
    return np.where(nan, 0, np.clip(r, -127, 127)).astype(np.int8)


def pow2(d) -> np.ndarray:
    """f32(2^d) for integer d in [-126, 127], exact, built from the exponent field."""
    d = np.asarray(d, dtype=np.int64)
    return from_bits(((d + 127) << 23).astype(U32))


def recip(x) -> np.ndarray:
    """1/x as the machine computes it (docs/isa.md "recip")."""
    x = ftz(x)
    xb = bits(x)
    mag = xb & U32(0x7FFFFFFF)
    sign = xb & U32(0x80000000)
    zero = mag == 0
    huge = mag >= U32(0x7E800000)                    # |x| >= 2^126, inf and NaN bits
    a = from_bits(U32(0x3F800000) | (mag & U32(0x7FFFFF)))           # significand in [1, 2)
    y = from_bits((U32(RECIP_MAGIC) - bits(a)).astype(U32))
    two, one = F32(2.0), F32(1.0)
    y = mul(y, sub(two, mul(a, y)))
    y = mul(y, sub(two, mul(a, y)))
    y = add(mul(y, sub(one, mul(a, y))), y)
    shift = 127 - (mag >> U32(23)).astype(np.int64)                  # exponent fix-up
    yb = bits(y).astype(np.int64) + np.where(zero | huge, 0, shift) * (1 << 23)
    yb = np.where(huge, 0, yb).astype(U32) | sign
    return np.where(zero, U32(0), yb).astype(U32).view(F32)


def abs_bits(x) -> np.ndarray:
    """|ftz(x)| as uint32 bits (a NaN's magnitude is above inf's)."""
    return bits(ftz(x)) & U32(0x7FFFFFFF)


def mx_offset(a_bits, amax_bits) -> np.ndarray:
    """Largest d <= 31 with a * 2^d <= amax, from the exponent fields and fraction bits
    (a <= amax, both non-negative bit patterns); 0 where a == 0."""
    a = np.asarray(a_bits, np.int64)
    m = np.asarray(amax_bits, np.int64)
    d = (m >> 23) - (a >> 23) - ((a & 0x7FFFFF) > (m & 0x7FFFFF)).astype(np.int64)
    return np.where(a == 0, 0, np.clip(d, 0, MX_DMAX)).astype(np.uint8)


def quantize_mx(x, g: int, row_mode: bool = False, lo: bool = False):
    """Rows of x [rows, n] -> (q int8 [rows, n], S fp32 [rows], d uint8 [rows, n/g]).

    S = amax * f32(1/127); inv = 127 * recip(amax) (both 0 for an all-zero row); group g's
    offset d_g = mx_offset(group amax, amax) (0 in row mode); q = q8(x * (inv * 2^d_g)).
    lo: the split's lo part instead, q8lo of the same products, with the scale S * 2^-8."""
    x = ftz(as_f32(x))
    rows, n = x.shape
    if n % g:
        raise ValueError(f"{n} columns are not whole groups of {g}")
    ab = abs_bits(x)
    amax_b = ab.max(axis=1)
    amax = from_bits(amax_b)
    zero = amax_b == 0
    S = np.where(zero, F32(0), mul(amax, INV127)).astype(F32)
    inv = np.where(zero, F32(0), mul(F32(127), recip(amax))).astype(F32)
    if row_mode:
        d = np.zeros((rows, n // g), np.uint8)
    else:
        gmax = ab.reshape(rows, n // g, g).max(axis=2)
        d = mx_offset(gmax, amax_b[:, None])
    scale = mul(inv[:, None], pow2(d))                                # [rows, n/g]
    p = mul(x.reshape(rows, n // g, g), scale[:, :, None])
    if lo:
        return q8lo(p).reshape(rows, n), mul(S, pow2(-8)), d
    return q8(p).reshape(rows, n), S, d


def qact(x, g: int = 32, row_mode: bool = False, rscale=None, cscale=None, lo: bool = False,
         hl: bool = False):
    """QACT of the rows of x [rows, n] (`opentpu/isasim.py:913-959`): RSCALE multiplies row r by
    rscale[r], then CSCALE column c by cscale[c] (x' = (x * r) * c, two rounded products), and
    the result is quantized as quantize_mx(x', g, row_mode, lo).  hl: both halves of one read,
    (q_hi, S_hi, d, q_lo, S_lo) (QACT HL)."""
    x = as_f32(x)
    if rscale is not None:
        x = mul(x, as_f32(rscale).reshape(-1, 1))
    if cscale is not None:
        x = mul(x, as_f32(cscale).reshape(1, -1))
    if hl:
        q, S, d = quantize_mx(x, g, row_mode)
        ql, Sl, _ = quantize_mx(x, g, row_mode, lo=True)
        return q, S, d, ql, Sl
    return quantize_mx(x, g, row_mode, lo)


QREC = 8           # a block's record in QACT ST's rows: fp32 S, then its four group offsets


def qrow_bytes(KB: int) -> int:
    """Bytes of one QACT ST row of KB blocks (`opentpu/isa.py:577-580`)."""
    return KB * 128 + KB * QREC


def qrows_store(q, S, d) -> np.ndarray:
    """QACT ST's DRAM rows [rows, qrow_bytes(KB)] of a QACT operand (q int8 [rows, KB*128],
    S fp32 [rows] (every block's record holds the row's S), d uint8 [rows, 4 KB]): the KB*128
    bytes, then block k's record at KB*128 + 8k: S (4 bytes, little-endian), d[4k .. 4k+3]."""
    q = np.asarray(q, np.int8)
    rows, K = q.shape
    KB = K // 128
    out = np.zeros((rows, qrow_bytes(KB)), np.uint8)
    out[:, :K] = q.view(np.uint8)
    sb = as_f32(S).reshape(rows, 1).view(np.uint8)                    # [rows, 4]
    d = np.asarray(d, np.uint8).reshape(rows, KB, 4)
    for k in range(KB):
        at = K + QREC * k
        out[:, at:at + 4] = sb
        out[:, at + 4:at + 8] = d[:, k]
    return out


def lda(rows_bytes, KB: int):
    """LDA: QACT ST's rows back into an operand: (q int8 [rows, KB*128], S fp32 [KB, rows]
    (block k's record scale of each row), d uint8 [rows, 4 KB]) (`opentpu/isasim.py:990-1006`)."""
    b = np.asarray(rows_bytes, np.uint8)
    rows = b.shape[0]
    K = KB * 128
    q = b[:, :K].copy().view(np.int8)
    rec = np.ascontiguousarray(b[:, K:K + QREC * KB]).reshape(rows, KB, QREC)
    S = np.ascontiguousarray(rec[:, :, :4]).view(np.float32).reshape(rows, KB).T.copy()
    d = rec[:, :, 4:].reshape(rows, 4 * KB).copy()
    return q, S, d


def quantize_rows(x):
    """One scale per row (QST ROW / `fp32.quantize(x, axis=1)` / RSC weights): (q, S)."""
    q, S, _ = quantize_mx(x, as_f32(x).shape[1], row_mode=True)
    return q, S
