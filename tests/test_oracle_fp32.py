"""The oracle's fp32 arithmetic and quantizer, pinned by host IEEE arithmetic, closed forms,
brute force and the known-answer cases of the reference's own tests (restated, not imported):
`tests/test_fp.py:191-246,324-345` and `tests/test_mx.py:34-69` of FeSens/openTPU."""
from fractions import Fraction

import numpy as np
import pytest

from oracle import fp32 as F


def _b(x):
    return int(np.asarray(x, np.float32).view(np.uint32))


def test_zero_signs_and_identity():
    pz, nz = np.float32(0.0), np.float32(-0.0)
    assert _b(F.add(nz, nz)) == 0x80000000 and _b(F.sub(nz, pz)) == 0x80000000
    assert _b(F.add(pz, nz)) == 0 and _b(F.sub(nz, nz)) == 0 and _b(F.add(nz, pz)) == 0
    x = F.from_bits(np.arange(1, 255, dtype=np.uint32) << 23 | np.uint32(0x2AAAAA)).copy()
    for v in (x, -x):
        assert np.all(F.bits(F.sub(v, v)) == 0) and np.all(F.bits(F.add(v, -v)) == 0)
        assert np.array_equal(F.bits(F.add(v, np.float32(-0.0))), F.bits(v))


def test_mul_rounds_to_the_subnormal_grid_then_flushes():
    # 0.5 * (2^-126 - 2^-149) is a tie on the subnormal grid that rounds up to 2^-126: kept
    assert _b(F.mul(np.float32(0.5), F.from_bits(np.uint32(0x00FFFFFF)))) == 0x00800000
    assert _b(F.mul(np.float32(-0.5), F.from_bits(np.uint32(0x00FFFFFF)))) == 0x80800000
    assert _b(F.mul(np.float32(0.5), F.from_bits(np.uint32(0x00FFFFFE)))) == 0
    # denormal operands are signed zeros; NaN results are canonical
    assert _b(F.mul(F.from_bits(np.uint32(1)), np.float32(3.0))) == 0
    assert _b(F.mul(F.from_bits(np.uint32(0x80000001)), np.float32(3.0))) == 0x80000000
    assert _b(F.mul(np.float32(np.inf), np.float32(0.0))) == 0x7FC00000
    assert _b(F.add(F.from_bits(np.uint32(0xFFC00001)), np.float32(1))) == 0x7FC00000


def test_mul_matches_exact_rounding_on_random_operands():
    """Every product against exact rational rounding to binary32 (RNE) plus the flush."""
    rng = np.random.default_rng(11)
    e = rng.integers(1, 255, 4000).astype(np.uint32)
    a = F.from_bits((rng.integers(0, 2, 4000).astype(np.uint32) << 31) | (e << 23)
                    | rng.integers(0, 1 << 23, 4000).astype(np.uint32))
    b = F.from_bits(rng.integers(0x30000000, 0x50000000, 4000).astype(np.uint32))
    got = F.mul(a, b)
    for x, y, r in zip(a[:600], b[:600], got[:600]):
        exact = Fraction(float(x)) * Fraction(float(y))
        assert _b(r) == _rne32_ftz(exact), (x, y)


def _rne32_ftz(v: Fraction) -> int:
    """Exact binary32 RNE of a rational (subnormal grid), then the flush; bits."""
    if v == 0:
        return 0
    s = 0x80000000 if v < 0 else 0
    v = abs(v)
    e = v.numerator.bit_length() - v.denominator.bit_length()
    if Fraction(2) ** e > v:
        e -= 1
    e = max(e, -126)
    ulp = Fraction(2) ** (e - 23)
    q, r = divmod(v, ulp)
    q = int(q)
    if r > ulp / 2 or (r == ulp / 2 and q & 1):
        q += 1
    val = Fraction(q) * ulp
    if val >= Fraction(2) ** 128:
        return s | 0x7F800000
    if val < Fraction(2) ** -126:
        return s
    f = np.float32(float(val))
    return s | int(f.view(np.uint32))


def _i2f_exact(i: int) -> int:
    return _b(np.float32(float(i))) if abs(i) < 2 ** 24 else _rne32_ftz(Fraction(i))


def test_i2f_is_round_to_nearest_even_at_ties():
    cases = []
    for p in range(24, 48):
        base = 1 << p
        h = 1 << (p - 24)                  # half an ulp at this binade
        cases += [base + h, base + 3 * h, base + h - 1, base + h + 1, base - 1, (1 << 47) - 1]
    cases += [-c for c in cases] + [0, 1, -1, 2 ** 24 - 1, 2 ** 24 + 1]
    got = F.i2f(np.array(cases, np.int64))
    for c, g in zip(cases, got):
        assert _b(g) == _i2f_exact(c), c


def test_recip_exact_at_powers_of_two_and_special_cases():
    p = np.exp2(np.arange(-125, 126)).astype(np.float32)
    for s in (1, -1):
        assert np.array_equal(F.recip(s * p), (s / p.astype(np.float64)).astype(np.float32))
    assert _b(F.recip(np.float32(0))) == 0 and _b(F.recip(np.float32(-0.0))) == 0
    assert _b(F.recip(np.float32(2.0 ** 126))) == 0
    assert _b(F.recip(np.float32(-2.0 ** 127))) == 0x80000000
    assert _b(F.recip(np.float32(-np.inf))) == 0x80000000
    assert _b(F.recip(F.from_bits(np.uint32(5)))) == 0          # denormal: a zero


def _ulps(y, ref):
    e = np.floor(np.log2(np.abs(ref)))
    return np.abs(y.astype(np.float64) - ref) / np.exp2(np.maximum(e, -126) - 23)


def test_recip_error_bound_every_significand_and_exponent():
    x = F.from_bits(np.uint32(127 << 23) | np.arange(1 << 23, dtype=np.uint32)).copy()
    for v in (x, -x):
        assert _ulps(F.recip(v), 1 / v.astype(np.float64)).max() < 1.2
    rng = np.random.default_rng(7)
    e = np.repeat(np.arange(1, 253, dtype=np.uint32), 512)
    v = F.from_bits((rng.integers(0, 2, len(e)).astype(np.uint32) << np.uint32(31))
                    | (e << np.uint32(23)) | rng.integers(0, 1 << 23, len(e)).astype(np.uint32))
    ref = 1 / v.astype(np.float64)
    ok = np.abs(ref) >= 2.0 ** -126
    assert _ulps(F.recip(v)[ok], ref[ok]).max() < 1.2


def test_q8_rounding_saturation_nan():
    x = np.float32([0.5, 1.5, 2.5, -0.5, -1.5, 126.5, 127.49, 200.0, -1e30, np.inf])
    assert F.q8(x).tolist() == [0, 2, 2, 0, -2, 126, 127, 127, -127, 127]
    assert F.q8(F.from_bits(np.uint32([0x7FC00000, 0xFFC00000]))).tolist() == [0, 0]
    # a tiny amax: inv = 127 * recip(amax) is inf, zeros (0 * inf) quantize to 0, S flushes
    x = np.zeros((1, 32), np.float32)
    x[0, 5] = F.from_bits(np.uint32(0x01000000))
    q, S = F.quantize_rows(x)
    assert q[0].tolist() == [0] * 5 + [127] + [0] * 26 and S[0] == 0


def _offset_brute(a: float, amax: float) -> int:
    if a == 0:
        return 0
    d = 0
    while d < 31 and a * 2.0 ** (d + 1) <= amax:
        d += 1
    return d


def test_mx_offset_against_brute_force():
    rng = np.random.default_rng(3)
    amax = np.float32(rng.uniform(0.5, 8.0, 400) * np.exp2(rng.integers(-60, 60, 400)))
    a = np.float32(amax * rng.uniform(0, 1, 400) * np.exp2(-rng.integers(0, 40, 400)))
    a[::17] = amax[::17]
    a[::23] = 0
    d = F.mx_offset(F.bits(a), F.bits(amax))
    for ai, mi, di in zip(a, amax, d):
        assert di == _offset_brute(float(ai), float(mi))


def ref_quantize(row, g, row_mode):
    """docs/isa.md "Quantization" of one row, scalar Python (the shape of the reference's
    tests/test_mx.py:34-45 model)."""
    vals = [np.float32(F.ftz(np.float32(t))) for t in row]
    mags = [abs(float(v)) for v in vals]
    amax = np.float32(max(mags))
    S = np.float32(0) if amax == 0 else F.mul(amax, F.INV127)
    inv = np.float32(0) if amax == 0 else F.mul(np.float32(127), F.recip(amax))
    q, ds = [], []
    for i in range(0, len(row), g):
        d = 0 if row_mode else _offset_brute(max(mags[i:i + g]), float(amax))
        ds.append(d)
        ig = F.mul(inv, np.float32(2.0 ** d))
        q += [int(F.q8(F.mul(v, ig))) for v in vals[i:i + g]]
    return q, np.float32(S), ds


@pytest.mark.parametrize("row_mode", [False, True])
@pytest.mark.parametrize("g", [8, 32, 128])
def test_quantize_mx_against_the_scalar_model(row_mode, g):
    rng = np.random.default_rng(1)
    rows, n = 3, 384
    x = (rng.standard_normal((rows, n)) * np.exp(rng.uniform(-6, 6, (rows, n // 8, 1)))
         .repeat(8, axis=2).reshape(rows, -1)).astype(np.float32)
    x[1, 8:40] = 0                                          # zero groups: d = 0
    x[2, 3] = F.from_bits(np.uint32(0x00000123))            # a denormal: flushed
    q, S, d = F.quantize_mx(x, g, row_mode)
    for r in range(rows):
        rq, rS, rd = ref_quantize(x[r], g, row_mode)
        assert q[r].tolist() == rq
        assert _b(S[r]) == _b(rS)
        assert d[r].tolist() == rd


def test_quantize_zero_row():
    q, S, d = F.quantize_mx(np.zeros((2, 128), np.float32), 32)
    assert not q.any() and not S.any() and not d.any()
