"""The oracle's QACT extensions, pinned independently of their restatement:
  * q8lo / quantize_mx(lo=True): a scalar model with exact rationals, as docs/isa.md words the
    lo byte (round(256 (p - q8(p))) half to even, saturated), brute force over a fine grid and
    the float32 neighbours of every half step, and the reconstruction bound the reference states
    (x ~ (q + lo / 256) S 2^-d within 2^-9 of S 2^-d, 2^-8 where lo saturates);
  * qact's RSCALE / CSCALE: a per-element scalar model in the documented order (x * r) * c on
    inputs where that order and x * (r * c) round differently;
  * QACT ST records / LDA: the layout field by field and the round trip;
  * MM SPL: a scalar Python-int model of docs/isa.md's advance table and the closed form at zero
    offsets."""
from fractions import Fraction

import numpy as np
import pytest

from conftest import same_bits
from oracle import fp32 as F
from oracle import mm as MM


def rne(fr: Fraction) -> int:
    """Round a rational to the nearest integer, half to even."""
    fl = fr.numerator // fr.denominator
    rem = fr - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2):
        return fl + 1
    return fl


def q8_scalar(p: float) -> int:
    if p != p:
        return 0
    if p in (np.inf, -np.inf):
        return 127 if p > 0 else -127
    return max(-127, min(127, rne(Fraction(float(p)))))


def q8lo_scalar(p: float) -> int:
    """docs/isa.md: lo = sat127(rint(256 p) - 256 q8(p)); 256 q8 is an integer, so this is the
    rounded 256 (p - q8(p))."""
    if p != p:
        return 0
    if p in (np.inf, -np.inf):
        return 127 if p > 0 else -127
    r = rne(256 * (Fraction(float(p)) - q8_scalar(p)))
    return max(-127, min(127, r))


def test_q8lo_brute_force_and_half_steps():
    grid = np.arange(-130 * 512, 130 * 512 + 1, dtype=np.float64) / 512.0     # every 2^-9 step
    xs = grid.astype(np.float32)
    up = np.nextafter(xs, np.float32(np.inf))
    dn = np.nextafter(xs, np.float32(-np.inf))
    specials = np.float32([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-41, -1e-41, 127.5, -127.5, 127.49998,
                           3e38, -3e38, 2.0 ** -130])
    x = np.concatenate([xs, up, dn, specials]).astype(np.float32)
    got = F.q8lo(x)
    sample = np.random.default_rng(0).choice(x.size, 4000, replace=False)
    for i in list(sample) + list(range(x.size - specials.size, x.size)):
        v = float(F.ftz(x[i:i + 1])[0])
        assert got[i] == q8lo_scalar(v), (x[i], got[i], q8lo_scalar(v))


def test_q8lo_ties_and_saturation_known_answers():
    x = np.float32([0.5, 1.5, 2.5, 1 + 1 / 512, 1 + 3 / 512, -1 - 3 / 512, 127.6, -127.6, np.nan])
    assert F.q8(x).tolist() == [0, 2, 2, 1, 1, -1, 127, -127, 0]
    # 0.5: 128 saturates; 1.5 -> q8 2: -128 saturates; 256.5 -> 256 (even); 257.5 -> 258
    assert F.q8lo(x).tolist() == [127, -127, 127, 0, 2, -2, 127, -127, 0]


@pytest.mark.parametrize("row_mode", [False, True])
def test_quantize_mx_lo_reconstructs_within_the_stated_bound(row_mode):
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((6, 512)) * np.exp(rng.uniform(-6, 6, (6, 16, 1))).repeat(32, 2)
         .reshape(6, 512)).astype(np.float32)
    x[2] = 0
    q, S, d = F.quantize_mx(x, 32, row_mode)
    lo, Sl, d2 = F.quantize_mx(x, 32, row_mode, lo=True)
    assert np.array_equal(d, d2)
    assert same_bits(Sl, F.mul(S, np.float32(2.0 ** -8)))
    for r in range(6):
        if S[r] == 0:
            assert not q[r].any() and not lo[r].any()
            continue
        amax = np.abs(x[r]).max()
        sc = np.repeat(np.exp2(-d[r].astype(np.float64)), 32)               # 2^-d per element
        p = x[r].astype(np.float64) / (amax / 127.0) / sc                   # ~ the product p
        rec = q[r].astype(np.float64) + lo[r].astype(np.float64) / 256.0
        err = np.abs(rec - p)
        sat = np.abs(lo[r]) == 127
        # within 2^-9 of one unit (plus the rounding of inv and of p, ~2^-22 relative)
        assert np.all(err[~sat] <= 2.0 ** -9 + 1e-4 * np.maximum(1, np.abs(p[~sat])))
        assert np.all(err[sat] <= 2.0 ** -8 + 1e-4 * np.maximum(1, np.abs(p[sat])))


def test_qact_premultiplies_in_the_documented_order():
    rng = np.random.default_rng(5)
    M, K = 4, 256
    x = (rng.standard_normal((M, K)) * 3).astype(np.float32)
    r = (rng.uniform(0.5, 2, M)).astype(np.float32)
    c = (rng.uniform(0.5, 2, K)).astype(np.float32)
    c[7] = np.float32(1e-39)                                    # a denormal factor: flushed
    xr = np.empty_like(x)
    for i in range(M):
        for j in range(K):
            xr[i, j] = F.mul(F.mul(x[i, j], r[i]), c[j])
    q0, S0, d0 = F.quantize_mx(xr, 32)
    q, S, d = F.qact(x, 32, rscale=r, cscale=c)
    assert np.array_equal(q, q0) and same_bits(S, S0) and np.array_equal(d, d0)
    # the other association rounds differently somewhere: the order is pinned
    alt = F.mul(x, F.mul(r[:, None], c[None, :]))
    assert not same_bits(alt, xr)
    # each factor alone
    q1, S1, _ = F.qact(x, 32, rscale=r)
    assert np.array_equal(q1, F.quantize_mx(F.mul(x, r[:, None]), 32)[0])
    q2, S2, _ = F.qact(x, 32, cscale=c)
    assert np.array_equal(q2, F.quantize_mx(F.mul(x, c[None, :]), 32)[0])
    # HL: both halves of one read
    qh, Sh, dh, ql, Sl = F.qact(x, 32, rscale=r, cscale=c, hl=True)
    assert np.array_equal(qh, q) and np.array_equal(dh, d)
    assert np.array_equal(ql, F.quantize_mx(xr, 32, lo=True)[0])


def test_qrows_store_layout_and_lda_round_trip():
    rng = np.random.default_rng(6)
    KB, rows = 3, 5
    x = (rng.standard_normal((rows, KB * 128)) * np.exp(rng.uniform(-4, 4, (rows, KB * 4, 1)))
         .repeat(32, 2).reshape(rows, -1)).astype(np.float32)
    q, S, d = F.quantize_mx(x, 32)
    b = F.qrows_store(q, S, d)
    assert b.shape == (rows, KB * 128 + 8 * KB) and F.qrow_bytes(KB) == KB * 136
    for r in range(rows):
        assert bytes(b[r, :KB * 128]) == q[r].tobytes()
        for k in range(KB):
            rec = b[r, KB * 128 + 8 * k:KB * 128 + 8 * k + 8]
            assert rec[:4].tobytes() == np.float32(S[r]).tobytes()            # little-endian S
            assert list(rec[4:]) == list(d[r, 4 * k:4 * k + 4])
    q2, S2, d2 = F.lda(b, KB)
    assert np.array_equal(q2, q) and np.array_equal(d2, d)
    assert S2.shape == (KB, rows) and all(same_bits(S2[k], S) for k in range(KB))


def spl_scalar(q, Sa, da, wh, wl, Sw, nterms):
    """docs/isa.md "Split terms": advance k's ACT block (KB 3: hi, lo, hi; KB 2: hi, hi), its
    weight part (KB 3: hi, hi, lo; KB 2: hi, lo), the extra offset (0, 8, 8 / 0, 8)."""
    M, N = q.shape[0], wh.shape[0]
    adv = [(0, "h", 0), (1, "h", 8), (0, "l", 8)] if nterms == 3 else [(0, "h", 0), (0, "l", 8)]
    y = np.zeros((M, N), np.float32)
    for j in range(M):
        for n in range(N):
            acc = 0
            for blk, part, e in adv:
                w = wh if part == "h" else wl
                for g in range(4):
                    c = sum(int(q[j, blk * 128 + g * 32 + i]) * int(w[n, g * 32 + i]) for i in range(32))
                    sh = 16 - (int(da[j, g]) + e)
                    if sh >= 0:
                        acc += c << sh
            y[j, n] = F.mul(F.mul(np.float32(float(acc)), Sw[n]), F.mul(np.float32(Sa[j]), np.float32(2.0 ** -16)))
    return y


@pytest.mark.parametrize("nterms", [2, 3])
def test_mm_spl_scalar_model_and_closed_form(nterms):
    rng = np.random.default_rng(nterms)
    M, N = 3, 6
    x = (rng.standard_normal((M, 128)) * np.exp(rng.uniform(-7, 1, (M, 4, 1))).repeat(32, 2)
         .reshape(M, 128)).astype(np.float32)
    x[0, 96:] *= np.float32(2.0 ** -11)       # a group at offset >= 9: its lo terms drop
    qh, Sa, da, ql, _ = F.qact(x, 32, hl=True)
    q = np.concatenate([qh, ql], 1)
    W = (rng.standard_normal((N, 128)) * 0.02).astype(np.float32)
    wh, Sw, _ = F.quantize_mx(W, 128, row_mode=True)
    wl, _, _ = F.quantize_mx(W, 128, row_mode=True, lo=True)
    got = MM.mm_spl(q if nterms == 3 else qh, Sa, da, wh, wl, Sw, nterms)
    assert same_bits(got, spl_scalar(q, Sa, da, wh, wl, Sw, nterms))
    assert da.max() >= 9                      # some lo terms drop (shift 8 - da < 0)
    # zero offsets: acc = 2^16 hi.wh + 2^8 (lo.wh + hi.wl)
    z = np.zeros_like(da)
    acc = (qh.astype(np.int64) @ wh.astype(np.int64).T) << 16
    acc += ((ql.astype(np.int64) @ wh.astype(np.int64).T) if nterms == 3 else 0) << 8
    acc += (qh.astype(np.int64) @ wl.astype(np.int64).T) << 8
    want = F.mul(F.mul(F.i2f(acc), Sw[None, :]), F.mul(Sa, np.float32(2.0 ** -16))[:, None])
    assert same_bits(MM.mm_spl(q if nterms == 3 else qh, Sa, z, wh, wl, Sw, nterms), want)
    old = rng.standard_normal((M, N)).astype(np.float32)
    assert same_bits(MM.mm_spl(q, Sa, da, wh, wl, Sw, nterms, old=old), F.add(old, got))
