"""The oracle's weight formats (oracle/formats.py), pinned by what the definitions fix: the
nibble decode tables against two's complement and the E2M1 / E4M3 encodings (OCP MX spec), the
row and scale-row sizes against the values the reference's tests and docs state
(tests/test_quant.py:90-119: K = 640; the configs' 12 / 24 / 40 / 72 / 104-byte scale rows),
scale-row packing round trips, the int8x packer against the pinned quantizer, and the
reference's layout checks (zero block dequantizes to zero, relative error bounds per format)."""
import numpy as np
import pytest

from oracle import formats as Q
from oracle import fp32 as F

D = Q.D


def test_int4_decode_is_twos_complement():
    for c in range(16):
        assert Q.DEC["int4"][c] == (c - 16 if c & 8 else c)


def _e2m1(c):
    """OCP E2M1: sign bit 3, exponent bits 2:1 (bias 1), mantissa bit 0; subnormal at E = 0."""
    s = -1.0 if c & 8 else 1.0
    e, m = (c >> 1) & 3, c & 1
    return s * (m * 0.5 if e == 0 else (1 + m / 2) * 2.0 ** (e - 1))


def test_fp4_decode_is_twice_e2m1():
    for c in range(16):
        assert Q.DEC["fp4"][c] == 2 * _e2m1(c)
        assert Q.DEC["nvfp4"][c] == 2 * _e2m1(c)


def _e4m3(c):
    """OCP E4M3 (bias 7), sign clear: subnormal mantissa / 8 * 2^-6 at E = 0."""
    e, m = (c >> 3) & 15, c & 7
    return m / 8 * 2.0 ** -6 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7)


def test_nvfp4_scale_decode_is_e4m3():
    """MM's B = m << (W - dw - da) with the nvfp4 (dw, m) of a code: m * 2^-dw is the E4M3 value
    times 2^-5 (the reference's `quant.py` note: m 2^(max(E,1) - 10) times 2^-5 Sw)."""
    e4 = np.arange(0x7F, dtype=np.uint8)
    KB = 16
    codes = np.resize(e4, (1, KB, 8))
    sr = Q.pack_scales("nvfp4", np.ones(1, np.float32), e4=codes)
    Sw, dw, m = Q.unpack_scales(sr, "nvfp4", KB)
    got = m * np.exp2(-dw.astype(np.float64))
    want = np.vectorize(_e4m3)(codes.astype(np.int64)) * 2.0 ** -5
    assert np.array_equal(got, want)


def test_nibble_order_low_first():
    assert list(Q.nibbles(np.array([[0x21, 0xF0]], np.uint8))[0]) == [1, 2, 0, 15]
    c = np.random.default_rng(0).integers(0, 16, (5, 64))
    assert np.array_equal(Q.nibbles(Q.pack_nibbles(c)), c)


@pytest.mark.parametrize("K,fmt,rb,sb", [
    (640, "int8", 640, 12), (640, "int4", 384, 32), (640, "fp4", 384, 32), (640, "nvfp4", 384, 64),
    (1024, "int8", 1024, 12), (2048, "int4", 1024, 72), (1024, "int4", 512, 40), (3072, "int4", 1536, 104),
    (2560, "int8", 2560, 24), (128, "int4", 128, 16),
])
def test_row_and_scale_bytes(K, fmt, rb, sb):
    assert Q.row_bytes(K, fmt) == rb
    assert Q.scale_bytes(K, fmt) == sb
    assert Q.scale_bytes(K, fmt, rsc=True) == 4


@pytest.mark.parametrize("fmt", ["int8", "int4", "fp4", "nvfp4"])
def test_scale_rows_round_trip(fmt):
    rng = np.random.default_rng(1)
    N, KB = 6, 5
    Sw = rng.standard_normal(N).astype(np.float32)
    if fmt == "nvfp4":
        e4 = rng.integers(0, 0x7F, (N, KB, 8)).astype(np.uint8)
        sr = Q.pack_scales(fmt, Sw, e4=e4)
        assert sr.shape[1] == Q.scale_bytes(KB * D, fmt)
        assert np.array_equal(sr[:, 16:16 + 8 * KB].reshape(N, KB, 8), e4)
        S2, _, _ = Q.unpack_scales(sr, fmt, KB)
        assert np.array_equal(S2.view(np.uint32), Sw.view(np.uint32))
        return
    dw = rng.integers(0, 256, (N, KB)).astype(np.uint8)
    m = rng.integers(0, 64, (N, KB, 4)).astype(np.uint8)
    sr = Q.pack_scales(fmt, Sw, dw=dw, m=None if fmt == "int8" else m)
    assert sr.shape[1] == Q.scale_bytes(KB * D, fmt)
    S2, dw2, m2 = Q.unpack_scales(sr, fmt, KB)
    assert np.array_equal(S2.view(np.uint32), Sw.view(np.uint32))
    assert np.array_equal(dw2, np.repeat(dw[:, :, None].astype(np.int64), 4, 2))
    if fmt != "int8":
        assert np.array_equal(m2, m)
        # a k0 window reads the later blocks
        _, dw3, m3 = Q.unpack_scales(sr, fmt, 2, k0=3)
        assert np.array_equal(m3, m[:, 3:5]) and np.array_equal(dw3[:, :, 0], dw[:, 3:5])


def test_int8x_is_quantize_mx_in_blocks():
    rng = np.random.default_rng(2)
    W = (rng.standard_normal((7, 640)) * 0.02).astype(np.float32)
    rows, sr = Q.pack_int8x(W)
    q, S, d = F.quantize_mx(W, D)
    assert np.array_equal(rows.view(np.int8), q)
    assert np.array_equal(sr[:, :4].copy().view(np.float32)[:, 0].view(np.uint32), S.view(np.uint32))
    assert np.array_equal(sr[:, 4:9], d) and not np.any(sr[:, 9:])          # padded with zeros


def _spread(rng, N, K, s):
    return (rng.standard_normal((N, K)) * np.exp(s * rng.standard_normal((N, K // 32, 1)))
            .repeat(32, 2).reshape(N, K) * 0.02).astype(np.float32)


@pytest.mark.parametrize("fmt,bound", [("int8", 0.006), ("int4", 0.12), ("fp4", 0.1)])
def test_layout_zero_block_and_error(fmt, bound):
    """The reference's layout check (tests/test_quant.py:90-119): shapes, an all-zero block
    dequantizes to zeros, the relative squared error ||W - deq||^2 / ||W||^2 within the format's
    bound, the 6-bit multipliers in 1..63."""
    rng = np.random.default_rng(2)
    W = _spread(rng, 16, 640, 1.0)
    W[3, 128:256] = 0
    rows, sr = Q.quantize_mxu(W, fmt)
    assert rows.shape == (16, Q.row_bytes(640, fmt)) and sr.shape == (16, Q.scale_bytes(640, fmt))
    deq = Q.dequantize(rows, sr, fmt, 640)
    assert np.all(deq[3, 128:256] == 0)
    err = ((deq - W) ** 2).sum() / (W.astype(np.float64) ** 2).sum()     # relative squared error
    assert err < bound
    if fmt != "int8":
        _, _, m = Q.unpack_scales(sr, fmt, 5)
        assert m.min() >= 1 and m.max() <= 63


def test_e4m3_rounding_is_nearest_even_on_the_grid():
    """oracle e4m3_code (from the binade) against a bracket search of the E4M3 grid: nearest,
    ties to the even code, saturating at 448; every grid value, every midpoint, and random
    values over the whole range and past it."""
    grid = Q.e4m3_value(np.arange(127))
    for c in range(127):
        assert grid[c] == _e4m3(c)
    rng = np.random.default_rng(0)
    a = np.concatenate([grid, (grid[1:] + grid[:-1]) / 2, rng.uniform(0, 500, 20000),
                        np.exp2(rng.uniform(-16, 10, 20000)), [464.0, 480.0, 1e30, 2.0 ** -10]])
    i = np.clip(np.searchsorted(grid, a), 1, 126)
    lo, hi = grid[i - 1], grid[i]
    want = np.where(a - lo < hi - a, i - 1, np.where(hi - a < a - lo, i, i - 1 + (i - 1) % 2))
    want = np.where(a >= 448.0, 126, want)
    assert np.array_equal(Q.e4m3_code(a), want)
    assert Q.e4m3_code(np.array([2.0 ** -10]))[0] == 0          # tie with 0: the even code
    assert Q.e4m3_code(np.array([464.0]))[0] == 126


def test_nv_packer_layout_and_error():
    """nvfp4 rows: Sw = 16 ts (ts = f32(amax / 2688)); the dequantized row is within half an E2M1
    step of a scaled group of W; an all-zero row packs to Sw 16 and scale 1.0 (0x38)."""
    rng = np.random.default_rng(1)
    W = (rng.standard_normal((6, 384)) * 0.02).astype(np.float32)
    W[4] = 0
    rows, srows = Q.pack_nv(W)
    assert rows.shape == (6, Q.row_bytes(384, "nvfp4")) and srows.shape == (6, 48)
    Sw = srows[:, :4].copy().view(np.float32)[:, 0]
    ts = (np.abs(W.astype(np.float64)).max(1) / 2688.0).astype(np.float32)
    assert np.array_equal(Sw[[0, 1, 2, 3, 5]], (16 * ts[[0, 1, 2, 3, 5]].astype(np.float64)).astype(np.float32))
    assert Sw[4] == 16.0 and np.all(srows[4, 16:40] == 0x38)
    assert not np.any(srows[:, 40:]) and not np.any(srows[:, 4:16])
    deq = Q.dequantize(rows, srows, "nvfp4", 384)
    err = np.abs(deq - W.astype(np.float64))
    assert err.max() <= np.abs(W).max() / 6 + 1e-12             # within an E2M1 step of amax


@pytest.mark.parametrize("fmt,qmax", [("int4", 7.0), ("fp4", 6.0)])
def test_packer_block_offset_log2_is_exact(fmt, qmax):
    """The 4-bit packers' block offset floor(log2(v)), v = 63 Sw / bmax in float64: numpy's
    rounded log2 (the reference) and the exponent of v (the GPU packer) agree because v is
    either a power of two or at least ~2^-34 (relative) away from every one: 63 qmax Sw has at
    most 33 significant bits and bmax = rnd(a / qmax) for a float32 a. Checked here on random
    rows, rows whose block maxima differ by powers of two, and the 441 * 2^k family that makes
    v exactly a power of two."""
    import math
    rng = np.random.default_rng(17)
    rows = [_spread(rng, 64, 1024, 2.0)]
    base = rng.standard_normal((64, 1024)).astype(np.float32)
    pw = np.exp2(rng.integers(-12, 1, (64, 8, 1))).astype(np.float32)
    rows.append((base.reshape(64, 8, 128) * 0 + pw * np.float32(0.5)).reshape(64, 1024).astype(np.float32))
    fam = np.zeros((8, 1024), np.float32)
    for r in range(8):
        fam[r, ::128] = np.float32(qmax * 63.0) * np.exp2(-np.arange(8) - r).astype(np.float32)
    rows.append(fam)
    gap_min, exact = 1.0, 0
    for W in rows:
        x = W.astype(np.float64).reshape(W.shape[0], -1, 4, 32)
        sb = np.abs(x).max(-1) / qmax
        top = sb.max(-1).max(-1)
        Sw = np.where(top == 0, 1.0, top / 63).astype(np.float32).astype(np.float64)
        bmax = sb.max(-1)
        ok = bmax > 0
        v = (63 * Sw[:, None] / np.where(ok, bmax, 1.0))[ok]
        e = np.array([math.frexp(t)[1] - 1 for t in v])
        assert np.array_equal(np.floor(np.log2(v)).astype(np.int64), e)
        rel = v / np.exp2(np.round(np.log2(v))) - 1.0
        exact += int((rel == 0).sum())
        gap_min = min(gap_min, float(np.abs(rel[rel != 0]).min()) if np.any(rel != 0) else 1.0)
    print(fmt, "exact powers of two:", exact, "smallest relative gap:", gap_min)
    assert exact > 0 and gap_min > 2.0 ** -36
