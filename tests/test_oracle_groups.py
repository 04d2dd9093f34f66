"""The oracle's grouped weight layouts (oracle/groups.py), pinned by what the layout's definition
fixes (docs/isa.md "Weight groups", the reference's tests/test_wg.py:125-216): the channel hash's
known answers, a scale area's offsets and a 4-bit chunk's nibbles checked field by field, WG = 1
the natural layout, round trips, the hash as its own inverse and as a per-chunk lane
permutation, and the strides' closed forms."""
import numpy as np
import pytest

from oracle import formats as Q
from oracle import groups as G

D = G.D
FMTS = ("int8", "int4", "fp4", "nvfp4")


def _rows(rng, N, K, fmt):
    """Natural element rows: int8 random bytes; 4-bit random codes packed, the pad zero."""
    if fmt == "int8":
        return rng.integers(0, 256, (N, K)).astype(np.uint8)
    out = np.zeros((N, Q.row_bytes(K, fmt)), np.uint8)
    out[:, :K // 2] = Q.pack_nibbles(rng.integers(0, 16, (N, K)))
    return out


def _srows(rng, N, K, fmt, rsc=False):
    """Natural scale rows: Sw and the blocks' data random, the reserved words and padding 0."""
    out = np.zeros((N, Q.scale_bytes(K, fmt, rsc)), np.uint8)
    out[:, :4] = rng.integers(0, 256, (N, 4))
    if not rsc:
        h, sb = G.swp(fmt, 1), G.SCALE_DATA[fmt]
        out[:, h:h + (K // D) * sb] = rng.integers(0, 256, (N, (K // D) * sb))
    return out


def _bits_fold(m, R):
    """The fold by its definition: bit i of m goes to bit i mod log2 R, XORed."""
    b = R.bit_length() - 1
    h = 0
    for i in range(max(m.bit_length(), 1)):
        if b and (m >> i) & 1:
            h ^= 1 << (i % b)
    return h


def test_chunk_fold_known_answers():
    assert G.chunk_fold(0b100_011_110, 8) == 1
    assert [G.chunk_fold(m, 1) for m in range(5)] == [0] * 5
    rng = np.random.default_rng(0)
    for R in (1, 2, 4, 8, 16, 32, 64):
        for m in [0, 1, R - 1, R, (1 << 31) - 1] + rng.integers(0, 1 << 40, 50).tolist():
            assert G.chunk_fold(int(m), R) == _bits_fold(int(m), R), (m, R)


@pytest.mark.parametrize("fmt,p", [("int8", 32), ("fp4", 64), ("nvfp4", 128)])
def test_scale_area_offsets(fmt, p):
    """WG 8: rows j's Sw word j + 1 at 4 j; block k's data at SWP + (k R + j) SB."""
    R, KB, sb, h = G.grp_r(fmt, 8), 3, G.SCALE_DATA[fmt], G.swp(fmt, 1)
    assert G.swp(fmt, R) == p and R == (8 if fmt == "int8" else 16)
    rows = np.zeros((R, Q.scale_bytes(KB * D, fmt)), np.uint8)
    for j in range(R):
        rows[j, :4] = np.array([j + 1], np.uint32).view(np.uint8)
        for k in range(KB):
            rows[j, h + sb * k:h + sb * (k + 1)] = (np.arange(sb) * 7 + 13 * k + j) % 251
    a = G.group_scales(rows, R, KB * D, fmt, 8)[0]
    assert a.size == G.grp_scale_bytes(KB * D, fmt, 8) == -(-(p + KB * R * sb) // p) * p
    assert a[:4 * R].view(np.uint32).tolist() == list(range(1, R + 1))
    for k in range(KB):
        for j in range(R):
            assert a[p + sb * (k * R + j):][:sb].tolist() == rows[j, h + sb * k:][:sb].tolist()


@pytest.mark.parametrize("fmt", ["int4", "fp4", "nvfp4"])
def test_4bit_chunk_layout(fmt):
    """Lane l of chunk c: byte i = element i of block c of row 2l (low nibble), 2l + 1 (high);
    an odd KB leaves no half-used chunk; rows past N read 0."""
    rng = np.random.default_rng(4)
    wg, N, KB = 8, 21, 3
    codes = rng.integers(0, 16, (N, KB * D))
    rows = np.zeros((N, Q.row_bytes(KB * D, fmt)), np.uint8)
    rows[:, :KB * D // 2] = Q.pack_nibbles(codes)
    g = G.group_rows(rows, N, KB * D, fmt, wg)
    assert g.shape == (2, KB * wg * D) == (2, G.grp_row_bytes(KB * D, fmt, wg))
    for n in range(32):
        q, l, hi = n // 16, n % 16 // 2, n % 2
        for c in range(KB):
            lane = g[q, c * wg * D + l * D:c * wg * D + (l + 1) * D]
            got = (lane >> 4) if hi else (lane & 15)
            want = codes[n, c * D:(c + 1) * D] if n < N else np.zeros(D)
            assert np.array_equal(got, want), (n, c)
    assert np.array_equal(G.ungroup_rows(g, N, KB * D, fmt, wg), rows)


def test_int8_chunk_layout():
    """Lane l of chunk c of group g: row g R + l's block c, D bytes."""
    rng = np.random.default_rng(5)
    wg, N, KB = 4, 10, 3
    rows = _rows(rng, N, KB * D, "int8")
    g = G.group_rows(rows, N, KB * D, "int8", wg)
    assert g.shape == (3, KB * wg * D)
    for n in range(12):
        for c in range(KB):
            got = g[n // wg, c * wg * D + (n % wg) * D:][:D]
            want = rows[n, c * D:(c + 1) * D] if n < N else np.zeros(D)
            assert np.array_equal(got, want)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("wg", [1, 2, 8])
@pytest.mark.parametrize("KB", [1, 3, 4])
def test_round_trips(fmt, wg, KB):
    rng = np.random.default_rng(wg * 10 + KB)
    N, K = 13, KB * D
    rows, srows = _rows(rng, N, K, fmt), _srows(rng, N, K, fmt)
    g, a = G.group_rows(rows, N, K, fmt, wg), G.group_scales(srows, N, K, fmt, wg)
    R = G.grp_r(fmt, wg)
    assert g.shape == (-(-N // R), G.grp_row_bytes(K, fmt, wg))
    assert a.shape == (-(-N // R), G.grp_scale_bytes(K, fmt, wg))
    assert np.array_equal(G.ungroup_rows(g, N, K, fmt, wg), rows)
    assert np.array_equal(G.ungroup_scales(a, N, K, fmt, wg), srows)
    if wg == 1:                                          # the natural layout, byte for byte
        assert np.array_equal(g, rows) and np.array_equal(a, srows)
    if fmt != "nvfp4":
        sr = srows[:, :4].copy()
        ar = G.group_scales(sr, N, K, fmt, wg, rsc=True)
        assert ar.shape[1] == 4 * R
        assert np.array_equal(G.ungroup_scales(ar, N, K, fmt, wg, rsc=True), sr)


def test_hash_is_a_per_chunk_lane_permutation():
    rng = np.random.default_rng(9)
    R, N, nc = 8, 24, 5
    g = G.group_rows(_rows(rng, N, nc * D, "int8"), N, nc * D, "int8", R)
    nat = g.reshape(-1, R, D)
    for at in (0, R * D, 37 * R * D, (1 << 31) - 4 * R * D):
        h = G.hash_rows(g, at, R)
        assert np.array_equal(G.hash_rows(h, at, R), g)
        hs = h.reshape(-1, R, D)
        for t in range(len(nat)):
            f = _bits_fold(at // (R * D) + t, R)
            for j in range(R):
                assert np.array_equal(hs[t, j ^ f], nat[t, j])
        moved = G.hash_rows(G.hash_rows(h, at, R), at + 3 * R * D, R)
        assert np.array_equal(moved, G.hash_rows(g, at + 3 * R * D, R))
    with pytest.raises(ValueError, match="whole 1024-byte chunks"):
        G.hash_rows(g, D, R)


def test_strides_closed_forms():
    for K in (128, 384, 2560):
        KB = K // D
        for wg in (1, 2, 8, 16):
            assert G.grp_row_bytes(K, "int8", wg) == K * wg
            x4 = G.grp_row_bytes(K, "int4", wg)
            assert x4 == (-(-K // 256) * 128 if wg == 1 else KB * wg * D)
            if wg > 1:      # two rows a lane: half of two rows' int8 bytes, no half-used chunk
                assert x4 == 2 * wg * K // 2
