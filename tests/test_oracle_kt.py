"""The oracle's MM KT pair layout (docs/isa.md "K tail", opentpu/quant.py:829-880), pinned by
the reference's own checks restated with own inputs (tests/test_kt.py:115-124: one chunk saved a
pair and the refusal of a non-zero upper half; :177-200: the pair stride), every chunk of a pair
against the layout's formula, and the inverse: the KT image ungrouped is the natural rows byte
for byte (so an MM over it is the padded MM bit for bit, tests/test_kt.py:94-106)."""
import numpy as np
import pytest

from oracle import formats as Q
from oracle import groups as G

D = Q.D


def kt_operand(rng, fmt, N, KB):
    """Natural rows and scale rows of a matrix of K = (KB - 1/2) D: the last block's upper half
    zero (the shape tests/test_kt.py:_operand builds)."""
    K = KB * D
    if fmt == "int8":
        el = rng.integers(-127, 128, (N, K))
        el[:, K - D // 2:] = 0
        rows = el.astype(np.int8).view(np.uint8)
    else:
        el = rng.integers(0, 16, (N, K))
        el[:, K - D // 2:] = 0
        rows = np.zeros((N, Q.row_bytes(K, fmt)), np.uint8)
        rows[:, :K // 2] = (el[:, 0::2] | (el[:, 1::2] << 4)).astype(np.uint8)
    sw = (rng.standard_normal(N) * 0.01).astype(np.float32)
    srows = np.zeros((N, Q.scale_bytes(K, fmt)), np.uint8)
    srows[:, :4] = sw[:, None].view(np.uint8)
    h = 4 if fmt == "int8" else 8
    if fmt == "int8":
        srows[:, h:h + KB] = rng.integers(0, 20, (N, KB))
    else:
        word = rng.integers(0, 20, (N, KB)) | sum(rng.integers(0, 64, (N, KB)) << (8 + 6 * b) for b in range(4))
        srows[:, h:h + 4 * KB] = word.astype(np.uint32).view(np.uint8).reshape(N, -1)
    return rows, srows


@pytest.mark.parametrize("fmt", ["int8", "int4", "fp4"])
@pytest.mark.parametrize("groups", [1, 2, 3, 4])
@pytest.mark.parametrize("KB", [1, 2, 5])
def test_kt_pairs_layout_and_inverse(fmt, groups, KB):
    wg = 4
    R = G.grp_r(fmt, wg)
    N = groups * R - (3 if groups == 3 else 0)
    rng = np.random.default_rng(100 * groups + KB + len(fmt))
    rows, srows = kt_operand(rng, fmt, N, KB)
    K = KB * D
    P = wg * D
    g = G.group_rows(rows, N, K, fmt, wg)
    k = G.kt_rows(g, wg)
    pairs = -(-g.shape[0] // 2)
    assert k.shape == (pairs, (2 * KB - 1) * P)                 # one chunk a pair less
    assert g.shape[1] == KB * P
    for p in range(pairs):                                       # every chunk where the formula says
        ev = g[2 * p].reshape(KB, wg, D)
        od = g[2 * p + 1].reshape(KB, wg, D) if 2 * p + 1 < g.shape[0] else np.zeros_like(ev)
        kp = k[p].reshape(2 * KB - 1, wg, D)
        for c in range(KB - 1):
            assert np.array_equal(kp[c], ev[c]) and np.array_equal(kp[KB + c], od[c])
        assert np.array_equal(kp[KB - 1, :, :D // 2], ev[KB - 1, :, :D // 2])
        assert np.array_equal(kp[KB - 1, :, D // 2:], od[KB - 1, :, :D // 2])
    assert np.array_equal(G.ungroup_kt_rows(k, N, K, fmt, wg), rows)
    at = 5 * P
    assert np.array_equal(G.ungroup_kt_rows(G.hash_rows(k, at, wg), N, K, fmt, wg, at=at), rows)
    # scales: the odd groups' entries rotate; the inverse restores every byte that meets data
    a = G.group_scales(srows, N, K, fmt, wg)
    ak = G.kt_scales(a, fmt, K, wg)
    back = G.ungroup_kt_scales(ak, N, K, fmt, wg)
    nat = G.ungroup_scales(a, N, K, fmt, wg)
    if fmt == "int8" or groups < 2:
        assert np.array_equal(back, nat)
    else:
        odd = (np.arange(N) // R) % 2 == 1
        assert np.array_equal(back[~odd], nat[~odd])
        tail = 8 + 4 * (KB - 1)
        mask = np.ones(back.shape[1], bool)
        mask[tail + 2:tail + 4] = False                          # bits 20..31 of the tail word
        assert np.array_equal(back[odd][:, mask], nat[odd][:, mask])
        w = back[odd][:, tail:tail + 4].copy().view("<u4")[:, 0]
        assert np.array_equal((w >> 20) & 0xFFF, (w >> 8) & 0xFFF)
    if groups >= 2 and fmt == "int8":                            # the tail's entry first
        R8 = G.grp_r(fmt, wg)
        pw = G.swp(fmt, R8)
        assert np.array_equal(ak[1, pw:pw + R8], a[1, pw + (KB - 1) * R8:pw + KB * R8])


def test_kt_refuses_a_nonzero_upper_half():
    rng = np.random.default_rng(3)
    rows, _ = kt_operand(rng, "fp4", 16, 3)
    g = G.group_rows(rows, 16, 3 * D, "fp4", 4)
    with pytest.raises(ValueError, match="upper halves"):
        G.kt_rows(g + 1, 4)
