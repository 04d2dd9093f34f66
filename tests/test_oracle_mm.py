"""The oracle's MM and ARGMAX, pinned by a scalar Python-int model written from docs/isa.md
(the shape of the reference's tests/test_mx.py:131-199: every format x UNIT/RSC/k0/big
offsets), the reference's integer model with asserted drops (tests/test_isa.py:85-118),
closed forms and the ARGMAX known answers of tests/test_autodecode.py:26-40 (restated)."""
import numpy as np
import pytest

from conftest import same_bits
from oracle import formats as Q
from oracle import fp32 as F
from oracle import mm as MM

D = Q.D


def scale_rows(rng, fmt, N, KBr, rsc, big):
    """Random scale rows [N, srs] and their (Sw, dw [N, KBr, G], m [N, KBr, G])."""
    G = 8 if fmt == "nvfp4" else 4
    sw = (rng.standard_normal(N) * 0.01).astype(np.float32)
    hi = 20 if big else 4
    if rsc:
        return (sw[:, None].view(np.uint8).copy(), sw, np.zeros((N, KBr, G), int),
                np.ones((N, KBr, G), int))
    if fmt == "int8":
        dw = rng.integers(0, hi, (N, KBr))
        return (Q.pack_scales("int8", sw, dw=dw), sw, np.repeat(dw[:, :, None], G, 2),
                np.ones((N, KBr, G), int))
    if fmt in ("int4", "fp4"):
        dw = rng.integers(0, hi, (N, KBr))
        m = rng.integers(0, 64, (N, KBr, G))
        return Q.pack_scales(fmt, sw, dw=dw, m=m), sw, np.repeat(dw[:, :, None], G, 2), m
    e4 = rng.integers(0, 0x7F, (N, KBr, G))
    if big:
        e4[rng.random(e4.shape) < 0.3] &= 0x0F                      # small exponents: drops
    E, mt = (e4 >> 3) & 15, e4 & 7
    return Q.pack_scales("nvfp4", sw, e4=e4), sw, 15 - np.maximum(E, 1), np.where(E > 0, 8 + mt, mt)


def ref_mm(q, Sa, da, wel, sw, dw, m, fmt):
    """MM's outputs from the definition with Python integers: q [M, K], wel [N, K] ints,
    da [M, K/32], dw / m [N, KB, G]."""
    M, K = q.shape
    N, KB, G = dw.shape
    W = Q.WINDOW[fmt]
    gs = D // G
    y = np.zeros((M, N), np.float32)
    for j in range(M):
        for n in range(N):
            acc = 0
            for k in range(KB):
                for g in range(G):
                    lo = k * D + g * gs
                    c = sum(int(q[j, i]) * int(wel[n, i]) for i in range(lo, lo + gs))
                    sh = W - int(dw[n, k, g]) - int(da[j, (k * D + g * gs) // 32])
                    if sh >= 0:
                        acc += (int(m[n, k, g]) << sh) * c
            assert abs(acc) < 2 ** 47
            y[j, n] = F.mul(F.mul(np.float32(float(acc)), sw[n]),
                            F.mul(np.float32(Sa[j]), np.float32(2.0 ** -W)))
    return y


CASES = [  # fmt, unit, rsc, k0, big offsets
    ("int8", False, False, 0, False), ("int8", False, False, 3, True),
    ("int8", False, True, 0, False), ("int8", True, False, 0, False),
    ("fp4", False, False, 1, False), ("fp4", False, False, 2, True),
    ("int4", False, False, 0, False), ("int4", False, False, 1, True),
    ("fp4", True, False, 0, False), ("fp4", False, True, 0, False),
    ("nvfp4", False, False, 1, True), ("nvfp4", False, False, 2, False),
]


def mm_case(fmt, unit, rsc, k0, big, KB, M=3, N=5, seed=None):
    rng = np.random.default_rng(seed if seed is not None else
                                1000 * Q.WF[fmt] + 10 * KB + k0 + 3 * unit + rsc)
    K = KB * D
    x = (rng.standard_normal((M, K)) * np.exp(rng.uniform(-8 if big else -2, 2, (M, K // 32, 1)))
         .repeat(32, axis=2).reshape(M, -1)).astype(np.float32)
    q, Sa, da = F.quantize_mx(x, 32)
    KBr = k0 + KB
    if fmt == "int8":
        wel = rng.integers(-127, 128, (N, K))
        rows = wel.astype(np.int8).view(np.uint8)
    else:
        codes = rng.integers(0, 16, (N, K))
        wel = Q.DEC[fmt][codes]
        rows = np.zeros((N, Q.row_bytes(K, fmt)), np.uint8)
        rows[:, :K // 2] = Q.pack_nibbles(codes)
    srows, sw, dw, m = scale_rows(rng, fmt, N, KBr, rsc, big)
    return dict(q=q, Sa=Sa, da=da, rows=rows, srows=srows, wel=wel, sw=sw, dw=dw, m=m, K=K)


@pytest.mark.parametrize("fmt,unit,rsc,k0,big", CASES)
@pytest.mark.parametrize("KB", [1, 3])
def test_mm_is_one_integer_per_output(fmt, unit, rsc, k0, big, KB):
    c = mm_case(fmt, unit, rsc, k0, big, KB)
    flags = (MM.UNIT if unit else 0) | (MM.RSC if rsc else 0)
    got = MM.mm(c["q"], c["Sa"], c["da"], c["rows"], c["srows"], fmt, c["K"], flags=flags, k0=k0)
    sw, dw, m = c["sw"], c["dw"][:, k0:k0 + KB], c["m"][:, k0:k0 + KB]
    if unit:
        sw, dw, m = np.ones_like(sw), np.zeros_like(dw), np.ones_like(m)
    want = ref_mm(c["q"], c["Sa"], c["da"], c["wel"], sw, dw, m, fmt)
    assert same_bits(got, want)


def test_mm_integer_model_with_drops():
    """Activations spread over 2^-14..1 per 32 and weight offsets up to 11: groups drop."""
    rng = np.random.default_rng(0)
    M, N, K = 3, 5, 256
    x = (rng.standard_normal((M, K)) * np.repeat(np.exp2(rng.integers(-14, 1, (M, K // 32))), 32, 1)
         ).astype(np.float32)
    w = rng.integers(-127, 128, (N, K)).astype(np.int8)
    sw = rng.uniform(0.01, 0.1, N).astype(np.float32)
    dw = rng.integers(0, 12, (N, 2)).astype(np.uint8)
    srows = Q.pack_scales("int8", sw, dw=dw)
    q, sa, da = F.quantize_mx(x, 32)
    y = MM.mm(q, sa, da, w.view(np.uint8), srows, "int8", K)
    acc = np.zeros((M, N), np.int64)
    dropped = 0
    for t in range(K // 32):
        g = slice(32 * t, 32 * t + 32)
        c = q[:, g].astype(np.int64) @ w[:, g].astype(np.int64).T
        sh = 16 - dw[None, :, t // 4].astype(np.int64) - da[:, t, None].astype(np.int64)
        acc += np.where(sh >= 0, c << np.maximum(sh, 0), 0)
        dropped += int((sh < 0).sum())
    want = F.mul(F.mul(acc.astype(np.float64).astype(np.float32), sw[None, :]),
                 F.mul(sa[:, None], np.float32(2.0 ** -16)))
    assert dropped > 0 and same_bits(y, want)


def test_rsc_with_row_activations_is_a_plain_integer_dot():
    """Closed form: RSC weights and ROW activations give acc = 2^16 * sum q w."""
    rng = np.random.default_rng(4)
    x = rng.standard_normal((4, 512)).astype(np.float32)
    W = (rng.standard_normal((7, 512)) * 0.02).astype(np.float32)
    q, Sa, da = F.quantize_mx(x, 32, row_mode=True)
    rows, srows = Q.pack_rsc(W)
    acc, _ = MM.mm_acc(q, da, rows, srows, "int8", 512, flags=MM.RSC)
    dot = q.astype(np.int64) @ rows.view(np.int8).astype(np.int64).T
    assert np.array_equal(acc, dot << 16)
    y = MM.mm(q, Sa, da, rows, srows, "int8", 512, flags=MM.RSC)
    Sw = srows.view(np.float32)[:, 0]
    want = F.mul(F.mul(F.i2f(dot), Sw[None, :]), Sa[:, None])      # 2^16 * 2^-16 cancel exactly
    assert same_bits(y, want)


def test_unit_is_the_plain_integer_dot():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((2, 256)).astype(np.float32)
    q, Sa, da = F.quantize_mx(x, 32, row_mode=True)
    codes = rng.integers(0, 16, (3, 256))
    rows = np.zeros((3, 128), np.uint8)
    rows[:, :128] = Q.pack_nibbles(codes)
    acc, Sw = MM.mm_acc(q, da, rows, np.zeros((3, 8), np.uint8), "int4", 256, flags=MM.UNIT)
    assert np.array_equal(acc, (q.astype(np.int64) @ Q.DEC["int4"][codes].T) << 11)
    assert np.all(Sw == 1)


def test_acc_ascale_rmax():
    rng = np.random.default_rng(6)
    M, N, K = 2, 3, 256
    x = rng.standard_normal((M, K)).astype(np.float32)
    q, Sa, da = F.quantize_mx(x, 32)
    wel = rng.integers(-127, 128, (N, K)).astype(np.int8)
    old = rng.standard_normal((M, N)).astype(np.float32)
    alpha = rng.standard_normal(M).astype(np.float32)
    srows = np.zeros((N, 12), np.uint8)
    base = MM.mm(q, Sa, da, wel.view(np.uint8), srows, "int8", K, flags=MM.UNIT)
    acc = MM.mm(q, Sa, da, wel.view(np.uint8), srows, "int8", K, flags=MM.UNIT | MM.ACC, old=old)
    assert same_bits(acc, F.add(old, base))
    asc = MM.mm(q, Sa, da, wel.view(np.uint8), srows, "int8", K,
                flags=MM.UNIT | MM.ACC | MM.ASCALE, old=old, alpha=alpha)
    assert same_bits(asc, F.add(F.mul(old, alpha[:, None]), base))
    y, mx = MM.mm(q, Sa, da, wel.view(np.uint8), srows, "int8", K, flags=MM.UNIT | MM.RMAX)
    assert same_bits(mx, [max(r, key=lambda v: float(v)) for r in y])
    with pytest.raises(ValueError):
        MM.mm(q, Sa, da, wel.view(np.uint8), srows, "int8", K, flags=MM.ASCALE)


def test_argmax_first_index_of_the_total_order_max():
    rng = np.random.default_rng(0)
    a = rng.standard_normal((5, 300)).astype(np.float32)
    a[1, [7, 40, 299]] = 9.0                       # ties: the first column
    a[2] = -np.inf
    a[2, 250] = -1e30
    a[3, :] = 0.0
    a[3, 100] = -0.0                               # -0 < +0: +0 at column 0 wins
    a[4, :] = -1.0
    a[4, 5], a[4, 9] = 1e-41, 0.0                  # a denormal flushes to +0: column 5 first
    v, idx = MM.argmax(a)
    assert list(idx) == [int(np.argmax(a[0])), 7, 250, 0, 5]
    assert same_bits(v, [a[0].max(), 9.0, -1e30, 0.0, 0.0])
    _, idx = MM.argmax(a, base=1000)
    assert idx[1] == 1007
    for r in a:
        w = MM.best_word(r)
        assert (~w & 0xFFFFFFFF) == MM.greedy(r)
    nan = np.float32([1.0, np.nan, 3.0])
    assert MM.greedy(nan) == 1                     # the canonical NaN is above +inf
