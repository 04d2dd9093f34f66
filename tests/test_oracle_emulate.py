"""The oracle's float64 emulation (oracle/emulate.py), pinned by what it must equal: the
machine's fp32 MM (oracle/mm.py, itself pinned) to fp32 rounding -- and, without the window's
drops, not (the reference's check, tests/test_quant.py:218-241, restated); fake_act's q equal
to the pinned quantizer's away from ties; mx_matmul equal to its definition summed group by
group on small cases."""
import numpy as np
import pytest

from oracle import emulate as EM
from oracle import formats as Q
from oracle import fp32 as F
from oracle import mm as MM

D = Q.D


def _x(rng, M, K, s):
    return (rng.standard_normal((M, K)) * np.exp(s * rng.standard_normal((M, K // 8, 1)))
            .repeat(8, 2).reshape(M, K)).astype(np.float32)


def _spread(rng, N, K, s):
    return (rng.standard_normal((N, K)) * np.exp(s * rng.standard_normal((N, K // 32, 1)))
            .repeat(32, 2).reshape(N, K) * 0.02).astype(np.float32)


@pytest.mark.parametrize("fmt", Q.FMTS)
def test_mm_follows_the_emulation(fmt):
    rng = np.random.default_rng(1)
    M, N, K = 3, 24, 8 * D
    x, W = _x(rng, M, K, 6.0), _spread(rng, N, K, 6.0)
    rows, srows = Q.quantize_mxu(W, fmt)
    q, S, d = F.quantize_mx(x, 32)
    got = MM.mm(q, S, d, rows, srows, fmt, K).astype(np.float64)
    hv, da = EM.fake_act(x)
    wv, dw = EM.fake_w(rows, srows, fmt, K)
    want = EM.mx_matmul(hv, wv, da, dw, Q.WINDOW[fmt])
    plain = EM.mx_matmul(hv, wv)
    assert np.abs(got - want).max() < 1e-6 * np.abs(want).max()
    assert np.abs(got - plain).max() > 100 * np.abs(got - want).max()


def test_fake_act_is_the_quantizer_away_from_ties():
    rng = np.random.default_rng(2)
    x = _x(rng, 8, 1024, 3.0)
    v, da = EM.fake_act(x)
    q, S, d = F.quantize_mx(x, 32)
    assert np.array_equal(np.repeat(d, 2, axis=1), da)              # the same offsets per 16
    amax = np.abs(x.astype(np.float64)).max(1, keepdims=True)
    unit = (amax / 127) * np.exp2(-np.repeat(d, 32, axis=1).astype(np.float64))
    qv = v / unit
    assert np.abs(qv - np.rint(qv)).max() < 1e-9                    # multiples of unit (rounded once)
    qv = np.rint(qv)
    r = x / unit
    far = np.abs(np.abs(r - np.floor(r)) - 0.5) > 1e-4              # not near a tie
    assert far.mean() > 0.99
    assert np.array_equal(qv[far], q.astype(np.float64)[far])
    assert np.abs(qv - q).max() <= 1


def test_fake_act_ties_are_the_devices():
    """Exact ties (x / unit = k + 1/2 in float64) round as the device quantizer rounds them."""
    K = 64
    x = np.zeros((1, K), np.float32)
    x[0, 0] = 127.0                                                 # amax 127: unit 1 (d = 0)
    x[0, 1:] = (np.arange(1, K) % 100 + 0.5).astype(np.float32)     # k + 1/2 exactly
    v, _ = EM.fake_act(x, row=True)
    q = F.quantize_mx(x, 32, row_mode=True)[0]
    assert np.array_equal(v[0], q[0].astype(np.float64))


def test_fake_act_near_ties_defer_to_the_device():
    """Near ties: float64's x / unit within 2^-31 of k + 1/2 without being one (an inexact
    unit = amax / 127), found by a seeded search.  fake_act takes the device quantizer's value
    there, and float64's own rint (a tie window of 0) disagrees with the device on a good share
    of them: the window is what makes fake_act the device's at near ties."""
    rng = np.random.default_rng(17)
    amax = rng.uniform(1, 100, 20000).astype(np.float32)
    s = amax.astype(np.float64) / 127
    k = np.arange(4)
    x = ((k[None, :] + 0.5) * s[:, None]).astype(np.float32)
    r = x.astype(np.float64) / s[:, None]
    dl = np.abs(r - (k[None, :] + 0.5))
    i, j = np.nonzero((dl > 0) & (dl < 2.0 ** -31))
    assert len(i) >= 100
    i, j = i[:128], j[:128]
    rows = np.zeros((len(i), 64), np.float32)
    rows[:, 0] = amax[i]
    rows[:, 1] = x[i, j]
    v, _ = EM.fake_act(rows, row=True)
    q = F.quantize_mx(rows, 32, row_mode=True)[0][:, 1].astype(np.float64)
    assert np.array_equal(np.rint(v[:, 1] / s[i]), q)
    assert (np.rint(r[i, j]) != q).sum() >= 16


def test_mx_matmul_is_its_definition():
    rng = np.random.default_rng(3)
    M, N, K, W = 3, 5, 64, 6
    h = rng.standard_normal((M, K))
    w = rng.standard_normal((N, K))
    da = rng.integers(0, 8, (M, K // 16))
    dw = rng.integers(0, 8, (N, K // 16))
    y = EM.mx_matmul(h, w, da, dw, W)
    for j in range(M):
        for n in range(N):
            t = 0.0
            for g in range(K // 16):
                if da[j, g] + dw[n, g] <= W:
                    t += float(np.dot(h[j, 16 * g:16 * g + 16], w[n, 16 * g:16 * g + 16]))
            assert abs(y[j, n] - t) <= 1e-12 * max(1.0, abs(t))
    assert np.allclose(EM.mx_matmul(h, w), h @ w.T)


def test_group_offsets_layout():
    rng = np.random.default_rng(4)
    W = _spread(rng, 4, 384, 3.0)
    for fmt in Q.FMTS:
        rows, srows = Q.quantize_mxu(W, fmt)
        dw = EM.group_offsets(srows, fmt, 384)
        assert dw.shape == (4, 24)
        _, dws, _ = Q.unpack_scales(srows, fmt, 3)
        assert np.array_equal(dw.reshape(4, 3, 8)[:, :, 0], dws[:, :, 0])
    rows, srows = Q.pack_rsc(W)
    assert not np.any(EM.group_offsets(srows, "int8", 384, rsc=True))
