"""GPU parity of the float64 emulation (otpu_fake_act, otpu_dequant, otpu_mx_matmul through
opentpu_amd.quant): fake_act's values and offsets and the dequantized weights bit for bit with
the oracle, mx_matmul within float64 summation rounding (1e-12 of the largest output), and the
reference's check on the GPU: the machine's fp32 MM is the emulation to fp32 rounding, and
without the window's drops it is not."""
import sys

import numpy as np
import pytest

from oracle import emulate as EM
from oracle import formats as Q
from oracle import fp32 as F

pytestmark = pytest.mark.gpu
D = Q.D


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def QA():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    from opentpu_amd import _lib, quant
    _lib.load()
    return quant


def _x(rng, M, K, s):
    return (rng.standard_normal((M, K)) * np.exp(s * rng.standard_normal((M, K // 8, 1)))
            .repeat(8, 2).reshape(M, K)).astype(np.float32)


def _spread(rng, N, K, s):
    return (rng.standard_normal((N, K)) * np.exp(s * rng.standard_normal((N, K // 32, 1)))
            .repeat(32, 2).reshape(N, K) * 0.02).astype(np.float32)


@pytest.mark.parametrize("M,K,n,row,g", [(3, 1024, None, False, 32), (5, 512, 256, False, 32),
                                         (2, 1024, None, True, 32), (4, 768, 384, False, 128),
                                         (1, 2560, None, False, 32)])
def test_fake_act(QA, M, K, n, row, g):
    """The reference's positional order fake_act(x, D, n, row, g): an MXAct whose values and da
    equal the oracle's."""
    say(f"fake_act M={M} K={K} n={n} row={row} g={g}")
    rng = np.random.default_rng(K + M)
    x = _x(rng, M, K, 4.0)
    x[0, :64] = (np.arange(64) % 50 + 0.5).astype(np.float32) * np.float32(x[0].max() / 127)   # near-ties
    x[-1, 5] = 1e-40                                                # a denormal
    a = QA.fake_act(x, 128, n, row, g)
    v0, da0 = EM.fake_act(x, n=n, row=row, g=g)
    assert isinstance(a, QA.MXAct) and a.shape == (M, K)
    assert np.array_equal(a.view(np.ndarray).view(np.uint64), v0.view(np.uint64))
    assert a.da.dtype == np.int64 and np.array_equal(a.da, da0)
    assert QA.fake_act(x, n=n, row=row, g=g if g != 32 else None).da.shape == (M, K // 16)


def test_fake_act_float64_ranges_and_leading_axes(QA):
    """float64 input read as float64 (values fp32 cannot hold), ranges of their own widths, and
    a [2, 3, K] input: the oracle's values, range by range."""
    say("fake_act float64, ranges, leading axes")
    rng = np.random.default_rng(4)
    x = rng.standard_normal((2, 3, 1024)) * np.exp(rng.uniform(-3, 3, (2, 3, 64, 1))).repeat(16, 3).reshape(2, 3, 1024)
    assert not np.array_equal(x, x.astype(np.float32))
    a = QA.fake_act(x)
    v0, da0 = EM.fake_act(x)
    assert np.array_equal(a.view(np.ndarray).view(np.uint64), v0.view(np.uint64))
    assert np.array_equal(a.da, da0.reshape(2, 3, 64))
    widths = [256, 512, 256]
    b = QA.fake_act(x, 128, widths)
    for i, (c0, w) in enumerate(zip((0, 256, 768), widths)):
        v1, d1 = EM.fake_act(x[..., c0:c0 + w])
        assert np.array_equal(b.view(np.ndarray)[..., c0:c0 + w].view(np.uint64), v1.view(np.uint64))
        assert np.array_equal(b.da[..., c0 // 16:(c0 + w) // 16], d1.reshape(2, 3, -1))
    with pytest.raises(ValueError):
        QA.fake_act(x, 128, [256, 256])
    with pytest.raises(ValueError):
        QA.fake_act(x, 64)                                          # D 64: not this path's


def test_fake_act_exact_ties(QA):
    say("fake_act exact ties")
    x = np.zeros((1, 64), np.float32)
    x[0, 0] = 127.0
    x[0, 1:] = (np.arange(1, 64) % 100 + 0.5).astype(np.float32)
    a = QA.fake_act(x, row=True)
    assert np.array_equal(a.view(np.ndarray)[0], F.quantize_mx(x, 32, row_mode=True)[0][0].astype(np.float64))


@pytest.mark.parametrize("fmt,rsc", [("int8", False), ("int8", True), ("int4", False), ("fp4", False),
                                     ("nvfp4", False)])
def test_dequant(QA, fmt, rsc):
    """dequantize_mxu(rows, srows, fmt, K, D, rsc) -> the matrix; group_offsets(srows, fmt, K, D,
    rsc) -> dw, both the oracle's; srows None: the elements themselves (UNIT)."""
    say(f"dequant {fmt} rsc={rsc}")
    rng = np.random.default_rng(7)
    W = _spread(rng, 40, 640, 4.0)
    rows, srows = Q.pack_rsc(W) if rsc else Q.quantize_mxu(W, fmt)
    srows = srows.copy()
    srows[3, :4] = np.array([1e-40], np.float32).view(np.uint8)     # a denormal Sw reads 0
    v = QA.dequantize_mxu(rows, srows, fmt, 640, 128, rsc)
    dw = QA.group_offsets(srows, fmt, 640, 128, rsc)
    v0, dw0 = EM.fake_w(rows, srows, fmt, 640, rsc=rsc)
    assert v.shape == (40, 640) and np.array_equal(v.view(np.uint64), v0.view(np.uint64))
    assert dw.dtype == np.int64 and np.array_equal(dw, dw0)
    u = QA.dequantize_mxu(rows, None, fmt, 640)
    assert np.array_equal(u, Q.elements(rows, fmt, 640).astype(np.float64))


@pytest.mark.parametrize("M,N,K,W,mode", [(3, 24, 1024, 16, "both"), (7, 100, 512, 11, "both"),
                                          (2, 33, 256, 13, "one_dw"), (4, 17, 384, 16, "no_da")])
def test_mx_matmul(QA, M, N, K, W, mode):
    """mx_matmul(h, w, dw, W, D) with h an MXAct (or plain), within float64 summation rounding
    (1e-12 of the largest output) of the oracle."""
    say(f"mx_matmul M={M} N={N} K={K} W={W} {mode}")
    rng = np.random.default_rng(M * N)
    h = rng.standard_normal((M, K))
    w = rng.standard_normal((N, K))
    da = rng.integers(0, 12, (M, K // 16)).astype(np.uint8)
    dw = rng.integers(0, 12, (1 if mode == "one_dw" else N, K // 16)).astype(np.uint8)
    if mode == "no_da":
        y = QA.mx_matmul(h, w)
        want = EM.mx_matmul(h, w)
    else:
        y = QA.mx_matmul(QA.MXAct.of(h, da), w, dw, W, 128)
        want = EM.mx_matmul(h, w, da, dw, W)
    assert isinstance(y, np.ndarray) and y.shape == (M, N)
    assert np.abs(y - want).max() <= 1e-12 * np.abs(want).max()


@pytest.mark.parametrize("fmt", Q.FMTS)
def test_mm_follows_the_emulation(QA, fmt):
    """The reference's own check (`tests/test_quant.py:218-241`) written as it writes it:
    fake_act(x) @ fake_w(W, fmt).T is the machine's MM to fp32 rounding, and without the window's
    drops (the plain float64 product) it is not."""
    from opentpu_amd import mxu
    say(f"mm vs emulation {fmt}")
    rng = np.random.default_rng(1)
    M, N, K = 3, 24, 8 * D
    x, W = _x(rng, M, K, 6.0), _spread(rng, N, K, 6.0)
    rows, srows = Q.quantize_mxu(W, fmt)
    q, S, d = F.quantize_mx(x, 32)
    got = mxu.mm(q, S, d, rows, srows, fmt, K).astype(np.float64)
    h = QA.fake_act(x)
    w = QA.fake_w(W, fmt, 128, (rows, srows))
    assert isinstance(w, QA.MXW) and w.mx[1] == QA.WINDOW[fmt]
    want = h @ w.T
    assert isinstance(want, np.ndarray) and not isinstance(want, (QA.MXW, QA.MXAct))
    assert np.array_equal(want, QA.mx_matmul(h, np.asarray(w).view(np.ndarray), w.mx[0], w.mx[1]))
    plain = np.asarray(h).view(np.ndarray) @ np.asarray(w).view(np.ndarray).T
    assert np.abs(got - want).max() < 1e-6 * np.abs(want).max()
    assert np.abs(got - plain).max() > 100 * np.abs(got - want).max()
    r = np.asarray(x[0], np.float64)
    v = w @ r                                                       # w @ h: a plain row, no drops
    v0 = np.asarray(w).view(np.ndarray) @ r
    assert np.abs(v - v0).max() <= 1e-12 * np.abs(v0).max()


def test_device_forms_follow_the_numpy_forms(QA):
    """Tensors in: DeviceMXAct / DeviceMXW, whose h @ w.T equals the numpy forms' bit for bit."""
    import torch
    say("emulation device forms")
    rng = np.random.default_rng(3)
    x, W = _x(rng, 2, 512, 5.0), _spread(rng, 40, 512, 5.0)
    h, w = QA.fake_act(x), QA.fake_w(W, "int4")
    hd, wd = QA.fake_act(torch.from_numpy(x).cuda()), QA.fake_w(torch.from_numpy(W).cuda(), "int4")
    assert isinstance(hd, QA.DeviceMXAct) and isinstance(wd, QA.DeviceMXW)
    assert np.array_equal(hd.values.cpu().numpy(), np.asarray(h).view(np.ndarray))
    y, yd = h @ w.T, hd @ wd.T
    assert isinstance(yd, torch.Tensor) and np.array_equal(yd.cpu().numpy(), y)
