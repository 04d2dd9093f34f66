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
    say(f"fake_act M={M} K={K} n={n} row={row} g={g}")
    rng = np.random.default_rng(K + M)
    x = _x(rng, M, K, 4.0)
    x[0, :64] = (np.arange(64) % 50 + 0.5).astype(np.float32) * np.float32(x[0].max() / 127)   # near-ties
    x[-1, 5] = 1e-40                                                # a denormal
    a = QA.fake_act(x, n=n, row=row, g=g)
    v0, da0 = EM.fake_act(x, n=n, row=row, g=g)
    assert np.array_equal(a.values.cpu().numpy().view(np.uint64), v0.view(np.uint64))
    assert np.array_equal(a.da.cpu().numpy(), da0)


def test_fake_act_exact_ties(QA):
    say("fake_act exact ties")
    x = np.zeros((1, 64), np.float32)
    x[0, 0] = 127.0
    x[0, 1:] = (np.arange(1, 64) % 100 + 0.5).astype(np.float32)
    a = QA.fake_act(x, row=True)
    assert np.array_equal(a.values.cpu().numpy()[0], F.quantize_mx(x, 32, row_mode=True)[0][0].astype(np.float64))


@pytest.mark.parametrize("fmt,rsc", [("int8", False), ("int8", True), ("int4", False), ("fp4", False),
                                     ("nvfp4", False)])
def test_dequant(QA, fmt, rsc):
    say(f"dequant {fmt} rsc={rsc}")
    rng = np.random.default_rng(7)
    W = _spread(rng, 40, 640, 4.0)
    rows, srows = Q.pack_rsc(W) if rsc else Q.quantize_mxu(W, fmt)
    srows = srows.copy()
    srows[3, :4] = np.array([1e-40], np.float32).view(np.uint8)     # a denormal Sw reads 0
    v, dw = QA.dequantize_mxu(rows, srows, fmt, 640, rsc=rsc)
    v0, dw0 = EM.fake_w(rows, srows, fmt, 640, rsc=rsc)
    assert np.array_equal(v.cpu().numpy().view(np.uint64), v0.view(np.uint64))
    assert np.array_equal(dw.cpu().numpy(), dw0)


@pytest.mark.parametrize("M,N,K,W,mode", [(3, 24, 1024, 16, "both"), (7, 100, 512, 11, "both"),
                                          (2, 33, 256, 13, "one_dw"), (4, 17, 384, 16, "no_da")])
def test_mx_matmul(QA, M, N, K, W, mode):
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
        y = QA.mx_matmul(QA.MXAct(QA.X.dev(h, np.float64), QA.X.dev(da, np.uint8)), w, dw, W)
        want = EM.mx_matmul(h, w, da, dw, W)
    y = y.cpu().numpy()
    assert np.abs(y - want).max() <= 1e-12 * np.abs(want).max()


@pytest.mark.parametrize("fmt", Q.FMTS)
def test_mm_follows_the_emulation(QA, fmt):
    from opentpu_amd import mxu
    say(f"mm vs emulation {fmt}")
    rng = np.random.default_rng(1)
    M, N, K = 3, 24, 8 * D
    x, W = _x(rng, M, K, 6.0), _spread(rng, N, K, 6.0)
    rows, srows = Q.quantize_mxu(W, fmt)
    q, S, d = F.quantize_mx(x, 32)
    got = mxu.mm(q, S, d, rows, srows, fmt, K).astype(np.float64)
    h = QA.fake_act(x)
    w = QA.fake_w(W, fmt, quantized=(rows, srows))
    want = QA.mx_matmul(h, w).cpu().numpy()
    plain = QA.mx_matmul(h.values, w.values).cpu().numpy()
    assert np.abs(got - want).max() < 1e-6 * np.abs(want).max()
    assert np.abs(got - plain).max() > 100 * np.abs(got - want).max()
