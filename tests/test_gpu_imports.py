"""GPU parity of the checkpoint imports (otpu_import_mxfp4 / otpu_import_nvfp4 through
opentpu_amd.quant) and of the nvfp4 packer (otpu_pack_x4 with OTPU_NVFP4): byte for byte the
oracle's rows and scale rows (the packer also the reference's golden vectors), the same format
choice and the same NotExact refusals."""
import os
import sys

import numpy as np
import pytest

from oracle import formats as Q
from oracle import fp32 as F
from oracle import imports as IM

pytestmark = pytest.mark.gpu
GOLD_NV = os.path.join(os.path.dirname(__file__), "golden", "nv_packer.npz")


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


def _mx(seed, N, K, span=5, top_span=None, dead=True):
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 16, (N, K)).astype(np.uint8)
    if dead:
        codes[N // 2, 64:96] &= 8                              # a sub-block of +-0 only
        codes[N - 1] = rng.integers(0, 2, K).astype(np.uint8) * 8   # a row of +-0
    base = rng.integers(100, 150, (N, 1))
    e = base + rng.integers(0, span + 1, (N, K // 32))
    if top_span is not None:
        e[:, 1] = base[:, 0] + top_span
    return codes, e.astype(np.uint8)


@pytest.mark.parametrize("N,K", [(6, 512), (37, 384), (300, 2816)])
@pytest.mark.parametrize("case", ["fp4", "nvfp4", "forced"])
def test_import_mxfp4(QA, N, K, case):
    say(f"import_mxfp4 {case} N={N} K={K}")
    codes, e = _mx(N + K, N, K, top_span=None if case != "nvfp4" else 17)
    want = "nvfp4" if case == "forced" else None
    r, s, f = QA.import_mxfp4(codes, e, want=want)
    r0, s0, f0 = IM.import_mxfp4(codes, e, want=want)
    assert f == f0 == ("fp4" if case == "fp4" else "nvfp4")
    assert np.array_equal(r, r0) and np.array_equal(s, s0)


def test_import_mxfp4_refusals(QA):
    say("import_mxfp4 refusals")
    codes, e = _mx(1, 8, 256)
    bad = e.copy()
    bad[3, 2] = 0xFF
    with pytest.raises(QA.NotExact, match="NaN"):
        QA.import_mxfp4(codes, bad)
    far = e.copy()
    far[0, 5] = int(e[0].min()) + 23
    with pytest.raises(QA.NotExact, match="span"):
        QA.import_mxfp4(codes, far)
    span = e.copy()
    span[0, 1] = int(e[0].min()) + 9
    with pytest.raises(QA.NotExact, match="5 octaves"):
        QA.import_mxfp4(codes, span, want="fp4")
    with pytest.raises(QA.NotExact, match="normal range"):
        QA.import_mxfp4(codes, np.zeros_like(e))
    with pytest.raises(ValueError):
        QA.import_mxfp4(codes, e[:, :3])


def _nv(seed, N, K):
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 16, (N, K)).astype(np.uint8)
    s = rng.integers(0, 127, (N, K // 16)).astype(np.uint8)
    s[0, :] = rng.integers(1, 8, K // 16)                      # subnormal scales
    s[1, 0] = 0x77
    s[2 % N, :] = 0                                            # a row of zero scales
    s[3 % N, 0], s[3 % N, 1], s[3 % N, 2] = 0x7E, 0x01, 0x03   # 17 octaves down
    return codes, s


@pytest.mark.parametrize("N,K", [(5, 256), (64, 384), (513, 2048)])
def test_import_nvfp4(QA, N, K):
    say(f"import_nvfp4 N={N} K={K}")
    codes, s = _nv(N, N, K)
    ts = np.float32(0.0123)
    r, sr = QA.import_nvfp4(codes, s, ts)
    r0, sr0 = IM.import_nvfp4(codes, s, ts)
    assert np.array_equal(r, r0) and np.array_equal(sr, sr0)


def test_import_nvfp4_every_scale(QA):
    say("import_nvfp4 every scale")
    rng = np.random.default_rng(3)
    codes = rng.integers(0, 16, (127, 128)).astype(np.uint8)
    s = np.zeros((127, 8), np.uint8)
    s[:, 0] = 0x7E
    s[:, 1] = np.arange(127)
    s[:, 2] = np.arange(127)[::-1]
    s[:, 3:] = rng.integers(0, 127, (127, 5))
    r, sr = QA.import_nvfp4(codes, s, 1.0)
    r0, sr0 = IM.import_nvfp4(codes, s, 1.0)
    assert np.array_equal(r, r0) and np.array_equal(sr, sr0)


def test_import_nvfp4_refusals(QA):
    say("import_nvfp4 refusals")
    codes = np.zeros((2, 128), np.uint8)
    s = np.full((2, 8), 0x38, np.uint8)
    for bad, what in ((0x80 | 0x30, "negative"), (0x7F, "NaN")):
        b = s.copy()
        b[1, 1] = bad
        with pytest.raises(QA.NotExact, match=what):
            QA.import_nvfp4(codes, b, 0.5)
    with pytest.raises(QA.NotExact, match="normal range"):
        QA.import_nvfp4(codes, s, 1e-38)


def test_mm_of_imported_fp4_is_the_float64_product(QA):
    """Activations with a 127 in every 32-group (offsets 0) against an imported MXFP4 matrix whose
    exponents stay within MM's window: the MM's words are the float64 product of the checkpoint's
    values, rounded once (to 2e-7 of the largest, as the reference's import check states)."""
    from opentpu_amd import mxu
    say("mm of imported fp4")
    rng = np.random.default_rng(5)
    N, K = 96, 512
    codes, e = _mx(5, N, K, span=3, dead=False)
    rows, srows, fmt = QA.import_mxfp4(codes, e)
    assert fmt == "fp4"
    x = rng.integers(-127, 128, (2, K)).astype(np.float32)
    x[:, ::32] = 127
    q, S, d = F.quantize_mx(x, 32)
    got = mxu.mm(q, S, d, rows, srows, "fp4", K)
    v = np.where(codes & 8, -1.0, 1.0) * Q.E2M1_MAG[codes & 7] * np.exp2(np.repeat(e.astype(np.int64), 32, 1) - 127.0)
    exact = x.astype(np.float64) @ v.T
    assert np.abs(got - exact).max() <= 2e-7 * np.abs(exact).max()


@pytest.mark.parametrize("name", ["c2", "spread", "grid"])
def test_pack_nvfp4_golden(QA, name):
    say(f"pack nvfp4 golden {name}")
    g = np.load(GOLD_NV)
    r, s = QA.quantize_mxu(g[f"{name}_W"], "nvfp4")
    assert np.array_equal(r, g[f"{name}_nvfp4_rows"]) and np.array_equal(s, g[f"{name}_nvfp4_srows"])


def test_pack_nvfp4_vs_oracle(QA):
    say("pack nvfp4 vs oracle")
    rng = np.random.default_rng(4)
    W = (rng.standard_normal((200, 640)) * np.exp(2.0 * rng.standard_normal((200, 40, 1)))
         .repeat(16, 2).reshape(200, 640) * 0.02).astype(np.float32)
    W[7, :128] = 0
    W[9] = 0
    r, s = QA.quantize_mxu(W, "nvfp4")
    r0, s0 = Q.pack_nv(W)
    assert np.array_equal(r, r0) and np.array_equal(s, s0)
