"""The 4-bit prefill GEMM (int4x / fp4x6 / nvfp4 weights, and their RSC / UNIT forms, on the int8
MFMA units: csrc/gemm4.hip) against the C oracle bit for bit: single activation planes (ROW),
several (MX, Horner over the planes), offsets past the window, weight blocks whose offsets spread
(the folded multipliers), nvfp4's per-16-group E4M3 scales (subnormal ones included), tiles the
bounds refuse (the exact VALU path), ACC / ASCALE, k0 column slices, ragged tiles, and the c3
shape at full size (`opentpu/isasim.py:749-910`)."""
import sys

import numpy as np
import pytest

from conftest import same_bits
from oracle import cpu as OC
from oracle import formats as Q
from oracle import fp32 as F
from oracle import mm as MM

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ops():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    from opentpu_amd import _lib, mxu, quant
    _lib.load()
    return quant, mxu


def spread(rng, M, K, s, g):
    return (rng.standard_normal((M, K)) * np.exp(rng.uniform(-s, s, (M, K // g, 1)))
            .repeat(g, 2).reshape(M, K)).astype(np.float32)


def activations(rng, M, K, ak):
    if ak == "row":
        return F.quantize_mx(rng.standard_normal((M, K)).astype(np.float32), 32, row_mode=True)
    if ak == "mx":
        return F.quantize_mx(spread(rng, M, K, 1.0, 32), 32)
    if ak == "wide":                                   # offsets over many binades: past the bound
        return F.quantize_mx(spread(rng, M, K, 7.0, 32), 32)
    dset = np.asarray(ak, np.uint8)                    # a given set of offsets (past the window too)
    q = rng.integers(-127, 128, (M, K)).astype(np.int8)
    Sa = (np.abs(rng.standard_normal(M)) + 0.5).astype(np.float32)
    return q, Sa, dset[rng.integers(0, len(dset), (M, K // 32))]


def weights(rng, N, K, fmt, wk, k0):
    KBr = K // 128 + k0
    s = {"x4": 1.5, "spread": 2.2, "wide": 4.0, "wider": 6.0}.get(wk, 1.5)
    W = (spread(rng, N, KBr * 128, s, 128) * 0.02).astype(np.float32)
    if wk == "tiny":                                   # 16-groups near zero: subnormal E4M3 scales
        g = W.reshape(N, -1, 16)
        g[rng.random(g.shape[:2]) < 0.25] *= np.float32(1e-6)
    rows, srows = Q.quantize_mxu(W, fmt)
    if wk == "rsc":
        srows = np.ascontiguousarray(srows[:, :4])
    elif wk == "unit":
        srows = np.zeros((N, 8), np.uint8)
    rows = np.ascontiguousarray(rows[:, k0 * 64:k0 * 64 + K // 2])
    return rows, srows


CASES = [  # M, N, K, fmt, weights (x4 | spread | wide | rsc | unit), activations, k0
    (512, 384, 2048, "int4", "x4", "row", 0),
    (200, 300, 1024, "int4", "x4", "mx", 0),
    (130, 257, 512, "fp4", "x4", "mx", 0),
    (64, 128, 384, "fp4", "x4", "row", 2),
    (96, 160, 256, "int4", "unit", "mx", 0),
    (72, 136, 640, "fp4", "rsc", "row", 0),         # RSC, five K stages
    (16, 16, 128, "int4", "x4", "row", 0),          # one K stage
    (33, 40, 256, "fp4", "x4", "mx", 0),            # two K stages
    (50, 64, 384, "int4", "spread", "row", 0),      # three K stages, dw spread over the row's blocks
    (100, 200, 4096, "int4", "x4", "mx", 0),
    (48, 130, 6144, "fp4", "spread", "row", 0),
    (16, 8192, 256, "int4", "x4", "row", 0),        # 64 column tiles: the XCD-major order
    (17, 1000, 128, "fp4", "x4", "mx", 0),
    (128, 128, 2048, "int4", "x4", "wide", 0),      # activation offsets past the Horner bound: VALU
    (80, 96, 1024, "fp4", "wide", "row", 0),        # weight offsets past the folding range: VALU
    (200, 256, 1024, "int4", "x4", (0, 1, 2), 0),
    (200, 256, 1024, "fp4", "x4", (0, 20), 0),      # offsets past the window: those groups drop
    (200, 256, 1024, "int4", "x4", (2, 5, 9), 0),   # drops where d + dw > 11
    (64, 96, 512, "int4", "x4", (20, 30), 0),       # every group drops: zero tiles
    # nvfp4: 16-groups with an E4M3 scale each, window 13 (no RSC form)
    (512, 384, 2048, "nvfp4", "x4", "row", 0),
    (200, 300, 1024, "nvfp4", "x4", "mx", 0),
    (64, 128, 384, "nvfp4", "x4", "row", 2),
    (96, 160, 256, "nvfp4", "unit", "mx", 0),
    (16, 16, 128, "nvfp4", "x4", "row", 0),         # one K stage
    (33, 40, 256, "nvfp4", "x4", "mx", 0),          # two K stages
    (50, 64, 384, "nvfp4", "spread", "row", 0),     # three K stages
    (130, 257, 640, "nvfp4", "tiny", "mx", 0),      # subnormal scales: those groups always drop
    (80, 96, 1024, "nvfp4", "wide", "row", 0),
    (80, 96, 1024, "nvfp4", "wider", "row", 0),     # scales past the folding range: VALU
    (128, 128, 2048, "nvfp4", "x4", "wide", 0),     # activation offsets past the Horner bound: VALU
    (200, 256, 1024, "nvfp4", "x4", (0, 20), 0),    # offsets past the window: those groups drop
    (200, 256, 1024, "nvfp4", "x4", (2, 5, 9, 13), 0),   # drops where d + dw > 13
    (16, 8192, 256, "nvfp4", "x4", "row", 0),       # 64 column tiles: the XCD-major order
]


@pytest.mark.parametrize("M,N,K,fmt,wk,ak,k0", CASES)
def test_gemm4(ops, M, N, K, fmt, wk, ak, k0):
    _, mxu = ops
    rng = np.random.default_rng(M + N + K + len(fmt) + len(wk))
    q, Sa, da = activations(rng, M, K, ak)
    rows, srows = weights(rng, N, K, fmt, wk, k0)
    flags = MM.RSC if wk == "rsc" else (MM.UNIT if wk == "unit" else 0)
    say("gemm4", M, N, K, fmt, wk, ak, k0)
    got = mxu.mm(q, Sa, da, rows, srows, fmt, K, rsc=wk == "rsc", unit=wk == "unit", k0=k0)
    want = OC.mm(q, Sa, da, rows, srows, fmt, K, flags=flags, k0=k0)
    assert same_bits(got, want)


@pytest.mark.parametrize("fmt", ["int4", "fp4", "nvfp4"])
def test_gemm4_acc_ascale(ops, fmt):
    _, mxu = ops
    rng = np.random.default_rng(9 + len(fmt))
    M, N, K = 72, 200, 512
    q, Sa, da = activations(rng, M, K, "mx")
    rows, srows = weights(rng, N, K, fmt, "x4", 0)
    old = rng.standard_normal((M, N)).astype(np.float32)
    alpha = rng.standard_normal(M).astype(np.float32)
    say("gemm4 acc / ascale", fmt)
    got = mxu.mm(q, Sa, da, rows, srows, fmt, K, acc=old)
    assert same_bits(got, OC.mm(q, Sa, da, rows, srows, fmt, K, flags=MM.ACC, old=old))
    zs = np.zeros((N, 8), np.uint8)
    got = mxu.mm(q, Sa, da, rows, zs, fmt, K, unit=True, acc=old, alpha=alpha)
    assert same_bits(got, OC.mm(q, Sa, da, rows, zs, fmt, K, flags=MM.UNIT | MM.ACC | MM.ASCALE, old=old,
                                alpha=alpha))


@pytest.mark.parametrize("fmt", ["int4", "fp4", "nvfp4"])
def test_gemm4_c3_full_size(ops, fmt):
    """c3's shape with 4-bit weights: M=512 x K=2048 x N=8192, packed on the GPU from N(0, 0.02),
    ROW and MX activations, every output bit against the C oracle."""
    import torch
    quant, mxu = ops
    M, K, N = 512, 2048, 8192
    gen = torch.Generator(device="cuda").manual_seed(3)
    rows_d, srows_d = quant.quantize_mxu(torch.randn((N, K), generator=gen, device="cuda") * 0.02, fmt)
    rows, srows = rows_d.cpu().numpy(), srows_d.cpu().numpy()
    x = np.random.default_rng(3).standard_normal((M, K)).astype(np.float32)
    for row_mode in (True, False):
        q, Sa, da = F.quantize_mx(x, 32, row_mode=row_mode)
        say("gemm4 c3", fmt, "row" if row_mode else "mx")
        got = mxu.mm(q, Sa, da, rows, srows, fmt, K)
        want = OC.mm(q, Sa, da, rows, srows, fmt, K)
        assert same_bits(got, want)
