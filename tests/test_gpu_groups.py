"""GPU parity of the grouped-image converters (otpu_ungroup_rows / otpu_ungroup_scales through
opentpu_amd.quant.ungrouped): a weight image in the reference machine's grouped layout (with and
without the channel hash) made by the oracle from natural rows comes back as those rows, byte for
byte, and an MM over the converted image is the MM over the natural rows bit for bit."""
import sys

import numpy as np
import pytest

from conftest import same_bits
from oracle import formats as Q
from oracle import groups as G
from oracle import fp32 as F
from oracle import mm as MM

pytestmark = pytest.mark.gpu
D = G.D


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def X():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    from opentpu_amd import _lib
    _lib.load()
    return _lib


def _image(rng, N, K, fmt, rsc=False):
    if fmt == "int8":
        rows = rng.integers(0, 256, (N, K)).astype(np.uint8)
    else:
        rows = np.zeros((N, Q.row_bytes(K, fmt)), np.uint8)
        rows[:, :K // 2] = Q.pack_nibbles(rng.integers(0, 16, (N, K)))
    srows = np.zeros((N, Q.scale_bytes(K, fmt, rsc)), np.uint8)
    srows[:, :4] = rng.integers(0, 256, (N, 4))
    if not rsc:
        h, sb = G.swp(fmt, 1), G.SCALE_DATA[fmt]
        srows[:, h:h + (K // D) * sb] = rng.integers(0, 256, (N, (K // D) * sb))
    return rows, srows


@pytest.mark.parametrize("fmt", ["int8", "int4", "fp4", "nvfp4"])
@pytest.mark.parametrize("wg", [1, 2, 8, 16, 64])
@pytest.mark.parametrize("hashed", [False, True])
@pytest.mark.parametrize("N,KB", [(13, 3), (100, 5), (7, 1)])
def test_ungroup_round_trip(X, fmt, wg, hashed, N, KB):
    from opentpu_amd import quant as QA
    say(f"ungroup fmt={fmt} wg={wg} hashed={hashed} N={N} KB={KB}")
    rng = np.random.default_rng(wg * 100 + N + KB)
    K = KB * D
    rows, srows = _image(rng, N, K, fmt)
    g, a = G.group_rows(rows, N, K, fmt, wg), G.group_scales(srows, N, K, fmt, wg)
    at = 37 * wg * D if hashed else None
    if hashed:
        g = G.hash_rows(g, at, wg)
    r2, s2 = QA.ungrouped(g, a, N, K, wg, fmt, at=at)
    assert np.array_equal(r2, rows)
    assert np.array_equal(s2, srows)


@pytest.mark.parametrize("fmt", ["int8", "int4", "fp4"])
@pytest.mark.parametrize("wg", [2, 8])
def test_ungroup_rsc_scales(X, fmt, wg):
    from opentpu_amd import quant as QA
    say(f"ungroup rsc fmt={fmt} wg={wg}")
    rng = np.random.default_rng(wg)
    N, K = 37, 4 * D
    _, srows = _image(rng, N, K, fmt, rsc=True)
    a = G.group_scales(srows, N, K, fmt, wg, rsc=True)
    assert np.array_equal(QA.ungroup_scales(a, N, K, wg, fmt, rsc=True), srows)


@pytest.mark.parametrize("fmt", ["int8", "int4", "fp4"])
def test_mm_over_a_grouped_image(X, fmt):
    """quantize_mxu's rows grouped at WG 8 and hashed at an address, converted on the GPU: the
    MM's words equal the oracle MM's over the natural rows."""
    from opentpu_amd import mxu, quant as QA
    say(f"mm over grouped fmt={fmt}")
    rng = np.random.default_rng(11)
    M, N, K, wg = 3, 200, 640, 8
    W = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    rows, srows = Q.quantize_mxu(W, fmt)
    x = rng.standard_normal((M, K)).astype(np.float32)
    q, S, d = F.quantize_mx(x, 32)
    at = 5 * wg * D
    g = G.hash_rows(G.group_rows(rows, N, K, fmt, wg), at, wg)
    a = G.group_scales(srows, N, K, fmt, wg)
    r2, s2 = QA.ungrouped(g, a, N, K, wg, fmt, at=at)
    got = mxu.mm(q, S, d, r2, s2, fmt, K)
    want = MM.mm(q, S, d, rows, srows, fmt, K)
    assert same_bits(got, want)


@pytest.mark.parametrize("fmt", ["int8", "int4", "fp4"])
@pytest.mark.parametrize("wg,hashed", [(2, False), (8, True), (16, False)])
@pytest.mark.parametrize("groups,KB", [(1, 1), (2, 5), (3, 2), (4, 23)])
def test_ungroup_kt_pairs(X, fmt, wg, hashed, groups, KB):
    """An image in MM KT's pairs (the oracle's kt_rows / kt_scales of a grouped image whose K ends
    in the first half of its last block) comes back as the padded natural rows byte for byte; its
    scale rows equal the natural ones wherever they meet data; the MM over it is the padded MM
    bit for bit (the reference's tests/test_kt.py:94-113 property)."""
    from opentpu_amd import mxu, quant as QA
    from test_oracle_kt import kt_operand
    say(f"ungroup kt fmt={fmt} wg={wg} hashed={hashed} groups={groups} KB={KB}")
    rng = np.random.default_rng(wg * 10 + groups * 100 + KB)
    R = G.grp_r(fmt, wg)
    N = groups * R - (3 if groups == 3 else 0)
    K = KB * D
    rows, srows = kt_operand(rng, fmt, N, KB)
    g = G.kt_rows(G.group_rows(rows, N, K, fmt, wg), wg)
    a = G.kt_scales(G.group_scales(srows, N, K, fmt, wg), fmt, K, wg)
    at = 11 * wg * D if hashed else None
    if hashed:
        g = G.hash_rows(g, at, wg)
    r2, s2 = QA.ungrouped(g, a, N, K, wg, fmt, at=at, kt=True)
    assert np.array_equal(r2, rows)
    assert np.array_equal(s2, G.ungroup_kt_scales(a, N, K, fmt, wg))
    x = rng.standard_normal((3, K)).astype(np.float32)
    x[:, K - D // 2:] = 0                                         # K ends in the tail block's first half
    q, S, d = F.quantize_mx(x, 32)
    assert same_bits(mxu.mm(q, S, d, r2, s2, fmt, K), MM.mm(q, S, d, rows, srows, fmt, K))


def test_ungroup_lm_head_shape(X):
    """An LM-head-sized int4 image (N 8192 of K 2560, WG 8, hashed): byte for byte."""
    from opentpu_amd import quant as QA
    say("ungroup lm-head shape")
    rng = np.random.default_rng(2)
    N, K, wg, fmt = 8192, 2560, 8, "int4"
    rows, srows = _image(rng, N, K, fmt)
    at = 1 << 30
    g = G.hash_rows(G.group_rows(rows, N, K, fmt, wg), at, wg)
    a = G.group_scales(srows, N, K, fmt, wg)
    r2, s2 = QA.ungrouped(g, a, N, K, wg, fmt, at=at)
    assert np.array_equal(r2, rows) and np.array_equal(s2, srows)


def test_ungroup_refusals(X):
    import torch
    from opentpu_amd import quant as QA
    say("ungroup refusals")
    N, K = 16, 256
    d = torch.zeros((2, K * 8), dtype=torch.uint8, device="cuda")
    out = torch.zeros((N, K), dtype=torch.uint8, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    with pytest.raises(X.OtpuError, match="power of two"):
        X.call("otpu_ungroup_rows", X.ptr(d), N, K, 3, 0, 0, -1, X.ptr(out), K, s)
    with pytest.raises(X.OtpuError, match="not a multiple"):
        X.call("otpu_ungroup_rows", X.ptr(d), N, K, 8, 0, 0, 128, X.ptr(out), K, s)
    with pytest.raises(X.OtpuError, match="need"):
        X.call("otpu_ungroup_rows", X.ptr(d), N, K, 8, 0, 0, -1, X.ptr(out), 128, s)
    with pytest.raises(X.OtpuError):
        X.call("otpu_ungroup_rows", X.ptr(d), N, K, 8, 7, 0, -1, X.ptr(out), K, s)
    with pytest.raises(X.OtpuError, match="NVFP4"):
        X.call("otpu_ungroup_scales", X.ptr(d), N, K, 8, 3, 1, 0, X.ptr(out), K, s)
    with pytest.raises(X.OtpuError, match="KT"):
        X.call("otpu_ungroup_rows", X.ptr(d), N, K, 1, 0, 1, -1, X.ptr(out), K, s)
    with pytest.raises(X.OtpuError, match="KT"):
        X.call("otpu_ungroup_scales", X.ptr(d), N, K, 8, 3, 0, 1, X.ptr(out), K, s)
    with pytest.raises(ValueError, match="image"):
        QA.ungroup_rows(d[:, :100], N, K, 8, "int8")
