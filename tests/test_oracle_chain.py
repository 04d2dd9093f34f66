"""The oracle's chained decode step (oracle/chain.py): the F-chunk rule against the closed form
of opentpu/kernels/mlp.py:8-30 and the chunk sizes it gives at F = 3072; the per-range ACC chain
against one MM over the row where one range covers it, and against independent per-range MMs
added in range order (the ACC semantics of opentpu/isasim.py:899-905: y = add(old, mm))."""
import numpy as np
import pytest

from conftest import same_bits
from oracle import chain as CH
from oracle import formats as Q
from oracle import fp32 as F
from oracle import mm as MM


@pytest.mark.parametrize("f_loc,fmt,want", [
    (3072, "int8", 384), (3072, "int4", 256), (3072, "fp4", 256),
    (256, "int8", 256), (256, "int4", 256), (768, "int4", 256), (1024, "int8", 256),
    (2816, "int8", None), (2944, "int8", 2944), (5120, "int4", None), (640, "int8", None),
])
def test_down_chunk(f_loc, fmt, want):
    """Qwen3-0.6B's F = 3072: int8 chunks of 384 (3 D-blocks), 4-bit chunks of 256 (one 128-byte
    chunk); small F: one chunk; else the largest multiple of q <= F/8 that divides F, >= 2D."""
    c = CH.down_chunk(f_loc, fmt)
    q = 128 if fmt == "int8" else 256
    assert c % q == 0 and f_loc % c == 0
    if want is not None:
        assert c == want
    # brute force over the rule's statement: the first divisor found scanning down from
    # max(2D-ish lower bound, F/8 rounded to q), else up
    lo = min(f_loc, -(-256 // q) * q)
    start = max(lo, (f_loc // 8) // q * q)
    down = [v for v in range(start, lo - 1, -q) if f_loc % v == 0]
    up = [v for v in range(start, f_loc + 1, q) if f_loc % v == 0]
    assert c == (down[0] if down else up[0])


def test_down_chunk_refuses_partial_blocks():
    with pytest.raises(ValueError):
        CH.down_chunk(2880, "int8")          # not whole D-blocks
    with pytest.raises(ValueError):
        CH.down_chunk(1152, "int4")          # not whole 128-byte chunks of 4-bit


def _packed(rng, N, K, fmt):
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    if fmt == "int8":
        return Q.pack_int8x(W)
    return Q.pack_x4(W, fmt)


@pytest.mark.parametrize("fmt", ["int8", "int4", "fp4"])
def test_ranges_dot_one_range_is_linear(fmt):
    rng = np.random.default_rng(11)
    w = _packed(rng, 24, 512, fmt)
    x = rng.standard_normal((2, 512)).astype(np.float32)
    assert same_bits(CH.ranges_dot(x, w, fmt, 512), CH.linear(x, w, fmt))


@pytest.mark.parametrize("fmt,width", [("int8", 128), ("int8", 256), ("int4", 256), ("fp4", 256)])
def test_ranges_dot_is_ordered_acc(fmt, width):
    """The chain equals per-range MMs computed on their own, folded with FTZ adds in order;
    reversing the order changes some bits (so the order is what the test pins)."""
    rng = np.random.default_rng(12)
    K = 1024
    rows, srows = _packed(rng, 40, K, fmt)
    x = (rng.standard_normal((3, K)) * np.exp(rng.uniform(-4, 4, (3, K)))).astype(np.float32)
    bpb = 128 if fmt == "int8" else 64
    parts = []
    for c0 in range(0, K, width):
        q, Sa, da = F.quantize_mx(x[:, c0:c0 + width], 32)
        k0 = c0 // 128
        parts.append(MM.mm(q, Sa, da, rows[:, k0 * bpb:(k0 + width // 128) * bpb], srows, fmt, width, k0=k0))
    y = parts[0]
    for p in parts[1:]:
        y = F.add(y, p)
    assert same_bits(CH.ranges_dot(x, (rows, srows), fmt, width), y)
    yr = parts[-1]
    for p in parts[-2::-1]:
        yr = F.add(yr, p)
    assert not same_bits(y, yr)


def test_layer_small():
    """A small layer's intermediates are the linears of the layer, in the layer's order."""
    rng = np.random.default_rng(13)
    h, qd, kv, Fd = 256, 512, 256, 768
    wts = {"qkv": _packed(rng, qd + 2 * kv, h, "int4"), "o": _packed(rng, h, qd, "int4"),
           "gu": _packed(rng, 2 * Fd, h, "int4"), "down": _packed(rng, h, Fd, "int4")}
    x = rng.standard_normal((1, h)).astype(np.float32)
    y, mid = CH.layer(x, wts, "int4", qd, Fd)
    assert same_bits(mid["qkv"], CH.linear(x, wts["qkv"], "int4"))
    assert same_bits(mid["o"], CH.linear(mid["qkv"][:, :qd], wts["o"], "int4"))
    assert same_bits(mid["h"], F.mul(mid["gu"][:, :Fd], mid["gu"][:, Fd:]))
    assert same_bits(y, CH.ranges_dot(mid["h"], wts["down"], "int4", 256))
    assert np.any(y != 0)
    from oracle import cpu                  # the C MM in the same chain: the same bits
    yc, midc = CH.layer(x, wts, "int4", qd, Fd, mm=cpu.mm)
    assert all(same_bits(midc[k], mid[k]) for k in mid) and same_bits(yc, y)


EMU_TOL = 1e-5       # of the largest output of each linear: the machine's fp32 chain vs float64


def test_emulated_layer_separates_quantization_from_rounding():
    """The float64 layer with the quantization points (emulated_layer, the structure of the
    reference's emulated_logits) is within EMU_TOL of the machine's fp32 layer at every linear;
    the same product without the quantization points, and the machine's layer with a wrong
    F-chunking of the down input, are hundreds of times further."""
    from oracle import emulate as EM
    rng = np.random.default_rng(1)
    h, qd, kv, Fd = 256, 512, 256, 768

    def pack(n, k):
        return Q.quantize_mxu((rng.standard_normal((n, k)) * 0.05).astype(np.float32), "int4")
    wts = {"qkv": pack(qd + 2 * kv, h), "o": pack(h, qd), "gu": pack(2 * Fd, h), "down": pack(h, Fd)}
    for _ in range(3):
        x = rng.standard_normal((1, h)).astype(np.float32)
        y, mid = CH.layer(x, wts, "int4", qd, Fd)
        ye, me = CH.emulated_layer(x, wts, "int4", qd, Fd)
        for k in ("qkv", "o", "gu", "down"):
            assert np.abs(np.asarray(mid[k], np.float64) - me[k]).max() <= EMU_TOL * np.abs(me[k]).max(), k

        def plain(xx, w):
            return xx @ EM.fake_w(w[0], w[1], "int4", xx.shape[1])[0].T
        xf = x.astype(np.float64)
        qkv = plain(xf, wts["qkv"])
        gu = plain(plain(qkv[:, :qd], wts["o"]), wts["gu"])
        yp = plain(gu[:, :Fd] * gu[:, Fd:], wts["down"])
        assert np.abs(yp - ye).max() > 100 * EMU_TOL * np.abs(ye).max()
        yb = CH.ranges_dot(mid["h"], wts["down"], "int4", 768)
        assert np.abs(yb - ye).max() > 100 * EMU_TOL * np.abs(ye).max()
