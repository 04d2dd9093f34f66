"""GPU parity: the HIP kernels through the C ABI (opentpu_amd) against the CPU oracle on the
same seeded inputs, bit for bit (int8 operands, int64 accumulators, fp32 outputs, tokens)."""
import os
import sys

import numpy as np
import pytest

from conftest import same_bits
from oracle import cpu as OC
from oracle import formats as Q
from oracle import fp32 as F
from oracle import mm as MM
from test_oracle_mm import CASES, mm_case

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(__file__), "golden", "x4_packer.npz")


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ops():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    from opentpu_amd import _lib, fp32, mxu, quant
    _lib.load()
    return fp32, quant, mxu


def spread(rng, M, K, s=6.0, g=8):
    return (rng.standard_normal((M, K)) * np.exp(rng.uniform(-s, s, (M, K // g, 1)))
            .repeat(g, 2).reshape(M, K)).astype(np.float32)


@pytest.mark.parametrize("g,row_mode", [(32, False), (32, True), (128, False), (8, False), (64, False)])
def test_qact(ops, g, row_mode):
    fp32, _, _ = ops
    rng = np.random.default_rng(g + row_mode)
    x = spread(rng, 9, 2560)
    x[1] = 0
    x[2, 5] = np.float32(1e-41)
    x[3, :] = rng.standard_normal(2560).astype(np.float32) * 1e-37   # mostly denormal: flushes
    x[4, 7] = np.inf
    say("qact", g, row_mode)
    q, S, d = fp32.quantize_mx(x, g, row_mode)
    q0, S0, d0 = F.quantize_mx(x, g, row_mode)
    assert np.array_equal(q, q0) and same_bits(S, S0) and np.array_equal(d, d0)


def test_qact_recip_every_significand(ops):
    """One row per significand pattern sweep: amax = each value, so S and the quantized
    values exercise recip over [1, 2) times many exponents."""
    fp32, _, _ = ops
    rng = np.random.default_rng(3)
    amax = F.from_bits(rng.integers(0x00800000, 0x7E000000, 4096).astype(np.uint32))
    x = (rng.uniform(-1, 1, (4096, 128)) * amax[:, None]).astype(np.float32)
    x[:, 0] = amax
    say("qact recip sweep")
    q, S, d = fp32.quantize_mx(x, 32)
    q0, S0, d0 = F.quantize_mx(x, 32)
    assert np.array_equal(q, q0) and same_bits(S, S0) and np.array_equal(d, d0)


@pytest.mark.parametrize("fmt,unit,rsc,k0,big", CASES)
@pytest.mark.parametrize("KB", [1, 3, 8])
def test_mm_cases(ops, fmt, unit, rsc, k0, big, KB):
    _, _, mxu = ops
    for M in (1, 3, 5):
        c = mm_case(fmt, unit, rsc, k0, big, KB, M=M, N=37)
        flags = (MM.UNIT if unit else 0) | (MM.RSC if rsc else 0)
        say("mm", fmt, unit, rsc, k0, big, KB, M)
        want_acc, _ = MM.mm_acc(c["q"], c["da"], c["rows"], c["srows"], fmt, c["K"], flags=flags, k0=k0)
        want = MM.mm(c["q"], c["Sa"], c["da"], c["rows"], c["srows"], fmt, c["K"], flags=flags, k0=k0)
        got = mxu.mm(c["q"], c["Sa"], c["da"], c["rows"], c["srows"], fmt, c["K"], rsc=rsc, unit=unit, k0=k0)
        acc = mxu.mm_acc(c["q"], c["da"], c["rows"], c["srows"], fmt, c["K"], rsc=rsc, unit=unit, k0=k0)
        assert np.array_equal(acc, want_acc)
        assert same_bits(got, want)


def test_mm_flags(ops):
    _, _, mxu = ops
    rng = np.random.default_rng(6)
    c = mm_case("int8", True, False, 0, False, 4, M=3, N=300)
    old = rng.standard_normal((3, 300)).astype(np.float32)
    alpha = rng.standard_normal(3).astype(np.float32)
    a = (c["q"], c["Sa"], c["da"], c["rows"], c["srows"], "int8", c["K"])
    say("mm flags")
    assert same_bits(mxu.mm(*a, unit=True, acc=old), MM.mm(*a, flags=MM.UNIT | MM.ACC, old=old))
    assert same_bits(mxu.mm(*a, unit=True, acc=old, alpha=alpha),
                     MM.mm(*a, flags=MM.UNIT | MM.ACC | MM.ASCALE, old=old, alpha=alpha))
    y, mx = mxu.mm(*a, unit=True, rmax=True)
    y0, mx0 = MM.mm(*a, flags=MM.UNIT | MM.RMAX)
    assert same_bits(y, y0) and same_bits(mx, mx0)


def test_mm_refuses_what_the_reference_refuses(ops):
    from opentpu_amd._lib import OtpuError
    _, _, mxu = ops
    c = mm_case("nvfp4", False, False, 0, False, 1)
    with pytest.raises(OtpuError):            # RSC does not take NVFP4
        mxu.mm(c["q"], c["Sa"], c["da"], c["rows"], c["srows"], "nvfp4", c["K"], rsc=True)
    c = mm_case("int8", False, False, 0, False, 1)
    with pytest.raises(OtpuError):            # ASCALE needs UNIT and ACC
        mxu.mm(c["q"], c["Sa"], c["da"], c["rows"], c["srows"], "int8", c["K"],
               acc=np.zeros((3, 5), np.float32), alpha=np.ones(3, np.float32))
    with pytest.raises(OtpuError):            # scale rows too short for k0
        mxu.mm(c["q"], c["Sa"], c["da"], c["rows"], c["srows"], "int8", c["K"], k0=9)


def test_packers(ops):
    _, quant, _ = ops
    rng = np.random.default_rng(2)
    W = spread(rng, 64, 1152, 3.0, 32) * np.float32(0.02)
    W[3, 128:256] = 0
    W[5] = 0
    say("pack int8")
    r, s = quant.quantize_mxu(W, "int8")
    r0, s0 = Q.pack_int8x(W)
    assert np.array_equal(r, r0) and np.array_equal(s, s0)
    r, s = quant.quantize_mxu(W, "int8", rsc=True)
    r0, s0 = Q.pack_rsc(W)
    assert np.array_equal(r, r0) and np.array_equal(s, s0)
    g = np.load(GOLD)
    for name in ("c2", "spread", "grid"):
        for fmt in ("int4", "fp4"):
            say("pack", name, fmt)
            r, s = quant.quantize_mxu(g[f"{name}_W"], fmt)
            assert np.array_equal(r, g[f"{name}_{fmt}_rows"]), (name, fmt)
            assert np.array_equal(s, g[f"{name}_{fmt}_srows"]), (name, fmt)
    for fmt in ("int4", "fp4"):
        Wb = spread(rng, 256, 640, 2.0, 32)
        say("pack vs oracle", fmt)
        r, s = quant.quantize_mxu(Wb, fmt)
        r0, s0 = Q.pack_x4(Wb, fmt)
        assert np.array_equal(r, r0) and np.array_equal(s, s0)


def _config_weights(seed, N, K, fmt, rsc=False):
    rng = np.random.default_rng(seed)
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    x = rng.standard_normal((1, K)).astype(np.float32)
    if fmt == "int8":
        rows, srows = Q.pack_rsc(W) if rsc else Q.pack_int8x(W)
    else:
        rows, srows = Q.pack_x4(W, fmt)
    return W, x, rows, srows


@pytest.mark.parametrize("name,N,K,fmt,rsc", [("c1 RSC", 4096, 1024, "int8", True),
                                              ("c1 int8x", 4096, 1024, "int8", False),
                                              ("c2 int4x", 6144, 2048, "int4", False)])
def test_configs_full_size(ops, name, N, K, fmt, rsc):
    _, _, mxu = ops
    W, x, rows, srows = _config_weights(1, N, K, fmt, rsc)
    q, Sa, da = F.quantize_mx(x, 32)
    say("config", name)
    got = mxu.mm(q, Sa, da, rows, srows, fmt, K, rsc=rsc)
    want = OC.mm(q, Sa, da, rows, srows, fmt, K, flags=MM.RSC if rsc else 0)
    assert same_bits(got, want)
    # the float64 product of the dequantized operands (no group drops at these scales)
    xa = (q.astype(np.float64).reshape(1, -1, 32) * np.exp2(-da.astype(np.float64))[..., None]
          ).reshape(1, -1) * np.float64(Sa[0])
    ref = xa @ Q.dequantize(rows, srows, fmt, K, rsc=rsc).T
    assert np.abs(got - ref).max() < 1e-5 * np.abs(ref).max()


def test_lm_head_argmax_full_size(ops):
    import torch
    _, quant, mxu = ops
    N, K = 262144, 2560
    gen = torch.Generator(device="cuda").manual_seed(5)
    W = torch.randn((N, K), generator=gen, device="cuda") * 0.02
    say("lm head c5: pack")
    rows_d, srows_d = quant.quantize_mxu(W, "int8", rsc=True)
    del W
    rows, srows = rows_d.cpu().numpy(), srows_d.cpu().numpy()
    x = np.random.default_rng(5).standard_normal((1, K)).astype(np.float32)
    q, Sa, da = F.quantize_mx(x, 32)
    say("lm head c5")
    tok, logits, best = mxu.lm_head_argmax(q, Sa, da, rows, srows, "int8", K, rsc=True)
    want = OC.mm(q, Sa, da, rows, srows, "int8", K, flags=MM.RSC)[0]
    assert same_bits(logits, want)
    t0, b0 = OC.argmax(want)
    assert tok == t0 == MM.greedy(want) and best == b0


def test_lm_head_ties_go_to_the_lowest_index(ops):
    _, _, mxu = ops
    rng = np.random.default_rng(7)
    N, K = 5000, 256
    rows = rng.integers(-127, 128, (N, K)).astype(np.int8)
    rows[4321] = 127
    rows[77] = 127                                   # the same logit, earlier
    rows[4999] = 127
    srows = np.full((N, 1), 0.01, np.float32).view(np.uint8)
    x = np.abs(rng.standard_normal((1, K))).astype(np.float32)
    q, Sa, da = F.quantize_mx(x, 32)
    say("lm head ties")
    tok, logits, best = mxu.lm_head_argmax(q, Sa, da, rows.view(np.uint8), srows, "int8", K, rsc=True, base=1000)
    assert tok == 1077 and MM.greedy(logits) == 77


def test_argmax_vop(ops):
    _, _, mxu = ops
    rng = np.random.default_rng(0)
    a = rng.standard_normal((5, 300)).astype(np.float32)
    a[1, [7, 40, 299]] = 9.0
    a[2] = -np.inf
    a[2, 250] = -1e30
    a[3, :] = 0.0
    a[3, 100] = -0.0
    a[4, :] = -1.0
    a[4, 5], a[4, 9] = 1e-41, 0.0
    say("argmax vop")
    v, idx = mxu.argmax(a)
    v0, i0 = MM.argmax(a)
    assert list(idx) == list(i0) == [int(np.argmax(a[0])), 7, 250, 0, 5]
    assert same_bits(v, v0)


def test_dot_ranges_accumulate_in_order(ops):
    """Two QACT ranges -> two MMs, the second ACC (compiler.py:2686-2720), as the oracle."""
    _, _, mxu = ops
    rng = np.random.default_rng(5)
    M, N, K = 2, 160, 512
    x = spread(rng, M, K, 2.0)
    x[:, 256:] *= 300.0
    for fmt in ("int8", "int4"):
        W = (spread(rng, N, K, 2.0) * 0.02).astype(np.float32)
        rows, srows = Q.pack_int8x(W) if fmt == "int8" else Q.pack_x4(W, fmt)
        w = mxu.QWeight.from_packed(rows, srows, fmt, K)
        say("dot ranges", fmt)
        got = mxu.dot(x, w, ranges=[256, 256])
        want = None
        for c0 in (0, 256):
            q, Sa, da = F.quantize_mx(x[:, c0:c0 + 256], 32)
            part = MM.mm(q, Sa, da, rows[:, (c0 if fmt == "int8" else c0 // 2):], srows, fmt, 256,
                         flags=0 if want is None else MM.ACC, k0=c0 // 128, old=want)
            want = part
        assert same_bits(np.asarray(got), want)


def test_batched_is_independent_mms(ops):
    import torch
    _, _, mxu = ops
    from opentpu_amd import _lib as X
    rng = np.random.default_rng(8)
    B, N, K = 5, 96, 1024
    qs, Sas, das, rs, ss, want = [], [], [], [], [], []
    for b in range(B):
        W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        x = rng.standard_normal((1, K)).astype(np.float32)
        r, s = Q.pack_x4(W, "int4")
        q, Sa, da = F.quantize_mx(x, 32)
        qs.append(q); Sas.append(Sa); das.append(da); rs.append(r); ss.append(s)
        want.append(MM.mm(q, Sa, da, r, s, "int4", K))
    qd = torch.from_numpy(np.concatenate(qs)).cuda()
    Sad = torch.from_numpy(np.concatenate(Sas)).cuda()
    dad = torch.from_numpy(np.concatenate(das)).cuda()
    rd = torch.from_numpy(np.concatenate(rs)).cuda()
    sd = torch.from_numpy(np.concatenate(ss)).cuda()
    out = torch.empty((B, 1, N), dtype=torch.float32, device="cuda")
    say("batched")
    X.call("otpu_mm_batched", B, X.ptr(qd), K, K, X.ptr(Sad), 1, X.ptr(dad), K // 32, K // 32, 1, K,
           X.ptr(rd), rd.shape[1], N * rd.shape[1], X.ptr(sd), sd.shape[1], N * sd.shape[1], N, X.FMT["int4"],
           0, 0, X.ptr(out), N, N, X.stream())
    got = out.cpu().numpy()
    for b in range(B):
        assert same_bits(got[b], want[b])


@pytest.mark.parametrize("fmt,rsc,K", [("int8", True, 1024), ("int8", False, 1024), ("int4", False, 1024),
                                       ("fp4", False, 1024), ("int4", False, 2048), ("fp4", False, 2048),
                                       ("nvfp4", False, 2048)])
def test_gemv_row_blocking_paths(ops, fmt, rsc, K):
    """One launch of 32 problems (a grid over every CU: 8 rows a team) and the same problems
    one launch each (a small grid: 4 rows a team), both against the C oracle.  K 2048 4-bit is
    the timed headline's kernel: a team of 64 lanes, one piece a lane, 8 rows a team."""
    import torch
    _, _, mxu = ops
    from opentpu_amd import _lib as X
    rng = np.random.default_rng(31 + len(fmt) + rsc + K)
    B, N = 32, 512
    qs, Sas, das, rs, ss, want = [], [], [], [], [], []
    flags = MM.RSC if rsc else 0
    for b in range(B):
        W = (spread(rng, N, K, 1.5, 128) * 0.02).astype(np.float32)
        x = spread(rng, 1, K, 2.0, 32)
        if fmt == "int8":
            r, sr = Q.pack_rsc(W) if rsc else Q.pack_int8x(W)
        else:
            r, sr = Q.quantize_mxu(W, fmt)
        q, Sa, da = F.quantize_mx(x, 32)
        qs.append(q); Sas.append(Sa); das.append(da); rs.append(r); ss.append(sr)
        want.append(OC.mm(q, Sa, da, r, sr, fmt, K, flags=flags))
    qd = torch.from_numpy(np.concatenate(qs)).cuda()
    Sad = torch.from_numpy(np.concatenate(Sas)).cuda()
    dad = torch.from_numpy(np.concatenate(das)).cuda()
    rd = torch.from_numpy(np.concatenate(rs)).cuda()
    sd = torch.from_numpy(np.concatenate(ss)).cuda()
    out = torch.empty((B, 1, N), dtype=torch.float32, device="cuda")
    say("gemv row blocking", fmt, rsc)
    X.call("otpu_mm_batched", B, X.ptr(qd), K, K, X.ptr(Sad), 1, X.ptr(dad), K // 32, K // 32, 1, K,
           X.ptr(rd), rd.shape[1], N * rd.shape[1], X.ptr(sd), sd.shape[1], N * sd.shape[1], N, X.FMT[fmt],
           flags, 0, X.ptr(out), N, N, X.stream())
    got = out.cpu().numpy()
    for b in range(B):
        assert same_bits(got[b], want[b])
        one = mxu.mm(qs[b], Sas[b], das[b], rs[b], ss[b], fmt, K, rsc=rsc)
        assert same_bits(one, want[b])


@pytest.mark.parametrize("fmt,K,rsc", [("int8", 4096, False), ("int8", 2560, True), ("int4", 8192, False),
                                       ("fp4", 8192, False)])
def test_gemv_four_or_more_pieces_a_lane(ops, fmt, K, rsc):
    """Rows of 4 or more 16-byte pieces a lane (the LM head's shape class), 1 to 4 activation
    rows a launch (the register tiling's MR 1, 2 and 4), against the C oracle."""
    _, _, mxu = ops
    rng = np.random.default_rng(K + len(fmt) + rsc)
    N = 300
    W = (spread(rng, N, K, 1.5, 128) * 0.02).astype(np.float32)
    if fmt == "int8":
        rows, srows = Q.pack_rsc(W) if rsc else Q.pack_int8x(W)
    else:
        rows, srows = Q.quantize_mxu(W, fmt)
    for M in (1, 2, 3, 4):
        x = spread(rng, M, K, 2.0, 32)
        q, Sa, da = F.quantize_mx(x, 32)
        say("gemv many pieces", fmt, K, rsc, M)
        got = mxu.mm(q, Sa, da, rows, srows, fmt, K, rsc=rsc)
        want = OC.mm(q, Sa, da, rows, srows, fmt, K, flags=MM.RSC if rsc else 0)
        assert same_bits(got, want)


def test_headline_batched_c2_full_size(ops):
    """The bench's timed headline launch itself: 80 independent c2 GEMVs (int4x N=6144 K=2048,
    weights N(0, 0.02) packed on the GPU, MX activations of N(0, 1) rows) in one otpu_mm_batched
    (a team of 64 lanes, one piece a lane, 8 rows a team), every output bit against the C
    oracle."""
    import torch
    _, quant, _ = ops
    from opentpu_amd import _lib as X
    from opentpu_amd import fp32 as GF
    B, N, K = 80, 6144, 2048
    gen = torch.Generator(device="cuda").manual_seed(2)
    rows = torch.empty((B, N, 1024), dtype=torch.uint8, device="cuda")
    srows = torch.empty((B, N, 72), dtype=torch.uint8, device="cuda")
    say("headline c2 x 80: pack")
    for b in range(B):
        W = torch.randn((N, K), generator=gen, device="cuda") * 0.02
        r, sr = quant.quantize_mxu(W, "int4")
        rows[b].copy_(r)
        srows[b].copy_(sr)
    x = torch.randn((B, K), generator=gen, device="cuda")
    q, Sa, da = GF.quantize_mx(x, 32)
    out = torch.empty((B, N), dtype=torch.float32, device="cuda")
    say("headline c2 x 80: run")
    X.call("otpu_mm_batched", B, X.ptr(q), K, K, X.ptr(Sa), 1, X.ptr(da), K // 32, K // 32, 1, K, X.ptr(rows), 1024,
           N * 1024, X.ptr(srows), 72, N * 72, N, X.FMT["int4"], 0, 0, X.ptr(out), N, N, X.stream())
    got = out.cpu().numpy()
    qh, Sh, dh = q.cpu().numpy(), Sa.cpu().numpy(), da.cpu().numpy()
    q0, S0, d0 = F.quantize_mx(x.cpu().numpy(), 32)
    assert np.array_equal(qh, q0) and same_bits(Sh, S0) and np.array_equal(dh, d0)
    rh, sh = rows.cpu().numpy(), srows.cpu().numpy()
    say("headline c2 x 80: oracle")
    for b in range(B):
        want = OC.mm(qh[b:b + 1], Sh[b:b + 1], dh[b:b + 1], rh[b], sh[b], "int4", K)
        assert same_bits(got[b:b + 1], want), f"problem {b}"


GEMM_CASES = [  # M, N, K, weights (rsc | int8x | unit), activations (row | mx | wide), k0
    (512, 384, 2048, "rsc", "row", 0),
    (200, 300, 1024, "rsc", "mx", 0),
    (130, 257, 512, "int8x", "mx", 0),
    (64, 128, 384, "int8x", "row", 2),
    (96, 160, 256, "unit", "mx", 0),
    (128, 128, 2048, "rsc", "wide", 0),      # offsets over > 6 binades: the VALU tiles
    (40, 70, 640, "int8x", "wide", 1),       # drops (d + e > 16) inside the planes
    (200, 300, 1024, "rsc", "row", 0),       # single plane, ragged tiles
    (72, 136, 640, "unit", "row", 0),        # single plane, an odd number of K stages
    (16, 16, 128, "rsc", "row", 0),          # single plane, one K stage
    (100, 200, 4096, "rsc", "mx", 0),        # 32 K stages, up to 5 offsets a tile: masked passes
    (64, 200, 8192, "rsc", "mx", 0),         # 64 K stages (the loaders count the passes' barriers)
    (300, 96, 4224, "int8x", "mx", 1),       # 33 K stages, weight planes, k0
    (48, 130, 6144, "rsc", "row", 0),        # single plane, a long ring walk
    (16, 8192, 256, "rsc", "row", 0),        # 64 column tiles: the XCD-major tile order
    (17, 1000, 128, "unit", "mx", 0),        # one row past a tile, a ragged last column tile
]


@pytest.mark.parametrize("M,N,K,wk,ak,k0", GEMM_CASES)
def test_gemm(ops, M, N, K, wk, ak, k0):
    _, _, mxu = ops
    rng = np.random.default_rng(M + N + K)
    if ak == "row":
        x = rng.standard_normal((M, K)).astype(np.float32)
    elif ak == "mx":
        x = spread(rng, M, K, 1.0, 32)
    else:
        x = spread(rng, M, K, 7.0, 32)
    q, Sa, da = F.quantize_mx(x, 32, row_mode=(ak == "row"))
    KBr = K // 128 + k0
    W = (spread(rng, N, KBr * 128, 1.5, 128) * 0.02).astype(np.float32)
    if wk == "rsc":
        rows, srows = Q.pack_rsc(W)
    else:
        rows, srows = Q.pack_int8x(W)
        if ak == "wide":
            srows[:, 4:4 + KBr] = rng.integers(0, 20, (N, KBr))     # large dw: more drops
    rows = np.ascontiguousarray(rows[:, k0 * 128:k0 * 128 + K])
    flags = MM.RSC if wk == "rsc" else (MM.UNIT if wk == "unit" else 0)
    say("gemm", M, N, K, wk, ak, k0)
    got = mxu.mm(q, Sa, da, rows, srows, "int8", K, rsc=wk == "rsc", unit=wk == "unit", k0=k0)
    want = OC.mm(q, Sa, da, rows, srows, "int8", K, flags=flags, k0=k0)
    assert same_bits(got, want)


@pytest.mark.parametrize("dset,K", [((0, 1), 1024), ((0, 1, 2), 1024), ((1, 3, 4), 1024), ((0, 1, 2, 3), 1024),
                                    ((0, 20), 1024), ((2, 5, 17), 1024), ((0, 31), 1024),
                                    ((0, 1), 4096), ((0, 2), 4224), ((1,), 8192)])
def test_gemm_activation_planes(ops, dset, K):
    """Plain (RSC) weights x activation groups whose offsets take the values dset: one to three
    planes in one K walk, four planes in the plane-by-plane passes, offsets past the window
    (dropped); two planes in one walk at 32 K stages (the staged offsets full) and in the
    plane-by-plane passes at 33; one offset everywhere over 64 stages; against the C oracle."""
    import torch
    _, _, mxu = ops
    rng = np.random.default_rng(sum(dset) * 7 + len(dset) + K)
    M, N = 200, 256
    q = rng.integers(-127, 128, (M, K)).astype(np.int8)
    Sa = np.abs(rng.standard_normal(M)).astype(np.float32) + np.float32(0.5)
    da = np.asarray(dset, np.uint8)[rng.integers(0, len(dset), (M, K // 32))]
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    rows, srows = Q.pack_rsc(W)
    say("gemm planes", dset, K)
    got = mxu.mm(q, Sa, da, rows, srows, "int8", K, rsc=True)
    want = OC.mm(q, Sa, da, rows, srows, "int8", K, flags=MM.RSC)
    assert same_bits(got, want)


def test_gemm_acc_ascale(ops):
    _, _, mxu = ops
    rng = np.random.default_rng(9)
    M, N, K = 72, 200, 512
    x = spread(rng, M, K, 1.0, 32)
    q, Sa, da = F.quantize_mx(x, 32)
    wel = rng.integers(-127, 128, (N, K)).astype(np.int8).view(np.uint8)
    srows = np.zeros((N, 8), np.uint8)
    old = rng.standard_normal((M, N)).astype(np.float32)
    alpha = rng.standard_normal(M).astype(np.float32)
    say("gemm acc / ascale")
    got = mxu.mm(q, Sa, da, wel, srows, "int8", K, unit=True, acc=old)
    assert same_bits(got, OC.mm(q, Sa, da, wel, srows, "int8", K, flags=MM.UNIT | MM.ACC, old=old))
    got = mxu.mm(q, Sa, da, wel, srows, "int8", K, unit=True, acc=old, alpha=alpha)
    assert same_bits(got, OC.mm(q, Sa, da, wel, srows, "int8", K, flags=MM.UNIT | MM.ACC | MM.ASCALE,
                                old=old, alpha=alpha))
    # ROW activations: the single-plane path's epilogue
    q, Sa, da = F.quantize_mx(x, 32, row_mode=True)
    got = mxu.mm(q, Sa, da, wel, srows, "int8", K, unit=True, acc=old)
    assert same_bits(got, OC.mm(q, Sa, da, wel, srows, "int8", K, flags=MM.UNIT | MM.ACC, old=old))
    got = mxu.mm(q, Sa, da, wel, srows, "int8", K, unit=True, acc=old, alpha=alpha)
    assert same_bits(got, OC.mm(q, Sa, da, wel, srows, "int8", K, flags=MM.UNIT | MM.ACC | MM.ASCALE,
                                old=old, alpha=alpha))


@pytest.mark.parametrize("row_mode", [True, False])
def test_gemm_acc_ascale_full_tiles(ops, row_mode):
    """ACC (RSC weights) and ACC + ASCALE (UNIT weights: ASCALE needs both) through the
    full-tile epilogue, whose rows the compute waves and the loader waves store half each:
    128 x 384 outputs, three whole 128 x 128 tiles."""
    _, _, mxu = ops
    rng = np.random.default_rng(11)
    M, N, K = 128, 384, 1024
    x = spread(rng, M, K, 1.0, 32)
    q, Sa, da = F.quantize_mx(x, 32, row_mode=row_mode)
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    rows, srows = Q.pack_rsc(W)
    old = rng.standard_normal((M, N)).astype(np.float32)
    alpha = rng.standard_normal(M).astype(np.float32)
    say("gemm acc / ascale, full tiles", "row" if row_mode else "mx")
    got = mxu.mm(q, Sa, da, rows, srows, "int8", K, rsc=True, acc=old)
    assert same_bits(got, OC.mm(q, Sa, da, rows, srows, "int8", K, flags=MM.RSC | MM.ACC, old=old))
    wel = rng.integers(-127, 128, (N, K)).astype(np.int8).view(np.uint8)
    zs = np.zeros((N, 8), np.uint8)
    got = mxu.mm(q, Sa, da, wel, zs, "int8", K, unit=True, acc=old, alpha=alpha)
    assert same_bits(got, OC.mm(q, Sa, da, wel, zs, "int8", K, flags=MM.UNIT | MM.ACC | MM.ASCALE,
                                old=old, alpha=alpha))


def test_gemm_c3_shape_tile_kinds(ops):
    """The c3 shape's kernel (loader waves beside the MFMA waves) on every kind of tile: each
    128-row tile's activation offsets drawn from its own set -- three planes (the masked passes,
    the loader waves matching their barriers), offsets 9 apart (the exact VALU path), all past
    the window (a zero tile), two planes without offset 0 (the two-plane walk) -- every output
    bit against the C oracle."""
    import torch
    _, quant, mxu = ops
    M, K, N = 512, 2048, 8192
    rng = np.random.default_rng(17)
    q = rng.integers(-127, 128, (M, K)).astype(np.int8)
    Sa = (np.abs(rng.standard_normal(M)) + 0.5).astype(np.float32)
    da = np.zeros((M, K // 32), np.uint8)
    for t, dset in enumerate([(0, 1, 2), (0, 9), (20,), (1, 3)]):
        da[128 * t:128 * (t + 1)] = np.asarray(dset, np.uint8)[rng.integers(0, len(dset), (128, K // 32))]
    gen = torch.Generator(device="cuda").manual_seed(5)
    rows_d, srows_d = quant.quantize_mxu(torch.randn((N, K), generator=gen, device="cuda") * 0.02, "int8", rsc=True)
    rows, srows = rows_d.cpu().numpy(), srows_d.cpu().numpy()
    say("gemm c3 shape: tile kinds")
    got = mxu.mm(q, Sa, da, rows, srows, "int8", K, rsc=True)
    want = OC.mm(q, Sa, da, rows, srows, "int8", K, flags=MM.RSC)
    assert same_bits(got, want)
    assert not np.any(got[256:384]), "offsets past the window: the tile drops every group"


@pytest.mark.parametrize("generic", [False, True])
def test_gemm_c3_full_size(ops, monkeypatch, generic):
    """c3: M=512 x K=2048 x N=8192, ROW activations x RSC weights (the headline GEMM) and MX
    activations (the plane path), every output bit against the C oracle; with the copy compiled
    for c3's sizes and with the generic copy on the same operands (OTPU_GENERIC_COPIES)."""
    import torch
    if generic:
        monkeypatch.setenv("OTPU_GENERIC_COPIES", "1")
    _, quant, mxu = ops
    M, K, N = 512, 2048, 8192
    gen = torch.Generator(device="cuda").manual_seed(3)
    Wd = torch.randn((N, K), generator=gen, device="cuda") * 0.02
    rows_d, srows_d = quant.quantize_mxu(Wd, "int8", rsc=True)
    rows, srows = rows_d.cpu().numpy(), srows_d.cpu().numpy()
    x = np.random.default_rng(3).standard_normal((M, K)).astype(np.float32)
    for row_mode in (True, False):
        q, Sa, da = F.quantize_mx(x, 32, row_mode=row_mode)
        say("gemm c3", "row" if row_mode else "mx", "generic copy" if generic else "c3 copy")
        got = mxu.mm(q, Sa, da, rows, srows, "int8", K, rsc=True)
        want = OC.mm(q, Sa, da, rows, srows, "int8", K, flags=MM.RSC)
        assert same_bits(got, want)
