"""GPU parity of the chained decode path: QACT over ranges (with the fused VOP MUL), the per-range
MMs with their ACC chain (otpu_mm_ranges), and the whole Qwen3-shaped decode step
(opentpu_amd.chain.DecodeChain, eager and as a replayed HIP graph) against oracle/chain.py,
bit for bit."""
import sys

import numpy as np
import pytest

from conftest import same_bits
from oracle import chain as CH
from oracle import cpu as OC
from oracle import fp32 as F
from oracle import mm as MM

pytestmark = pytest.mark.gpu


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


def spread(rng, M, K, s=5.0, g=8):
    return (rng.standard_normal((M, K)) * np.exp(rng.uniform(-s, s, (M, K // g, 1)))
            .repeat(g, 2).reshape(M, K)).astype(np.float32)


@pytest.mark.parametrize("width,mul", [(256, False), (256, True), (384, True), (3072, False), (128, True)])
def test_qact_ranges(X, width, mul):
    import torch
    rng = np.random.default_rng(width + mul)
    M, K = 3, 3072
    a = spread(rng, M, 2 * K)                      # [g | u] side by side, like the gate/up output
    a[1, 5:300] = 0
    x, u = a[:, :K], a[:, K:]
    say("qact_ranges", width, mul)
    ad = torch.from_numpy(a).cuda()
    R = K // width
    q = torch.empty((M, K), dtype=torch.int8, device="cuda")
    S = torch.empty((R * M,), dtype=torch.float32, device="cuda")
    d = torch.empty((M, K // 32), dtype=torch.uint8, device="cuda")
    X.call("otpu_qact_ranges", X.ptr(ad), X.ptr(ad[:, K:]) if mul else None, M, K, 2 * K, width, 32, 0,
           None, None, X.ptr(q), K, X.ptr(S), X.ptr(d), K // 32, X.stream())
    src = F.mul(x, u) if mul else x
    qh, Sh, dh = q.cpu().numpy(), S.cpu().numpy().reshape(R, M), d.cpu().numpy()
    for r in range(R):
        q0, S0, d0 = F.quantize_mx(src[:, r * width:(r + 1) * width], 32)
        assert np.array_equal(qh[:, r * width:(r + 1) * width], q0)
        assert same_bits(Sh[r], S0)
        assert np.array_equal(dh[:, r * width // 32:(r + 1) * width // 32], d0)


def _weights(rng, N, K, fmt, rsc=False):
    from oracle import formats as Q
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    if rsc:
        return Q.pack_rsc(W)
    return Q.pack_int8x(W) if fmt == "int8" else Q.pack_x4(W, fmt)


@pytest.mark.parametrize("fmt,width,M,acc,rsc", [
    ("int8", 128, 1, False, False), ("int8", 384, 3, True, False), ("int8", 256, 2, False, True),
    ("int4", 256, 1, False, False), ("int4", 512, 4, True, False), ("fp4", 256, 2, False, False),
])
def test_mm_ranges(X, fmt, width, M, acc, rsc):
    import torch
    rng = np.random.default_rng(7 * width + M)
    K, N = 1536, 200
    rows, srows = _weights(rng, N, K, fmt, rsc)
    x = spread(rng, M, K)
    R = K // width
    qs, Sas, das = [], [], []
    for r in range(R):
        q0, S0, d0 = F.quantize_mx(x[:, r * width:(r + 1) * width], 32, row_mode=rsc)
        qs.append(q0), Sas.append(S0), das.append(d0)
    q, Sa, da = np.concatenate(qs, 1), np.stack(Sas), np.concatenate(das, 1)
    old = rng.standard_normal((M, N)).astype(np.float32)
    bpb = 128 if fmt == "int8" else 64
    y = old if acc else None
    for r in range(R):
        k0 = 0 if rsc else r * width // 128
        part = rows[:, r * width // 128 * bpb:(r + 1) * width // 128 * bpb]
        y = MM.mm(qs[r], Sas[r], das[r], part, srows, fmt, width, k0=k0,
                  flags=(MM.ACC if y is not None else 0) | (MM.RSC if rsc else 0), old=y)
    say("mm_ranges", fmt, width, M, acc, rsc)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    qd, Sad, dad, wd, sd = d(q), d(Sa.reshape(-1)), d(da), d(rows), d(srows)
    out = d(old if acc else np.zeros((M, N), np.float32))
    part = torch.empty((R, M, N), dtype=torch.float32, device="cuda")
    fl = (X.ACC if acc else 0) | (X.RSC if rsc else 0)
    X.call("otpu_mm_ranges", X.ptr(qd), K, X.ptr(Sad), X.ptr(dad), K // 32, M, K, width, X.ptr(wd), rows.shape[1],
           X.ptr(sd), srows.shape[1], N, X.FMT[fmt], fl, 0, X.ptr(part), X.ptr(out), N, X.stream())
    assert same_bits(out.cpu().numpy(), y)


def test_mm_ranges_refusals(X):
    import torch
    from opentpu_amd._lib import OtpuError
    t = torch.zeros(1 << 16, dtype=torch.uint8, device="cuda")
    p = X.ptr(t)
    with pytest.raises(OtpuError):      # 4-bit ranges must be whole 128-byte chunks (256 columns)
        X.call("otpu_mm_ranges", p, 1024, p, p, 32, 1, 1024, 128, p, 512, p, 40, 8, X.FMT["int4"], 0, 0, p, p, 8,
               X.stream())
    with pytest.raises(OtpuError):      # ranges must tile K
        X.call("otpu_mm_ranges", p, 1024, p, p, 32, 1, 1024, 384, p, 1024, p, 12, 8, X.FMT["int8"], 0, 0, p, p, 8,
               X.stream())


@pytest.mark.parametrize("fmt,K,width,nsum,mul", [
    ("int4", 1024, 1024, 1, False), ("int4", 1024, 1024, 12, False), ("int4", 2048, 2048, 1, False),
    ("int4", 3072, 256, 1, True), ("fp4", 1536, 512, 2, True), ("int8", 1024, 1024, 3, False),
    ("int8", 3072, 384, 1, True), ("int8", 2560, 2560, 1, False),
])
def test_mm_qin(X, fmt, K, width, nsum, mul):
    """QACT + MM in one launch: each range's output equals QACT (oracle) of the range of the
    folded (and multiplied) row followed by the oracle MM on that range's weight columns."""
    import torch
    rng = np.random.default_rng(K + width + nsum)
    N = 300
    rows, srows = _weights(rng, N, K, fmt)
    xs = spread(rng, nsum, K)
    xm = spread(rng, 1, K) if mul else None
    src = xs[0:1]
    for i in range(1, nsum):
        src = F.add(src, xs[i:i + 1])
    if mul:
        src = F.mul(src, xm)
    R = K // width
    bpb = 128 if fmt == "int8" else 64
    say("mm_qin", fmt, K, width, nsum, mul)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    xd, wd, sd = d(xs), d(rows), d(srows)
    xmd = d(xm) if mul else None
    out = torch.full((R, N), 7.0, dtype=torch.float32, device="cuda")
    X.call("otpu_mm_qin", X.ptr(xd), X.ptr(xmd), None, None, nsum, K, K, width, X.ptr(wd), rows.shape[1],
           X.ptr(sd), srows.shape[1], N, X.FMT[fmt], 0, 0, X.ptr(out), N, N, X.stream())
    got = out.cpu().numpy()
    for r in range(R):
        q, Sa, da = F.quantize_mx(src[:, r * width:(r + 1) * width], 32)
        part = rows[:, r * width // 128 * bpb:(r + 1) * width // 128 * bpb]
        y = MM.mm(q, Sa, da, part, srows, fmt, width, k0=r * width // 128)
        assert same_bits(got[r:r + 1], y), f"range {r}"


@pytest.mark.parametrize("fmt,K,N,width", [("int4", 3072, 1024, 256), ("int4", 1024, 300, 256),
                                            ("fp4", 1536, 257, 256), ("nvfp4", 2048, 130, 256),
                                            ("int4", 4096, 77, 256), ("int4", 4096, 150, 512),
                                            ("int4", 6144, 200, 768), ("fp4", 8192, 96, 1024),
                                            ("nvfp4", 6144, 64, 1536), ("int4", 7680, 40, 2560)])
def test_mm_qin_fold(X, fmt, K, N, width):
    """The down projection folded in one launch: QACT of every range of width columns of
    mul(g, u) (256, and the reference's wider chunks: 768 at F = 6144, 1024 at 8192; ranges that
    straddle a team slot's 256-column sub-ranges), an MM per range and the ACC of the ranges in
    order, against the oracle's ranges_dot."""
    import torch
    from oracle import formats as Q
    rng = np.random.default_rng(K + N + len(fmt))
    W = (spread(rng, N, K, 1.5, 128) * 0.02).astype(np.float32)
    rows, srows = Q.quantize_mxu(W, fmt)
    g, u = spread(rng, 1, K), spread(rng, 1, K)
    want = CH.ranges_dot(F.mul(g, u), (rows, srows), fmt, width)
    say("mm_qin_fold", fmt, K, N, width)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    gd, ud, wd, sd = d(g), d(u), d(rows), d(srows)
    out = torch.full((1, N), 7.0, dtype=torch.float32, device="cuda")
    X.call("otpu_mm_qin_fold", X.ptr(gd), X.ptr(ud), None, None, K, width, X.ptr(wd), rows.shape[1], X.ptr(sd),
           srows.shape[1], N, X.FMT[fmt], 0, 0, X.ptr(out), X.stream())
    assert same_bits(out.cpu().numpy(), want)


def test_mm_qin_fold_refusals(X):
    from opentpu_amd._lib import OtpuError
    p = 256
    for args in [(1024, 256, X.FMT["int8"], 0), (1000, 256, X.FMT["int4"], 0), (8448, 256, X.FMT["int4"], 0),
                 (1024, 256, X.FMT["int4"], X.RSC), (1024, 384, X.FMT["int4"], 0), (1536, 1024, X.FMT["int4"], 0),
                 (1024, 0, X.FMT["int4"], 0)]:
        K, width, fmt, flags = args
        with pytest.raises(OtpuError):
            X.call("otpu_mm_qin_fold", p, p, None, None, K, width, p, 512, p, 40, 8, fmt, flags, 0, p, X.stream())


def test_acc_rows(X):
    import torch
    rng = np.random.default_rng(9)
    p = (rng.standard_normal((5, 1000)) * np.exp(rng.uniform(-30, 30, (5, 1000)))).astype(np.float32)
    old = rng.standard_normal(1000).astype(np.float32)
    pd, od = torch.from_numpy(p).cuda(), torch.from_numpy(old).cuda()
    out = torch.empty(1000, dtype=torch.float32, device="cuda")
    X.call("otpu_acc_rows", X.ptr(pd), 5, 1000, 1000, None, X.ptr(out), X.stream())
    y = p[0]
    for i in range(1, 5):
        y = F.add(y, p[i])
    assert same_bits(out.cpu().numpy(), y)
    X.call("otpu_acc_rows", X.ptr(pd), 5, 1000, 1000, X.ptr(od), X.ptr(out), X.stream())
    y = old
    for i in range(5):
        y = F.add(y, p[i])
    assert same_bits(out.cpu().numpy(), y)


def _host_layers(chain):
    return [{k: (r.cpu().numpy(), s.cpu().numpy()) for k, (r, s) in w.items()} for w in chain.layers]


def test_chain_layers_small(X):
    """Each layer on its own N(0,1) input: every intermediate (qkv, o, gate/up, down) bit-exact."""
    import torch
    from opentpu_amd.chain import DecodeChain, Shape
    sh = Shape(hidden=256, q_dim=512, kv_dim=256, F=768, layers=3)
    say("chain small: pack")
    ch = DecodeChain.synthetic(sh, "int4", seed0=7, std=0.05)
    assert ch.width == CH.down_chunk(768, "int4") == 256
    host = _host_layers(ch)
    rng = np.random.default_rng(5)
    for l in range(sh.layers):
        x = rng.standard_normal((1, 256)).astype(np.float32)
        xd = torch.from_numpy(x).cuda()
        yd = torch.empty((1, 256), dtype=torch.float32, device="cuda")
        say("chain small: layer", l)
        ch.layer(l, xd, yd)
        y0, mid = CH.layer(x, host[l], "int4", 512, 768)
        assert same_bits(ch.qkv.cpu().numpy(), mid["qkv"])
        assert same_bits(ch.o.cpu().numpy(), mid["o"])
        assert same_bits(ch.gu.cpu().numpy(), mid["gu"])
        assert same_bits(yd.cpu().numpy(), y0)
    x = rng.standard_normal((1, 256)).astype(np.float32)
    want = CH.step(x, host, "int4", 512, 768)
    ch.fused = False
    assert same_bits(ch.step(x).cpu().numpy(), want)
    ch.fused = True
    assert ch.fold and ch.persistent and ch.kernels_per_step == 1
    say("chain small: persistent step")
    assert same_bits(ch.step(x).cpu().numpy(), want)
    # every phase's plain output row: the last layer's
    assert same_bits(ch.gu.cpu().numpy(), CH.layer(CH.step(x, host[:2], "int4", 512, 768), host[2], "int4", 512,
                                                   768)[1]["gu"])
    assert ch.chain_error() == 0
    ch.persistent = False
    assert same_bits(ch.step(x).cpu().numpy(), want)
    ch.persistent = True
    ch.fold = False                                # the down chunks' partial rows, folded later
    assert same_bits(ch.step(x).cpu().numpy(), want)
    ch.fold = True
    yd = torch.empty((1, 256), dtype=torch.float32, device="cuda")
    ch.layer_folded(1, torch.from_numpy(x).cuda(), yd)
    assert same_bits(yd.cpu().numpy(), CH.layer(x, host[1], "int4", 512, 768)[0])


def test_chain_with_norms(X):
    """Per-layer RMSNorm factors riding in the qkv and gate / up QACTs (CSCALE gamma, RSCALE r):
    every path (fused, folded, partial rows, unfused, graph replay) against the oracle's layers
    with the same factors, bit for bit."""
    import torch
    from opentpu_amd.chain import DecodeChain, Shape
    sh = Shape(hidden=256, q_dim=512, kv_dim=256, F=768, layers=3)
    say("chain with norms: pack")
    base = DecodeChain.synthetic(sh, "int4", seed0=9, std=0.05)
    rng = np.random.default_rng(8)
    norms = [(rng.uniform(0.5, 2.0, 256).astype(np.float32), rng.uniform(0.5, 2.0, 256).astype(np.float32))
             for _ in range(sh.layers)]
    ch = DecodeChain(base.layers, sh, "int4", True, norms)
    r = rng.uniform(0.5, 3.0, (sh.layers, 2)).astype(np.float32)
    ch.rnorm.copy_(torch.from_numpy(r).cuda())
    host = _host_layers(ch)
    onorms = [(norms[l][0], norms[l][1], r[l, 0:1], r[l, 1:2]) for l in range(sh.layers)]
    x = rng.standard_normal((1, 256)).astype(np.float32)
    want = CH.step(x, host, "int4", 512, 768, onorms)
    assert not same_bits(want, CH.step(x, host, "int4", 512, 768))
    for fused, fold, pers in ((True, True, True), (True, True, False), (True, False, False), (False, True, False)):
        ch.fused, ch.fold, ch.persistent = fused, fold, pers
        say("chain with norms", fused, fold, pers)
        assert same_bits(ch.step(x).cpu().numpy(), want), (fused, fold, pers)
    ch.fused, ch.fold = True, True
    for pers in (True, False):
        ch.persistent = pers
        ch.capture()
        for i in range(2):
            assert same_bits(ch.replay(x).cpu().numpy(), want), f"replay {i} persistent {pers}"
            torch.cuda.synchronize()
    assert ch.chain_error() == 0


def test_chain_c4_full_and_graph(X, monkeypatch):
    """The c4 workload (28 layers, Qwen3-0.6B linears, int4x weights seeded 100 + layer): the
    eager step and three replays of its HIP graph (with eager work between them) all equal the
    oracle's step bit for bit; the first layers' outputs are not all zero."""
    import torch
    from opentpu_amd.chain import DecodeChain, Shape
    say("chain c4: pack")
    ch = DecodeChain.synthetic(Shape(), "int4", seed0=100)
    host = _host_layers(ch)
    rng = np.random.default_rng(4)
    x = rng.standard_normal((1, 1024)).astype(np.float32)
    say("chain c4: layer by layer")
    xo, xd = x, torch.from_numpy(x).cuda()
    nonzero = []
    for l in range(28):
        yd = torch.empty((1, 1024), dtype=torch.float32, device="cuda")
        ch.layer(l, xd, yd)
        xo, _ = CH.layer(xo, host[l], "int4")
        assert same_bits(yd.cpu().numpy(), xo), f"layer {l}"
        nonzero.append(int(np.count_nonzero(xo)))
        xd = yd
    say("nonzero outputs per layer", nonzero)
    assert nonzero[0] > 900
    want = xo
    say("chain c4: eager step, persistent, fused (folded down projection, and partial rows) and unfused")
    assert ch.fold and ch.persistent and ch.kernels_per_step == 1
    assert same_bits(ch.step(x).cpu().numpy(), want)
    assert ch.chain_error() == 0
    say("chain c4: eager step, the persistent kernel's generic copy (OTPU_GENERIC_COPIES at plan time)")
    monkeypatch.setenv("OTPU_GENERIC_COPIES", "1")
    ch._plan = None                                # (a plan reads the setting when it is built)
    assert same_bits(ch.step(x).cpu().numpy(), want)
    assert ch.chain_error() == 0
    monkeypatch.delenv("OTPU_GENERIC_COPIES")
    ch._plan = None
    ch.persistent = False
    assert ch.kernels_per_step == 112
    assert same_bits(ch.step(x).cpu().numpy(), want)
    ch.fold = False
    assert same_bits(ch.step(x).cpu().numpy(), want)
    ch.fold = True
    ch.fused = False
    assert same_bits(ch.step(x).cpu().numpy(), want)
    ch.fused = True
    say("chain c4: layers on N(0,1) inputs, fused")
    for l in (0, 13, 27):                          # mid-stack layers on live (nonzero) inputs
        xl = rng.standard_normal((1, 1024)).astype(np.float32)
        ch.x.copy_(torch.from_numpy(xl).cuda())
        ch.layer_fused(l, ch.x, 1, ch.parts[0])
        yl = torch.empty((1, 1024), dtype=torch.float32, device="cuda")
        X.call("otpu_acc_rows", X.ptr(ch.parts[0]), ch.R, 1024, 1024, None, X.ptr(yl), X.stream())
        want_l = CH.layer(xl, host[l], "int4")[0]
        assert same_bits(yl.cpu().numpy(), want_l), f"fused layer {l}"
        ch.layer_folded(l, ch.x, yl)
        assert same_bits(yl.cpu().numpy(), want_l), f"folded layer {l}"
    x1 = rng.standard_normal((1, 1024)).astype(np.float32)
    want1 = CH.step(x1, host, "int4")
    for pers in (False, True):
        say("chain c4: graph, persistent", pers)
        ch.persistent = pers
        ch.capture()
        for i in range(3):
            got = ch.replay(x1 if i == 1 else x).cpu().numpy()
            assert same_bits(got, want1 if i == 1 else want), f"replay {i} persistent {pers}"
            torch.cuda.synchronize()
            ch.qkv.fill_(float(i))                 # eager work between replays
    assert ch.chain_error() == 0


def test_chain_c4_layers_against_the_float64_emulation(X):
    """The c4 layers 0, 13 and 27 on live N(0, 1) inputs, every linear of the GPU's fused, folded
    layer against the float64 layer with the quantization points (oracle/chain.py
    emulated_layer: the reference's emulated_logits structure) within EMU_TOL of the linear's
    largest output: quantization error and machine rounding apart from kernel bugs."""
    import torch
    from opentpu_amd.chain import DecodeChain, Shape
    from test_oracle_chain import EMU_TOL
    say("chain c4 emulation: pack")
    ch = DecodeChain.synthetic(Shape(), "int4", seed0=100)
    rng = np.random.default_rng(13)
    for l in (0, 13, 27):
        host = {k: (r.cpu().numpy(), s.cpu().numpy()) for k, (r, s) in ch.layers[l].items()}
        x = rng.standard_normal((1, 1024)).astype(np.float32)
        yd = torch.empty((1, 1024), dtype=torch.float32, device="cuda")
        say("chain c4 emulation: layer", l)
        ch.layer_folded(l, torch.from_numpy(x).cuda(), yd)
        ye, me = CH.emulated_layer(x, host, "int4")
        got = {"qkv": ch.qkv.cpu().numpy(), "o": ch.o.cpu().numpy(), "gu": ch.gu.cpu().numpy(),
               "down": yd.cpu().numpy()}
        for k, g in got.items():
            err = np.abs(g.astype(np.float64) - me[k]).max()
            assert err <= EMU_TOL * np.abs(me[k]).max(), (l, k, err / np.abs(me[k]).max())


@pytest.mark.parametrize("fmt,hidden,q_dim,kv_dim,F,layers", [("int4", 256, 512, 512, 768, 2),
                                                            ("fp4", 512, 1024, 256, 1536, 4),
                                                            ("int4", 512, 1024, 256, 1536, 4),
                                                            ("int4", 1024, 2048, 512, 3840, 2),
                                                            ("fp4", 1024, 2048, 1024, 3072, 2),
                                                            ("int4", 2048, 2048, 1024, 6144, 2),
                                                            ("fp4", 1536, 2048, 512, 8192, 2),
                                                            ("nvfp4", 1024, 2048, 1024, 3072, 2),
                                                            ("nvfp4", 2048, 2048, 1024, 6144, 2)])
def test_chain_persistent_formats_and_shapes(X, monkeypatch, fmt, hidden, q_dim, kv_dim, F, layers):
    """The persistent step (otpu_chain_step) on fp4x6 and int4x weights, at a shape whose q/k/v
    rows span more workgroups than o's (96 against 64: o then waits for the k and v entries as
    well), at a shape whose phases leave most workgroups without rows, at the largest F of the one-piece teams' copy with
    256-column down chunks (3840), at the Qwen3-0.6B shape in fp4x6 (its shape's own copy; int4x
    is the c4 test's), and in the wider teams' copies at the Qwen3-1.7B shape (hidden 2048,
    F 6144: its own copy) and at F 8192 (its largest), nvfp4 weights at both Qwen3 shapes (the
    generic copies: nvfp4's scale rows match no shape copy), with per-layer norms: the oracle's step
    bit for bit, eager and over graph replays with new inputs, the error word 0; then one step
    on the generic copy (OTPU_GENERIC_COPIES), the same bits."""
    import torch
    from opentpu_amd.chain import DecodeChain, Shape
    sh = Shape(hidden=hidden, q_dim=q_dim, kv_dim=kv_dim, F=F, layers=layers)
    say("chain persistent", fmt, hidden, q_dim, kv_dim, F, layers)
    base = DecodeChain.synthetic(sh, fmt, seed0=21, std=0.04)
    rng = np.random.default_rng(22)
    norms = [(rng.uniform(0.5, 2.0, hidden).astype(np.float32), rng.uniform(0.5, 2.0, hidden).astype(np.float32))
             for _ in range(sh.layers)]
    ch = DecodeChain(base.layers, sh, fmt, True, norms)
    assert ch.persistent and ch.kernels_per_step == 1
    r = rng.uniform(0.5, 3.0, (sh.layers, 2)).astype(np.float32)
    ch.rnorm.copy_(torch.from_numpy(r).cuda())
    host = _host_layers(ch)
    onorms = [(norms[l][0], norms[l][1], r[l, 0:1], r[l, 1:2]) for l in range(sh.layers)]
    xs = [rng.standard_normal((1, hidden)).astype(np.float32) for _ in range(3)]
    wants = [CH.step(x, host, fmt, q_dim, F, onorms, mm=OC.mm) for x in xs]
    assert same_bits(ch.step(xs[0]).cpu().numpy(), wants[0])
    ch.capture()
    for i in range(4):
        assert same_bits(ch.replay(xs[i % 3]).cpu().numpy(), wants[i % 3]), f"replay {i}"
        torch.cuda.synchronize()
    assert same_bits(ch.step(xs[2]).cpu().numpy(), wants[2])
    assert ch.chain_error() == 0
    say("chain persistent: the generic copy")
    monkeypatch.setenv("OTPU_GENERIC_COPIES", "1")
    ch._plan = None                                # (a plan reads the setting when it is built)
    assert same_bits(ch.step(xs[1]).cpu().numpy(), wants[1])
    assert ch.chain_error() == 0


@pytest.mark.parametrize("fmt,hidden,q_dim,kv_dim,F,std", [("int4", 2048, 2048, 1024, 6144, 0.03),
                                                             ("fp4", 2048, 2048, 1024, 6144, 0.03),
                                                             ("nvfp4", 1024, 2048, 1024, 3072, 0.04)])
def test_chain_full_depth_persistent_equals_launches(X, fmt, hidden, q_dim, kv_dim, F, std):
    """28 layers at the Qwen3-1.7B shape (its own copy of the persistent kernel, int4x and fp4x6)
    and in nvfp4 at the Qwen3-0.6B shape (the generic copy): every row the persistent step leaves
    (the last layer's q/k/v, o, gate/up products and output) equals the launch-per-linear path's
    bit for bit (whose kernels the oracle checks: test_mm_qin_fold, the c4 test's layers), eager
    and over graph replays; the output row is live (mostly nonzero)."""
    import torch
    from opentpu_amd.chain import DecodeChain, Shape
    sh = Shape(hidden=hidden, q_dim=q_dim, kv_dim=kv_dim, F=F)
    say("chain full depth", fmt, hidden, q_dim, kv_dim, F)
    ch = DecodeChain.synthetic(sh, fmt, seed0=300, std=std)
    assert ch.persistent and ch.kernels_per_step == 1
    rng = np.random.default_rng(5)
    xs = [rng.standard_normal((1, hidden)).astype(np.float32) for _ in range(2)]

    def rows():
        return [t.cpu().numpy().copy() for t in (ch.qkv, ch.o, ch.gu, ch.y)]
    ch.persistent = False
    wants = []
    for x in xs:
        ch.step(x)
        wants.append(rows())
    say("nonzero outputs", [int(np.count_nonzero(w[3])) for w in wants])
    assert all(np.count_nonzero(w[3]) > hidden // 2 for w in wants)
    ch.persistent = True
    for x, want in zip(xs, wants):
        ch.step(x)
        for g, w in zip(rows(), want):
            assert same_bits(g, w)
    assert ch.chain_error() == 0
    ch.capture()
    for i in range(3):
        ch.replay(xs[i % 2])
        torch.cuda.synchronize()
        for g, w in zip(rows(), wants[i % 2]):
            assert same_bits(g, w), f"replay {i}"
    assert ch.chain_error() == 0


def test_chain_plan_refusals(X):
    """otpu_chain_plan refuses what its compiled phases cannot hold, before touching the plan."""
    import ctypes as C
    import torch
    from opentpu_amd._lib import OtpuError
    buf = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    P4 = C.c_void_p * 4
    I4 = C.c_int64 * 4
    p = X.ptr(buf)
    arr = P4(p, p, p, p)
    for layers, hidden, q, kv, F, fmt in ((1, 2304, 2048, 512, 3072, 1), (1, 1024, 4096, 512, 3072, 1),
                                         (1, 1024, 2048, 512, 3200, 1), (1, 1024, 2048, 512, 3072, 0),
                                         (1, 1024, 2048, 512, 8448, 2), (0, 1024, 2048, 512, 3072, 1)):
        with pytest.raises(OtpuError):
            X.call("otpu_chain_plan", layers, hidden, q, kv, F, 256, fmt, arr, I4(512, 1024, 512, 1536), arr,
                   I4(64, 128, 64, 192), None, None, p, arr, p, 1 << 20)
    # o waits for k and v when the q/k/v rows span more workgroups than o's (hidden 256: o on 64
    # workgroups, q/k/v on 129); that wait holds 2048 entries
    with pytest.raises(OtpuError, match="kv_dim"):
        X.call("otpu_chain_plan", 1, 256, 2048, 1040, 768, 256, 1, arr, I4(512, 1024, 512, 1536), arr,
               I4(64, 128, 64, 192), None, None, p, arr, p, 1 << 20)
    assert X.load().otpu_chain_plan_bytes(0, 1024, 2048, 512, 3072) == -1


def test_chain_wait_timeout_sets_the_error_word(X, monkeypatch):
    """The persistent step's bounded waits, driven from the host: with a poll limit of 0
    (OTPU_CHAIN_SPIN, read when the plan is built) the waits give up at once, the step still
    ends (every wave exits) and the plan's error word says the outputs are invalid; a plan with
    the default limit on the same chain then runs clean and bit-exact."""
    import torch
    from opentpu_amd._lib import OtpuError
    from opentpu_amd.chain import DecodeChain, Shape
    sh = Shape(hidden=256, q_dim=512, kv_dim=256, F=768, layers=4)
    base = DecodeChain.synthetic(sh, "int4", seed0=31, std=0.05)
    x = np.random.default_rng(32).standard_normal((1, 256)).astype(np.float32)
    want = CH.step(x, _host_layers(base), "int4", 512, 768)
    monkeypatch.setenv("OTPU_CHAIN_SPIN", "0")
    ch = DecodeChain(base.layers, sh, "int4")
    say("chain timeout: spin 0")
    for _ in range(3):
        ch.step(x, check=False)
    torch.cuda.synchronize()
    assert ch.chain_error() == 1
    with pytest.raises(OtpuError, match="timed out"):       # the checked paths raise
        ch.check()
    with pytest.raises(OtpuError, match="timed out"):
        ch.step(x)
    with pytest.raises(OtpuError, match="timed out"):
        ch.replay(x)
    monkeypatch.delenv("OTPU_CHAIN_SPIN")
    ok = DecodeChain(base.layers, sh, "int4")
    assert same_bits(ok.step(x).cpu().numpy(), want)
    assert ok.chain_error() == 0
