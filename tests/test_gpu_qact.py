"""GPU parity of QACT's whole instruction and the split operands, through the C ABI, bit for bit
against the oracle: the RSCALE / CSCALE pre-multiplies (each alone, both, denormal products) in
otpu_qact, otpu_qact_ranges and the fused QACT prologues of otpu_mm_qin / otpu_mm_qin_fold; the
split quantizer's LO and HL parts and QST LO rows; QACT ST's DRAM rows and LDA; MM SPL (2 and 3
terms, ACC); quantize() over any shape; the LM head called twice on one best buffer."""
import sys

import numpy as np
import pytest

from conftest import same_bits
from oracle import chain as CH
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
    from opentpu_amd import _lib, fp32, mxu, quant
    _lib.load()
    return _lib, fp32, mxu, quant


def spread(rng, M, K, s=5.0, g=8):
    return (rng.standard_normal((M, K)) * np.exp(rng.uniform(-s, s, (M, K // g, 1)))
            .repeat(g, 2).reshape(M, K)).astype(np.float32)


def factors(rng, M, K):
    r = rng.uniform(0.25, 4.0, M).astype(np.float32)
    c = rng.uniform(0.25, 4.0, K).astype(np.float32)
    r[0] = np.float32(3e-39)                  # a denormal row factor: the row flushes to zero
    c[3] = np.float32(1e-38)                  # products that land on the subnormal grid
    c[5] = np.float32(2.0 ** -100)
    return r, c


@pytest.mark.parametrize("which", ["r", "c", "rc"])
@pytest.mark.parametrize("g,row_mode", [(32, False), (32, True), (128, False)])
def test_qact_premultiplies(ops, which, g, row_mode):
    _, fp32, _, _ = ops
    rng = np.random.default_rng(len(which) + g + row_mode)
    M, K = 7, 1024
    x = spread(rng, M, K)
    x[2, 10] = np.float32(1e-30)
    r, c = factors(rng, M, K)
    rs = r if "r" in which else None
    cs = c if "c" in which else None
    say("qact premultiplies", which, g, row_mode)
    got = fp32.qact(x, g, row_mode, rscale=rs, cscale=cs)
    want = F.qact(x, g, row_mode, rscale=rs, cscale=cs)
    assert np.array_equal(got[0], want[0]) and same_bits(got[1], want[1]) and np.array_equal(got[2], want[2])


@pytest.mark.parametrize("row_mode", [False, True])
def test_qact_lo_and_hl(ops, row_mode):
    _, fp32, _, _ = ops
    rng = np.random.default_rng(11 + row_mode)
    M, K = 9, 2048
    x = spread(rng, M, K, 7.0)
    x[1] = 0
    x[4, 7] = np.inf
    x[5, 9] = np.nan
    r, c = factors(rng, M, K)
    say("qact lo / hl", row_mode)
    q, S, d = fp32.qact(x, 32, row_mode, lo=True)
    q0, S0, d0 = F.quantize_mx(x, 32, row_mode, lo=True)
    assert np.array_equal(q, q0) and same_bits(S, S0) and np.array_equal(d, d0)
    got = fp32.qact(x, 32, row_mode, rscale=r, cscale=c, hl=True)
    want = F.qact(x, 32, row_mode, rscale=r, cscale=c, hl=True)
    for a, b in zip(got, want):
        assert np.array_equal(np.asarray(a).view(np.uint8), np.asarray(b).view(np.uint8))
    assert not np.array_equal(got[0], got[3])


def test_qact_st_rows_and_lda(ops):
    _, fp32, mxu, _ = ops
    rng = np.random.default_rng(12)
    M, K = 6, 640
    x = spread(rng, M, K)
    r, c = factors(rng, M, K)
    say("qact st / lda")
    q, S, d, st = fp32.qact(x, 32, rscale=r, cscale=c, st=True)
    q0, S0, d0 = F.qact(x, 32, rscale=r, cscale=c)
    assert np.array_equal(q, q0) and same_bits(S, S0) and np.array_equal(d, d0)
    assert np.array_equal(st, F.qrows_store(q0, S0, d0))
    ql, Sl, dl, stl = fp32.qact(x, 32, lo=True, st=True)                  # ST of the lo part
    assert np.array_equal(stl, F.qrows_store(*F.quantize_mx(x, 32, lo=True)))
    q2, S2, d2 = fp32.lda(st, K // 128)
    qw, Sw_, dw_ = F.lda(F.qrows_store(q0, S0, d0), K // 128)
    assert np.array_equal(q2, qw) and same_bits(S2, Sw_) and np.array_equal(d2, dw_)
    # an MM over the loaded operand, from block 2 on (Sa = S + 2 rows), equals the QACT's
    rows = rng.integers(0, 256, (40, K)).astype(np.uint8)
    sw = np.full((40, 1), 0.01, np.float32).view(np.uint8)
    y = mxu.mm(q2[:, 256:], S2[2], d2[:, 8:], rows[:, 256:], sw, "int8", K - 256, rsc=True)
    assert same_bits(y, MM.mm(q0[:, 256:], S0, d0[:, 8:], rows[:, 256:], sw, "int8", K - 256, flags=MM.RSC))


@pytest.mark.parametrize("width,mul,lo", [(256, True, False), (384, False, True), (1024, True, True)])
def test_qact_ranges_premultiplies(ops, width, mul, lo):
    import torch
    X = ops[0]
    rng = np.random.default_rng(width + mul)
    M, K = 3, 3072
    a = spread(rng, M, 2 * K)
    x, u = a[:, :K], a[:, K:]
    r, c = factors(rng, M, K)
    ad = torch.from_numpy(a).cuda()
    rd, cd = torch.from_numpy(r).cuda(), torch.from_numpy(c).cuda()
    R = K // width
    q = torch.empty((M, K), dtype=torch.int8, device="cuda")
    S = torch.empty((R * M,), dtype=torch.float32, device="cuda")
    d = torch.empty((M, K // 32), dtype=torch.uint8, device="cuda")
    say("qact ranges premultiplies", width, mul, lo)
    X.call("otpu_qact_ranges", X.ptr(ad), X.ptr(ad[:, K:]) if mul else None, M, K, 2 * K, width, 32,
           X.Q_LO if lo else 0, X.ptr(rd), X.ptr(cd), X.ptr(q), K, X.ptr(S), X.ptr(d), K // 32, X.stream())
    src = F.mul(x, u) if mul else x
    qh, Sh, dh = q.cpu().numpy(), S.cpu().numpy().reshape(R, M), d.cpu().numpy()
    for i in range(R):
        cols = slice(i * width, (i + 1) * width)
        q0, S0, d0 = F.qact(src[:, cols], 32, rscale=r, cscale=c[cols], lo=lo)
        assert np.array_equal(qh[:, cols], q0) and same_bits(Sh[i], S0)
        assert np.array_equal(dh[:, i * width // 32:(i + 1) * width // 32], d0)


@pytest.mark.parametrize("fmt,K,width,nsum,mul", [("int4", 1024, 1024, 1, False), ("int4", 2048, 2048, 3, False),
                                                   ("int8", 1024, 256, 1, True), ("fp4", 3072, 256, 1, True)])
def test_mm_qin_premultiplies(ops, fmt, K, width, nsum, mul):
    import torch
    from oracle import formats as Q
    X = ops[0]
    rng = np.random.default_rng(K + width + nsum)
    N = 300
    W = (spread(rng, N, K, 1.5, 128) * 0.02).astype(np.float32)
    rows, srows = Q.quantize_mxu(W, fmt)
    xs = spread(rng, nsum, K)
    xm = spread(rng, 1, K) if mul else None
    r, c = factors(rng, 1, K)
    r[0] = np.float32(1.7)
    src = xs[0:1]
    for i in range(1, nsum):
        src = F.add(src, xs[i:i + 1])
    if mul:
        src = F.mul(src, xm)
    R = K // width
    bpb = 128 if fmt == "int8" else 64
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    xd, wd, sd, rd, cd = d(xs), d(rows), d(srows), d(r), d(c)
    xmd = d(xm) if mul else None
    out = torch.full((R, N), 7.0, dtype=torch.float32, device="cuda")
    say("mm_qin premultiplies", fmt, K, width, nsum, mul)
    X.call("otpu_mm_qin", X.ptr(xd), X.ptr(xmd), X.ptr(rd), X.ptr(cd), nsum, K, K, width, X.ptr(wd), rows.shape[1],
           X.ptr(sd), srows.shape[1], N, X.FMT[fmt], 0, 0, X.ptr(out), N, N, X.stream())
    got = out.cpu().numpy()
    for i in range(R):
        cols = slice(i * width, (i + 1) * width)
        q, Sa, da = F.qact(src[:, cols], 32, rscale=r, cscale=c[cols])
        part = rows[:, i * width // 128 * bpb:(i + 1) * width // 128 * bpb]
        assert same_bits(got[i:i + 1], MM.mm(q, Sa, da, part, srows, fmt, width, k0=i * width // 128)), i


@pytest.mark.parametrize("fmt,K,N,rc", [("int4", 3072, 1024, "rc"), ("fp4", 1536, 257, "c"), ("nvfp4", 2048, 130, "r")])
def test_mm_qin_fold_premultiplies(ops, fmt, K, N, rc):
    import torch
    from oracle import formats as Q
    X = ops[0]
    rng = np.random.default_rng(K + N)
    W = (spread(rng, N, K, 1.5, 128) * 0.02).astype(np.float32)
    rows, srows = Q.quantize_mxu(W, fmt)
    g, u = spread(rng, 1, K), spread(rng, 1, K)
    r, c = factors(rng, 1, K)
    r[0] = np.float32(0.37)
    h = F.mul(g, u)
    if "r" in rc:
        h = F.mul(h, r[:, None])
    if "c" in rc:
        h = F.mul(h, c[None, :])
    want = CH.ranges_dot(h, (rows, srows), fmt, 256)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    gd, ud, wd, sd, rd, cd = d(g), d(u), d(rows), d(srows), d(r), d(c)
    out = torch.full((1, N), 7.0, dtype=torch.float32, device="cuda")
    say("mm_qin_fold premultiplies", fmt, K, N, rc)
    X.call("otpu_mm_qin_fold", X.ptr(gd), X.ptr(ud), X.ptr(rd) if "r" in rc else None,
           X.ptr(cd) if "c" in rc else None, K, 256, X.ptr(wd), rows.shape[1], X.ptr(sd), srows.shape[1], N,
           X.FMT[fmt], 0, 0, X.ptr(out), X.stream())
    assert same_bits(out.cpu().numpy(), want)


def test_pack_int8_lo_rows(ops):
    _, fp32, _, quant = ops
    rng = np.random.default_rng(13)
    W = (spread(rng, 50, 512, 3.0) * 0.02).astype(np.float32)
    say("pack int8 lo rows")
    rows, sw = quant.quantize_mxu(W, "int8", rsc=True, lo=True)
    q0, S0, _ = F.quantize_mx(W, 512, row_mode=True, lo=True)
    assert np.array_equal(rows.view(np.int8), q0) and same_bits(sw.view(np.float32)[:, 0], S0)


@pytest.mark.parametrize("nterms,M,N", [(3, 1, 300), (3, 5, 64), (2, 3, 130), (3, 16, 17)])
def test_mm_spl(ops, nterms, M, N):
    _, fp32, mxu, quant = ops
    rng = np.random.default_rng(nterms * 100 + M + N)
    x = spread(rng, M, 128, 6.0, 32)
    x[0, 96:] *= np.float32(2.0 ** -11)                     # lo terms that drop
    W = (spread(rng, N, 128, 2.0, 32) * 0.02).astype(np.float32)
    qh, Sa, da, ql, _ = F.qact(x, 32, hl=True)
    q = np.concatenate([qh, ql], 1) if nterms == 3 else qh
    wh, Sw, _ = F.quantize_mx(W, 128, row_mode=True)
    wl, _, _ = F.quantize_mx(W, 128, row_mode=True, lo=True)
    say("mm spl", nterms, M, N)
    # the operands from the GPU's own quantizers equal the oracle's
    g = fp32.qact(x, 32, hl=True)
    assert np.array_equal(g[0], qh) and np.array_equal(g[3], ql)
    rh, sh = quant.quantize_mxu(W, "int8", rsc=True)
    rl, _ = quant.quantize_mxu(W, "int8", rsc=True, lo=True)
    assert np.array_equal(rh.view(np.int8), wh) and np.array_equal(rl.view(np.int8), wl)
    got = mxu.mm_spl(q, Sa, da, rh, rl, sh.view(np.float32)[:, 0], nterms)
    want = MM.mm_spl(q, Sa, da, wh, wl, Sw, nterms)
    assert same_bits(got, want)
    old = rng.standard_normal((M, N)).astype(np.float32)
    got = mxu.mm_spl(q, Sa, da, rh, rl, Sw, nterms, acc=old)
    assert same_bits(got, MM.mm_spl(q, Sa, da, wh, wl, Sw, nterms, old=old))


def test_mm_spl_refusals(ops):
    X = ops[0]
    p = 256
    for nterms, flags in [(4, X.RSC), (3, 0), (3, X.RSC | X.UNIT), (2, X.RSC | X.RMAX)]:
        with pytest.raises(X.OtpuError):
            X.call("otpu_mm_spl", p, 256, p, p, 4, 1, nterms, p, 256, 128, p, 4, 8, flags, p, 8, X.stream())


@pytest.mark.parametrize("shape,axis", [((3, 5, 7), -1), ((4, 9), 0), ((1000,), 0), ((2, 3, 130), 1)])
def test_quantize_any_shape(ops, shape, axis):
    _, fp32, _, _ = ops
    rng = np.random.default_rng(len(shape) + axis)
    x = (rng.standard_normal(shape) * 3).astype(np.float32)
    say("quantize", shape, axis)
    q, S = fp32.quantize(x, axis)
    xm = np.moveaxis(x, axis, -1)
    q0, S0 = F.quantize_rows(xm.reshape(-1, xm.shape[-1]))
    assert np.array_equal(np.moveaxis(q, axis, -1).reshape(q0.shape), q0)
    assert same_bits(S.reshape(-1), S0)


def test_lm_head_twice_on_one_best_buffer(ops):
    """The running maxima are left zero by each call: a later call with other weights (and
    another grid) picks its own token, not an earlier call's; the third call's best logit equals
    the second's at a higher index, so a maximum left over would win the tie."""
    import torch
    X = ops[0]
    rng = np.random.default_rng(14)
    K = 256
    x = np.abs(rng.standard_normal((1, K))).astype(np.float32)
    q, Sa, da = F.quantize_mx(x, 32)
    best = torch.zeros((X.LM_STATE_BYTES // 8,), dtype=torch.int64, device="cuda")
    tok = torch.empty((1,), dtype=torch.int32, device="cuda")
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    qd, Sad, dad = d(q), d(Sa), d(da)
    say("lm head twice")
    for N, hot, scale in ((3000, 2500, 0.05), (1000, 17, 0.01), (3000, 2999, 0.01)):
        rows = rng.integers(-20, 21, (N, K)).astype(np.int8)
        rows[hot] = 127
        srows = np.full((N, 1), scale, np.float32).view(np.uint8)
        wd, sd = d(rows.view(np.uint8)), d(srows)
        X.call("otpu_lm_head_argmax", X.ptr(qd), X.ptr(Sad), X.ptr(dad), K, X.ptr(wd), K, X.ptr(sd), 4, N,
               X.FMT["int8"], X.RSC, 0, 0, None, X.ptr(best), X.ptr(tok), X.stream())
        logits = MM.mm(q, Sa, da, rows.view(np.uint8), srows, "int8", K, flags=MM.RSC)[0]
        assert int(tok.item()) == MM.greedy(logits) == hot
        b = best.cpu().numpy().view(np.uint64)
        assert int(b[0]) == MM.best_word(logits) and not b[1:].any()
