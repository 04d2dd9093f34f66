"""GPU parity of the sampler (otpu_sample through opentpu_amd.sampler): the ids of the
reference's device sampler (golden vectors written from generate.reference_pick, including a
soft cap, a repetition penalty and a vocabulary with masked blocks), the oracle's candidate
values and ids, a 262144-token vocabulary, and the LM head's logits sampled on one stream."""
import os
import sys

import numpy as np
import pytest

from conftest import same_bits
from oracle import formats as Q
from oracle import fp32 as F
from oracle import mm as MM
from oracle import sampler as SP

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden", "sampler.npz")


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def S():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    from opentpu_amd import _lib, sampler
    _lib.load()
    return sampler


@pytest.mark.parametrize("i", range(10))
@pytest.mark.parametrize("nu", [4096, 1, 16, 17])
def test_picks_match_the_reference(S, i, nu):
    """Every uniform of a golden case (the pick's wave loop), and the first 1, 16 and 17 (a decode
    step's one uniform: the pick's path for at most 16 uniforms, and the boundary after it)."""
    g = np.load(GOLD)
    T, k, P, R, cap, V, masked = g["cases"][i]
    say(f"sampler golden case {i}: T={T} k={k} P={P} R={R} cap={cap} V={int(V)} masked={int(masked)} nu={nu}")
    samp = S.Sampling(T, int(k), P, R)
    u = g[f"s{i}_u"][:nu]
    got = S.pick(g[f"s{i}_logits"], samp, g[f"s{i}_ctx"].tolist(), u, cap or None)
    assert np.array_equal(got, g[f"s{i}_ids"][:nu])


@pytest.mark.parametrize("nu,offset", [(1, 0), (16, 0), (17, 0), (1, 1), (5, 3)])
def test_pick_few_uniforms_and_misaligned_logits(S, nu, offset):
    """V 262144 with masked blocks, few uniforms (the decode step's path, up to 16), and logits
    that start 4 or 12 bytes past a 16-byte boundary (the scalar-load path), against the oracle."""
    import torch
    V = 262144
    rng = np.random.default_rng(nu + 10 * offset)
    lg = (rng.standard_normal(V) * 3).astype(np.float32)
    for b in rng.choice(V // 64, 40, replace=False):
        lg[64 * b:64 * (b + 1)] = -np.inf
    ctx = rng.integers(0, V, 30).tolist()
    samp, osamp = S.Sampling(0.8, 50, 0.9, 1.1), SP.Sampling(0.8, 50, 0.9, 1.1)
    u = rng.random(nu).astype(np.float32)
    say(f"sampler few uniforms nu={nu} offset={offset}")
    buf = torch.zeros(V + 8, dtype=torch.float32, device="cuda")
    buf[offset:offset + V] = torch.from_numpy(lg).cuda()
    sm = S.Sampler(V, samp, ctx)
    ids = sm.pick_device(buf[offset:offset + V], torch.from_numpy(u).cuda())
    sm.check()
    assert np.array_equal(ids.cpu().numpy(), SP.pick(lg, osamp, ctx, u))


@pytest.mark.parametrize("V,T,k,P,R,cap,masked", [
    (3000, 1.0, 64, 0.95, 1.2, 0.0, 0), (262144, 0.8, 50, 0.9, 1.1, 0.0, 0),
    (262144, 1.0, 64, 1.0, 1.0, 30.0, 200), (1000, 1.0, 64, 1.0, 1.0, 0.0, 13),
    (40, 1.0, 64, 1.0, 1.0, 0.0, 0), (130, 0.5, 7, 0.7, 1.0, 0.0, 1)])
def test_candidates_and_picks_match_the_oracle(S, V, T, k, P, R, cap, masked):
    """The k candidate values and ids (the knock-out rounds, with -inf blocks and vocabularies
    smaller than k blocks: the rounds that take a position again) and the picks."""
    say(f"sampler vs oracle V={V} k={k} cap={cap} masked={masked}")
    rng = np.random.default_rng(V + k)
    lg = (rng.standard_normal(V) * 3).astype(np.float32)
    lg[rng.integers(0, V, 5)] = lg.max()                       # ties at the top
    if masked:
        for b in rng.choice(max(V // 64, 1), masked, replace=False):
            lg[64 * b:64 * (b + 1)] = -np.inf
    ctx = rng.integers(0, V, 30).tolist()
    samp = S.Sampling(T, k, P, R)
    osamp = SP.Sampling(T, k, P, R)
    u = ((np.arange(2000) + 0.5) / 2000).astype(np.float32)
    import torch
    sm = S.Sampler(V, samp, ctx, cap or None)
    ids = sm.pick_device(torch.from_numpy(lg).cuda(), torch.from_numpy(u).cuda())
    sm.check()
    vs, si = sm.candidates()
    vs0, si0 = SP.candidates(lg, osamp, ctx, cap or None)
    assert same_bits(vs, vs0) and np.array_equal(si, si0)
    assert np.array_equal(ids.cpu().numpy(), SP.pick(lg, osamp, ctx, u, cap or None))


@pytest.mark.parametrize("V,grid,k", [(262144, 1.0, 50), (262144, 0.0, 64), (5000, 0.5, 64), (70000, 2.0, 33)])
def test_heavy_ties_match_the_oracle(S, V, grid, k):
    """Logits on a coarse grid (grid 0: every logit equal), so that many blocks share the
    largest maxima and many candidates sit exactly at a selection's bound: the order among
    equal keys comes from the positions alone."""
    say(f"sampler heavy ties V={V} grid={grid} k={k}")
    rng = np.random.default_rng(V + k + 7)
    if grid:
        lg = (np.round(rng.standard_normal(V) * 3 / grid) * grid).astype(np.float32)
    else:
        lg = np.full(V, 1.5, np.float32)
    ctx = rng.integers(0, V, 30).tolist()
    samp, osamp = S.Sampling(1.0, k, 0.9, 1.1), SP.Sampling(1.0, k, 0.9, 1.1)
    u = ((np.arange(300) + 0.5) / 300).astype(np.float32)
    import torch
    sm = S.Sampler(V, samp, ctx)
    ids = sm.pick_device(torch.from_numpy(lg).cuda(), torch.from_numpy(u).cuda())
    sm.check()
    vs, si = sm.candidates()
    vs0, si0 = SP.candidates(lg, osamp, ctx, None)
    assert same_bits(vs, vs0) and np.array_equal(si, si0)
    assert np.array_equal(ids.cpu().numpy(), SP.pick(lg, osamp, ctx, u, None))


def test_lm_head_then_sample(S):
    """An int8 LM head (vocabulary 65536 x 1024) and the sampler on one stream: the ids are the
    oracle's pick over the oracle MM's logits."""
    import torch
    from opentpu_amd import mxu
    say("lm head + sample")
    rng = np.random.default_rng(3)
    N, K = 65536, 1024
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    x = rng.standard_normal((1, K)).astype(np.float32)
    rows, srows = Q.pack_int8x(W)
    w = mxu.QWeight.from_packed(rows, srows, "int8", K)
    samp = S.Sampling(0.9, 40, 0.95, 1.1)
    ctx = rng.integers(0, N, 20).tolist()
    sm = S.Sampler(N, samp, ctx)
    u = torch.from_numpy(((np.arange(512) + 0.5) / 512).astype(np.float32)).cuda()
    ids = S.lm_head_sample(x, w, sm, u).cpu().numpy()
    q, Sa, da = F.quantize_mx(x, 32)
    logits = MM.mm(q, Sa, da, rows, srows, "int8", K)[0]
    want = SP.pick(logits, SP.Sampling(0.9, 40, 0.95, 1.1), ctx, u.cpu().numpy())
    assert np.array_equal(ids, want)
    sm.after(int(ids[0]))
    assert float(sm.pa[int(ids[0])]) == float(np.float32(1.0) / np.float32(1.1))


def test_sampler_refusals(S):
    import torch
    from opentpu_amd import _lib as X
    say("sampler refusals")
    lg = torch.zeros(100, device="cuda")
    u = torch.zeros(4, device="cuda")
    ids = torch.zeros(4, dtype=torch.int32, device="cuda")
    st = torch.zeros(1, dtype=torch.int32, device="cuda")
    work = torch.zeros(4096, dtype=torch.uint8, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    with pytest.raises(X.OtpuError, match="top_k"):
        X.call("otpu_sample", X.ptr(lg), 100, None, None, 0.0, 65, 1.0, 1.0, X.ptr(u), 4, X.ptr(work),
               X.ptr(ids), X.ptr(st), s)
    with pytest.raises(X.OtpuError, match="together"):
        X.call("otpu_sample", X.ptr(lg), 100, X.ptr(lg), None, 0.0, 5, 1.0, 1.0, X.ptr(u), 4, X.ptr(work),
               X.ptr(ids), X.ptr(st), s)
    with pytest.raises(ValueError):
        S.Sampling(1.0, 65)
