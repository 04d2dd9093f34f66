"""The oracle's sampler (oracle/sampler.py): its exp2 and its picks against golden vectors
written from the reference (tests/golden/make_golden.py), and the properties the mathematics
fixes: exp2 exact at the integers and within its polynomial's error elsewhere; the picks' shares
of u in [0, 1) equal a float64 sampler's probabilities (the reference's own check,
tests/test_autodecode.py:289-322, restated); temperature 0 and top-1 are the argmax."""
import os

import numpy as np
import pytest

from oracle import fp32 as F
from oracle import sampler as SP

GOLD = os.path.join(os.path.dirname(__file__), "golden", "sampler.npz")


def test_exp2_matches_the_reference():
    g = np.load(GOLD)
    got = SP.exp2(g["exp2_x"])
    assert np.array_equal(F.bits(got), F.bits(g["exp2_y"]))


def test_exp2_by_the_mathematics():
    for i in range(-126, 128):
        assert SP.exp2(np.float32(i)) == np.float32(2.0 ** i)
    x = np.random.default_rng(0).uniform(-125, 127, 200000).astype(np.float32)
    y = SP.exp2(x).astype(np.float64)
    rel = np.abs(y / np.exp2(x.astype(np.float64)) - 1)
    assert rel.max() < 2.0 ** -21
    assert SP.exp2(np.float32(-126.5)) == 0 and SP.exp2(np.float32(128)) == np.inf
    assert SP.exp2(np.float32(np.nan)) == np.inf
    assert np.all(np.diff(SP.exp2(np.linspace(-10, 10, 100001).astype(np.float32))) >= 0)


def test_tree_sum_order():
    """64 partials folded pairwise (the first half plus the second): terms 16 and 48 meet
    before either meets term 0, so 1 + 2^-24 + 2^-24 is 1 + 2^-23; terms 32 and 48 meet term 0
    one at a time, and each 1 + 2^-24 rounds back to 1 (ties to even)."""
    a = np.zeros((1, 64), np.float32)
    a[0, 0] = 1.0
    a[0, 16] = a[0, 48] = 2.0 ** -24
    assert SP.tree_sum(a)[0] == np.float32(1 + 2.0 ** -23)
    b = np.zeros((1, 64), np.float32)
    b[0, 0] = 1.0
    b[0, 32] = 2.0 ** -24
    b[0, 16] = 2.0 ** -24
    assert SP.tree_sum(b)[0] == np.float32(1.0)
    assert SP.tree_sum(np.array([[1.0, 2.0 ** -24, 2.0 ** -24]], np.float32))[0] == 1.0


@pytest.mark.parametrize("i", range(10))
def test_picks_match_the_reference(i):
    g = np.load(GOLD)
    T, k, P, R, cap, V, masked = g["cases"][i]
    samp = SP.Sampling(T, int(k), P, R)
    got = SP.pick(g[f"s{i}_logits"], samp, g[f"s{i}_ctx"].tolist(), g[f"s{i}_u"], cap or None)
    assert np.array_equal(got, g[f"s{i}_ids"])


def _f64_sampler(lg, ctx, T, k, P, R):
    """Penalty, top-k (ties: lower id), softmax at temperature T, top-p (keep the first i with
    the sum before it below P), in float64."""
    w = lg.astype(np.float64)
    ix = np.unique(ctx)
    w[ix] = np.where(w[ix] > 0, w[ix] / np.float32(R), w[ix] * np.float32(R))
    idx = np.lexsort((np.arange(len(w)), -w))[:k]
    z = w[idx] / T
    p = np.exp(z - z[0])
    p /= p.sum()
    keep = min(len(p), int(np.searchsorted(np.cumsum(p), P)) + 1)
    return idx[:keep], p[:keep] / p[:keep].sum()


@pytest.mark.parametrize("T,k,P,R", [(0.7, 20, 0.8, 1.0), (1.5, 50, 1.0, 1.05),
                                     (3.0, 64, 0.95, 1.2), (2.0, 3, 1.0, 1.0), (2.5, 64, 0.5, 1.0)])
def test_picks_draw_from_the_distribution(T, k, P, R):
    rng = np.random.default_rng(int(10 * T) + k)
    V = 3000
    lg = (rng.standard_normal(V) * 3).astype(np.float32)
    ctx = [int(x) for x in rng.integers(0, V, 40)] + [int(np.argmax(lg))]
    idx, p = _f64_sampler(lg, ctx, T, k, P, R)
    n = 100000
    picks = SP.pick(lg, SP.Sampling(T, k, P, R), ctx, (np.arange(n) + 0.5) / n)
    ids, cnt = np.unique(picks, return_counts=True)
    assert set(ids) <= set(idx.tolist())
    share = dict(zip(ids.tolist(), cnt / n))
    assert max(abs(share.get(i, 0.0) - q) for i, q in zip(idx.tolist(), p)) < 1e-4


def test_greedy_is_the_argmax():
    rng = np.random.default_rng(1)
    lg = (rng.standard_normal(5000) * 2).astype(np.float32)
    lg[[17, 4000]] = lg.max() + 1                              # a tie: the lower id
    for samp in (SP.Sampling(0.0, 1), SP.Sampling(0.9, 1), SP.Sampling(1.0, 20, top_p=0.0)):
        assert SP.pick(lg, samp, [], np.array([0.01, 0.5, 0.99])).tolist() == [17, 17, 17]
