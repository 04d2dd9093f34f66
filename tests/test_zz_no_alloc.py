"""The entry point that allocates nothing (otpu_sample_static: the sampler's work area in the
library's static device array) against otpu_sample with a caller's work area, through the C ABI,
on two calls in a row (the second with a smaller vocabulary, so the array holds the first call's
contents when it starts), and its refusal of a vocabulary past the array's size."""
import sys

import numpy as np
import pytest

from oracle import sampler as SP

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


def _case(rng, V):
    lg = (rng.standard_normal(V) * 3).astype(np.float32)
    for b in rng.choice(max(V // 64, 1), min(20, max(V // 64 - 1, 0)), replace=False):
        lg[64 * b:64 * (b + 1)] = -np.inf
    return lg


def test_sample_static_matches_sample(X):
    import torch
    from opentpu_amd import sampler as S
    rng = np.random.default_rng(21)
    samp = S.Sampling(0.8, 50, 0.9, 1.1)
    for V, nu in ((262144, 17), (5000, 3)):
        say(f"sample_static V={V} nu={nu}")
        lg = _case(rng, V)
        ctx = rng.integers(0, V, 30).tolist()
        u = rng.random(nu).astype(np.float32)
        sm = S.Sampler(V, samp, ctx)                      # the penalty rows and a work area
        lgd, ud = torch.from_numpy(lg).cuda(), torch.from_numpy(u).cuda()
        ids_w = torch.full((nu,), -1, dtype=torch.int32, device="cuda")
        ids_s = torch.full((nu,), -2, dtype=torch.int32, device="cuda")
        st_w = torch.full((1,), 7, dtype=torch.int32, device="cuda")
        st_s = torch.full((1,), 7, dtype=torch.int32, device="cuda")
        args = (X.ptr(lgd), V, X.ptr(sm.pa), X.ptr(sm.pb), 0.0, samp.k, float(np.float32(samp.itemp)),
                float(np.float32(samp.top_p)), X.ptr(ud), nu)
        X.call("otpu_sample", *args, X.ptr(sm.work), X.ptr(ids_w), X.ptr(st_w), X.stream())
        X.call("otpu_sample_static", *args, X.ptr(ids_s), X.ptr(st_s), X.stream())
        a, b = ids_s.cpu().numpy(), ids_w.cpu().numpy()
        assert np.array_equal(a, b) and int(st_s.item()) == int(st_w.item()) == 0
        assert np.array_equal(a, SP.pick(lg, SP.Sampling(0.8, 50, 0.9, 1.1), ctx, u))


def test_sample_static_refuses_a_larger_vocabulary(X):
    p = 256
    with pytest.raises(X.OtpuError, match="static"):
        X.call("otpu_sample_static", p, 262145, None, None, 0.0, 50, 1.0, 1.0, p, 1, p, p, X.stream())
