"""Long rows: MM's K past what one register walk of the decode GEMV holds (int8 rows of more
than 8192 bytes are walked in segments), up to the reference's field limit (KB < 256 blocks,
`opentpu/isa.py:521-523`; every board target's ACT_BLOCKS = 128 gives K = 16384,
`targets/bcu1525.toml:17`).  Each case against the C oracle bit for bit: outputs, exact
accumulators, ACC, the LM head's token, the GEMM (M >= 16) and the QACT prologue of
otpu_mm_qin over rows of up to 16384 columns."""
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
    from opentpu_amd import _lib, mxu
    _lib.load()
    return _lib, mxu


def spread(rng, M, K, s, g):
    return (rng.standard_normal((M, K)) * np.exp(rng.uniform(-s, s, (M, K // g, 1)))
            .repeat(g, 2).reshape(M, K)).astype(np.float32)


def weights(rng, fmt, rsc, N, K):
    W = (spread(rng, N, K, 1.5, 128) * 0.02).astype(np.float32)
    if fmt == "int8":
        return Q.pack_rsc(W) if rsc else Q.pack_int8x(W)
    return Q.quantize_mxu(W, fmt)


LONG = [("int8", True, 12288), ("int8", False, 12288), ("int8", True, 16384), ("int8", False, 16384),
        ("int8", True, 32640), ("int4", False, 16384), ("fp4", False, 16384), ("nvfp4", False, 16384),
        ("int4", False, 32512)]


@pytest.mark.parametrize("fmt,rsc,K", LONG)
def test_gemv_long_rows(ops, fmt, rsc, K):
    """M 1-4 (one and two activation rows a register walk), outputs and exact accumulators."""
    _, mxu = ops
    rng = np.random.default_rng(K + len(fmt) + rsc)
    N = 203
    rows, srows = weights(rng, fmt, rsc, N, K)
    flags = MM.RSC if rsc else 0
    for M in (1, 2, 3, 4):
        x = spread(rng, M, K, 2.0, 32)
        q, Sa, da = F.quantize_mx(x, 32)
        say("gemv long K", fmt, rsc, K, M)
        want, acc0 = OC.mm(q, Sa, da, rows, srows, fmt, K, flags=flags, want_acc=True)
        assert same_bits(mxu.mm(q, Sa, da, rows, srows, fmt, K, rsc=rsc), want)
        assert np.array_equal(mxu.mm_acc(q, da, rows, srows, fmt, K, rsc=rsc), acc0)


def test_gemv_long_rows_acc_and_k0(ops):
    """ACC onto an old output, and a column slice of the scale rows (k0) of a wider matrix."""
    _, mxu = ops
    rng = np.random.default_rng(77)
    N, K, Kw = 150, 12288, 16384
    rows, srows = weights(rng, "int8", False, N, Kw)
    k0 = 16                                         # blocks 16 .. 111 of the 128
    part = np.ascontiguousarray(rows[:, 128 * k0:128 * k0 + K])
    x = spread(rng, 3, K, 2.0, 32)
    q, Sa, da = F.quantize_mx(x, 32)
    old = rng.standard_normal((3, N)).astype(np.float32)
    say("gemv long K acc k0")
    want = OC.mm(q, Sa, da, part, srows, "int8", K, flags=MM.ACC, k0=k0, old=old)
    got = mxu.mm(q, Sa, da, part, srows, "int8", K, k0=k0, acc=old)
    assert same_bits(got, want)


def test_lm_head_long_rows(ops):
    _, mxu = ops
    rng = np.random.default_rng(5)
    N, K = 3000, 16384
    rows, srows = weights(rng, "int8", True, N, K)
    x = spread(rng, 1, K, 2.0, 32)
    q, Sa, da = F.quantize_mx(x, 32)
    say("lm head long K")
    tok, logits, _ = mxu.lm_head_argmax(q, Sa, da, rows, srows, "int8", K, rsc=True)
    want = OC.mm(q, Sa, da, rows, srows, "int8", K, flags=MM.RSC)[0]
    assert same_bits(logits, want) and tok == OC.argmax(want)[0]


@pytest.mark.parametrize("fmt,rsc,row_mode", [("int8", True, True), ("int8", True, False), ("int8", False, False)])
def test_gemm_long_rows(ops, fmt, rsc, row_mode):
    """M >= 16 (the int8 MFMA GEMM) at K 16384: one activation plane (ROW x RSC), several (MX),
    and per-block weight offsets (int8x)."""
    _, mxu = ops
    rng = np.random.default_rng(16 + rsc + row_mode)
    M, N, K = 40, 160, 16384
    rows, srows = weights(rng, fmt, rsc, N, K)
    x = spread(rng, M, K, 2.0, 32)
    q, Sa, da = F.quantize_mx(x, 32, row_mode=row_mode)
    say("gemm long K", fmt, rsc, row_mode)
    want = OC.mm(q, Sa, da, rows, srows, fmt, K, flags=MM.RSC if rsc else 0)
    assert same_bits(mxu.mm(q, Sa, da, rows, srows, fmt, K, rsc=rsc), want)


@pytest.mark.parametrize("fmt,K", [("int8", 6144), ("int8", 8192), ("int8", 12288), ("int8", 16384),
                                   ("int4", 8192), ("int4", 12288), ("int4", 16384), ("fp4", 16384)])
def test_mm_qin_long_rows(ops, fmt, K):
    """otpu_mm_qin (QACT of the fp32 row in the prologue, then MM) over rows of up to 16384
    columns: the oracle's QACT then the C oracle's MM."""
    import torch
    X, _ = ops
    rng = np.random.default_rng(K + len(fmt))
    N = 180
    rows, srows = weights(rng, fmt, False, N, K)
    x = spread(rng, 1, K, 3.0, 32)
    q, Sa, da = F.quantize_mx(x, 32)
    want = OC.mm(q, Sa, da, rows, srows, fmt, K)
    xd = torch.from_numpy(x).cuda()
    rd, sd = torch.from_numpy(rows).cuda(), torch.from_numpy(srows).cuda()
    out = torch.empty((1, N), dtype=torch.float32, device="cuda")
    say("mm_qin long K", fmt, K)
    X.call("otpu_mm_qin", X.ptr(xd), None, None, None, 1, K, K, K, X.ptr(rd), rd.shape[1], X.ptr(sd), sd.shape[1], N,
           X.FMT[fmt], 0, 0, X.ptr(out), N, N, X.stream())
    assert same_bits(out.cpu().numpy(), want)


def test_long_rows_refusals(ops):
    """K of 256 blocks or more is refused, as the reference's MM field refuses it."""
    X, mxu = ops
    rng = np.random.default_rng(1)
    K = 32768
    rows, srows = weights(rng, "int8", True, 16, K)
    q, Sa, da = F.quantize_mx(spread(rng, 1, K, 1.0, 32), 32)
    with pytest.raises(X.OtpuError, match="at most"):
        mxu.mm(q, Sa, da, rows, srows, "int8", K, rsc=True)
