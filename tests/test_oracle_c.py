"""The C oracle (oracle/cpu_mm.c) against the numpy oracle, bit for bit: QACT in every mode,
MM for every format and flag, greedy argmax."""
import numpy as np
import pytest

from conftest import same_bits
from oracle import cpu
from oracle import fp32 as F
from oracle import mm as MM
from test_oracle_mm import CASES, mm_case


@pytest.mark.parametrize("g,row_mode", [(32, False), (32, True), (128, False), (8, False)])
def test_qact_same_as_numpy(g, row_mode):
    rng = np.random.default_rng(9)
    x = (rng.standard_normal((7, 1024)) * np.exp(rng.uniform(-9, 9, (7, 128, 1)))
         .repeat(8, 2).reshape(7, -1)).astype(np.float32)
    x[2] = 0
    x[3, 100] = np.float32(1e-40)
    q0, S0, d0 = F.quantize_mx(x, g, row_mode)
    q1, S1, d1 = cpu.qact(x, g, row_mode)
    assert np.array_equal(q0, q1) and same_bits(S0, S1) and np.array_equal(d0, d1)


@pytest.mark.parametrize("fmt,unit,rsc,k0,big", CASES)
def test_mm_same_as_numpy(fmt, unit, rsc, k0, big):
    c = mm_case(fmt, unit, rsc, k0, big, KB=4, M=5, N=33)
    flags = (MM.UNIT if unit else 0) | (MM.RSC if rsc else 0)
    a0, _ = MM.mm_acc(c["q"], c["da"], c["rows"], c["srows"], fmt, c["K"], flags=flags, k0=k0)
    y0 = MM.mm(c["q"], c["Sa"], c["da"], c["rows"], c["srows"], fmt, c["K"], flags=flags, k0=k0)
    y1, a1 = cpu.mm(c["q"], c["Sa"], c["da"], c["rows"], c["srows"], fmt, c["K"], flags=flags,
                    k0=k0, want_acc=True)
    assert np.array_equal(a0, a1) and same_bits(y0, y1)


def test_mm_flags_same_as_numpy():
    c = mm_case("int8", True, False, 0, False, KB=2, M=3, N=17)
    rng = np.random.default_rng(1)
    old = rng.standard_normal((3, 17)).astype(np.float32)
    alpha = rng.standard_normal(3).astype(np.float32)
    args = (c["q"], c["Sa"], c["da"], c["rows"], c["srows"], "int8", c["K"])
    for fl in (MM.UNIT | MM.ACC, MM.UNIT | MM.ACC | MM.ASCALE, MM.UNIT | MM.RMAX):
        r0 = MM.mm(*args, flags=fl, old=old, alpha=alpha)
        r1 = cpu.mm(*args, flags=fl, old=old, alpha=alpha)
        if fl & MM.RMAX:
            assert same_bits(r0[0], r1[0]) and same_bits(r0[1], r1[1])
        else:
            assert same_bits(r0, r1)


def test_argmax_same_as_numpy():
    rng = np.random.default_rng(2)
    for n in (1, 7, 1000, 262144):
        x = rng.standard_normal(n).astype(np.float32)
        x[rng.integers(0, n, 3)] = x.max()
        tok, best = cpu.argmax(x)
        assert tok == MM.greedy(x) and best == MM.best_word(x)
