"""The reference-side binding the repository's integration guide shows (the ctypes module a
maintainer would add to openTPU), run as written with the library path filled in: its argument
lists against include/otpu.h's prototypes and its ABI check (CPU), then its quantize_mx and mm
against the oracle bit for bit (GPU; `opentpu/fp32.py:321-343`, `opentpu/isasim.py:749-910`)."""
import os
import re

import numpy as np
import pytest

from opentpu_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def example_source():
    doc = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    sec = doc[doc.index("## The reference-side binding"):]
    src = sec[sec.index("```python\n") + len("```python\n"):]
    src = src[:src.index("```")]
    assert '"/path/to/opentpu_amd/libotpu_amd.so"' in src
    return src.replace('"/path/to/opentpu_amd/libotpu_amd.so"', repr(_lib.LIB_PATH))


def load_example():
    ns = {"__name__": "hip_mxu_example"}
    exec(compile(example_source(), "the integration guide's binding example", "exec"), ns)
    return ns


def prototypes():
    src = open(os.path.join(ROOT, "include", "otpu.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return {m.group(1): [a.strip() for a in m.group(2).split(",") if a.strip()]
            for m in re.finditer(r"int\s+(otpu_\w+)\s*\(([^)]*)\)\s*;", src)}


@pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH), reason="libotpu_amd.so not built")
def test_example_binds_the_header():
    """Every argtypes list the example sets has the header's length, with 64-bit integers where
    the header has int64_t and pointers where it has pointers."""
    import ctypes as C
    ns = load_example()
    lib, protos = ns["_lib"], prototypes()
    bound = 0
    for name in ("otpu_mm", "otpu_qact"):
        types, params = getattr(lib, name).argtypes, protos[name]
        assert len(types) == len(params), name
        for t, p in zip(types, params):
            if "*" in p or "otpu_stream_t" in p:
                assert t is C.c_void_p, (name, p)
            elif p.startswith("int64_t"):
                assert t is C.c_int64, (name, p)
            else:
                assert t is C.c_int, (name, p)
        bound += 1
    assert bound == 2 and lib.otpu_version() == _lib.ABI_VERSION


@pytest.mark.gpu
def test_example_matches_the_oracle():
    """The example's quantize_mx (MX and ROW) and mm (int4x weights, then ACC on its output) on
    the GPU: the oracle's bytes and words bit for bit."""
    import torch
    from conftest import same_bits
    from oracle import cpu as OC
    from oracle import formats as Q
    from oracle import fp32 as F
    from oracle import mm as MM
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    ns = load_example()
    rng = np.random.default_rng(31)
    M, K, N = 5, 512, 96
    x = (rng.standard_normal((M, K)) * np.exp(rng.uniform(-3, 3, (M, K // 32, 1))).repeat(32, 2).reshape(M, K))
    x = x.astype(np.float32)
    for row_mode in (False, True):
        q, S, d = ns["quantize_mx"](torch.from_numpy(x).cuda(), 32, row_mode)
        wq, wS, wd = F.quantize_mx(x, 32, row_mode=row_mode)
        assert np.array_equal(q.cpu().numpy(), wq) and same_bits(S.cpu().numpy(), wS)
        assert np.array_equal(d.cpu().numpy(), wd)
    q, S, d = F.quantize_mx(x, 32)
    rows, srows = Q.quantize_mxu((rng.standard_normal((N, K)) * 0.02).astype(np.float32), "int4")
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    got = ns["mm"](dev(q), dev(S), dev(d), dev(rows), dev(srows), "int4", K)
    want = OC.mm(q, S, d, rows, srows, "int4", K)
    assert same_bits(got.cpu().numpy(), want)
    got2 = ns["mm"](dev(q), dev(S), dev(d), dev(rows), dev(srows), "int4", K, acc=True, out=got)
    assert same_bits(got2.cpu().numpy(), OC.mm(q, S, d, rows, srows, "int4", K, flags=MM.ACC, old=want))
