"""The GPU kernels against the reference's own golden vectors directly (tests/golden/, written by
make_golden.py from the reference in the build container): QACT in MX, ROW and LO modes and
`quantize(x, axis=1)` (`opentpu/fp32.py:295-343`), the int8x and RSC packers
(`opentpu/quant.py:316-324`, `opentpu/runtime.py:66-76`), the int4x / fp4x6 / nvfp4 packers
(`opentpu/quant.py:325-400`) and the MXFP4 / NVFP4 imports (`opentpu/quant.py:1084-1182`), bit
for bit.  The oracle is checked against the same vectors in tests/test_golden.py."""
import os
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def words(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def ops():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    from opentpu_amd import _lib, fp32, quant
    _lib.load()
    return fp32, quant


@pytest.mark.parametrize("mode", ["mx", "row", "lo"])
def test_qact_matches_the_reference_golden(ops, mode):
    fp32, _ = ops
    g = np.load(os.path.join(GOLD, "fp32_quant.npz"))
    say("golden qact", mode)
    q, S, d = fp32.quantize_mx(g["qx"], 32, row_mode=mode == "row", lo=mode == "lo")
    assert np.array_equal(q, g[f"{mode}_q"])
    assert np.array_equal(words(S), words(g[f"{mode}_S"]))
    assert np.array_equal(d, g[f"{mode}_d"])


def test_quantize_rows_matches_the_reference_golden(ops):
    fp32, _ = ops
    g = np.load(os.path.join(GOLD, "fp32_quant.npz"))
    say("golden quantize axis=1")
    q, S = fp32.quantize(g["qx"], axis=1)
    assert np.array_equal(q, g["quantize_q"]) and np.array_equal(words(S), words(g["quantize_S"]))


def test_int8_packers_match_the_reference_golden(ops):
    _, quant = ops
    g = np.load(os.path.join(GOLD, "fp32_quant.npz"))
    say("golden int8x / rsc packers")
    rows, srows = quant.quantize_mxu(g["w8"], "int8")
    assert np.array_equal(rows, g["int8x_rows"]) and np.array_equal(srows, g["int8x_srows"])
    rows, srows = quant.quantize_mxu(g["w8"], "int8", rsc=True)
    assert np.array_equal(rows.view(np.int8), g["rsc_q"])
    assert np.array_equal(srows.view(np.uint32).reshape(-1), words(g["rsc_S"]))


@pytest.mark.parametrize("name", ["c2", "spread", "grid"])
@pytest.mark.parametrize("fmt", ["int4", "fp4", "nvfp4"])
def test_4bit_packers_match_the_reference_golden(ops, name, fmt):
    _, quant = ops
    g = np.load(os.path.join(GOLD, "nv_packer.npz" if fmt == "nvfp4" else "x4_packer.npz"))
    say("golden packer", fmt, name)
    rows, srows = quant.quantize_mxu(g[f"{name}_W"], fmt)
    want_s = g[f"{name}_{fmt}_srows"]
    assert np.array_equal(rows, g[f"{name}_{fmt}_rows"])
    assert np.array_equal(srows[:, :want_s.shape[1]], want_s)


@pytest.mark.parametrize("seed", [7, 8])
@pytest.mark.parametrize("want", [None, "nvfp4"])
def test_import_mxfp4_matches_the_reference_golden(ops, seed, want):
    _, quant = ops
    g = np.load(os.path.join(GOLD, "imports.npz"))
    tag = f"mx{seed}_{want or 'any'}"
    say("golden import mxfp4", seed, want)
    rows, srows, fmt = quant.import_mxfp4(g[f"mx{seed}_codes"], g[f"mx{seed}_e"], want=want)
    assert fmt == str(g[f"{tag}_fmt"])
    assert np.array_equal(rows, g[f"{tag}_rows"]) and np.array_equal(srows, g[f"{tag}_srows"])


@pytest.mark.parametrize("name", ["nv", "nvall"])
def test_import_nvfp4_matches_the_reference_golden(ops, name):
    _, quant = ops
    g = np.load(os.path.join(GOLD, "imports.npz"))
    say("golden import nvfp4", name)
    rows, srows = quant.import_nvfp4(g[f"{name}_codes"], g[f"{name}_s"], float(g[f"{name}_ts"]))
    assert np.array_equal(rows, g[f"{name}_rows"]) and np.array_equal(srows, g[f"{name}_srows"])
