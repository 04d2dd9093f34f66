"""The oracle's int4x / fp4x6 and nvfp4 packers against golden vectors written from the reference
(tests/golden/make_golden.py, `opentpu/quant.py:325-400`): bit-identical element and scale rows."""
import os

import numpy as np
import pytest

from oracle import formats as Q

GOLD = os.path.join(os.path.dirname(__file__), "golden", "x4_packer.npz")
GOLD_NV = os.path.join(os.path.dirname(__file__), "golden", "nv_packer.npz")


@pytest.mark.parametrize("name", ["c2", "spread", "grid"])
@pytest.mark.parametrize("fmt", ["int4", "fp4"])
def test_x4_packer_matches_the_reference(name, fmt):
    g = np.load(GOLD)
    rows, srows = Q.pack_x4(g[f"{name}_W"], fmt)
    assert np.array_equal(rows, g[f"{name}_{fmt}_rows"])
    assert np.array_equal(srows, g[f"{name}_{fmt}_srows"])


def test_golden_layouts():
    g = np.load(GOLD)
    for name in ("c2", "spread", "grid"):
        W = g[f"{name}_W"]
        K = W.shape[1]
        for fmt in ("int4", "fp4"):
            assert g[f"{name}_{fmt}_rows"].shape == (W.shape[0], Q.row_bytes(K, fmt))
            assert g[f"{name}_{fmt}_srows"].shape == (W.shape[0], Q.scale_bytes(K, fmt))
            _, _, m = Q.unpack_scales(g[f"{name}_{fmt}_srows"], fmt, K // Q.D)
            assert m.min() >= 1 and m.max() <= Q.MMAX


@pytest.mark.parametrize("name", ["c2", "spread", "grid"])
def test_nv_packer_matches_the_reference(name):
    g = np.load(GOLD_NV)
    rows, srows = Q.pack_nv(g[f"{name}_W"])
    assert np.array_equal(rows, g[f"{name}_nvfp4_rows"])
    assert np.array_equal(srows, g[f"{name}_nvfp4_srows"])
    assert not np.any(srows[:, 16:] & 0x80)                    # unsigned E4M3 scales, no NaN
    assert not np.any(srows[:, 16:] == 0x7F)


# ------------------------------------------------------------------ recip and the quantizers
# Golden vectors of the reference's `fp32.recip` / `quantize_mx` / `quantize` and
# `quant.quantize_mxu(W, "int8")` (tests/golden/make_golden.py fp32 -> fp32_quant.npz).  recip's
# magic-seed iteration is not correctly rounded, so only the reference's own outputs fix its
# bits: both restatements (oracle/fp32.py and oracle/cpu_mm.c) are checked on every significand
# of [1, 2) through a SHA-256 of the 2^23 output words, on every exponent field and on the
# special values.
import hashlib  # noqa: E402

from oracle import cpu  # noqa: E402
from oracle import fp32 as F  # noqa: E402
from oracle import imports as IM  # noqa: E402

GOLD_FP = os.path.join(os.path.dirname(__file__), "golden", "fp32_quant.npz")
GOLD_IM = os.path.join(os.path.dirname(__file__), "golden", "imports.npz")
RECIP_STRIDE = 509                       # the golden sample's stride (make_golden.RECIP_STRIDE)
RECIP = {"numpy": F.recip, "c": cpu.recip}


def _words(y):
    return np.ascontiguousarray(y, np.float32).view(np.uint32)


@pytest.mark.parametrize("impl", ["numpy", "c"])
def test_recip_every_significand_matches_the_reference(impl):
    g = np.load(GOLD_FP)
    sig = (np.uint32(127 << 23) | np.arange(1 << 23, dtype=np.uint32)).view(np.float32)
    y = _words(RECIP[impl](sig))
    bad = np.nonzero(y[::RECIP_STRIDE] != g["recip_sig_sample"])[0]
    assert bad.size == 0, f"recip differs first at significand {bad[0] * RECIP_STRIDE:#x}"
    assert hashlib.sha256(y.astype("<u4").tobytes()).hexdigest() == str(g["recip_sig_sha256"])


@pytest.mark.parametrize("impl", ["numpy", "c"])
def test_recip_every_exponent_and_the_specials_match_the_reference(impl):
    g = np.load(GOLD_FP)
    y = _words(RECIP[impl](g["recip_x"]))
    bad = np.nonzero(y != _words(g["recip_y"]))[0]
    assert bad.size == 0, f"recip({_words(g['recip_x'])[bad[0]]:#010x}) differs"


def test_recip_golden_is_sensitive_to_the_seed():
    """A recip whose magic constant is one off (a plausible slip) fails the golden hash."""
    g = np.load(GOLD_FP)
    sig = (np.uint32(127 << 23) | np.arange(1 << 23, dtype=np.uint32)).view(np.float32)
    old = F.RECIP_MAGIC
    try:
        F.RECIP_MAGIC = old - 1
        y = _words(F.recip(sig))
    finally:
        F.RECIP_MAGIC = old
    assert hashlib.sha256(y.astype("<u4").tobytes()).hexdigest() != str(g["recip_sig_sha256"])
    assert not np.array_equal(y[::RECIP_STRIDE], g["recip_sig_sample"])


@pytest.mark.parametrize("mode", ["mx", "row", "lo"])
def test_quantize_mx_matches_the_reference(mode):
    g = np.load(GOLD_FP)
    kw = {"row": {"row_mode": True}, "lo": {"lo": True}}.get(mode, {})
    q, S, d = F.quantize_mx(g["qx"], 32, **kw)
    assert np.array_equal(q, g[f"{mode}_q"])
    assert np.array_equal(_words(S), _words(g[f"{mode}_S"]))
    assert np.array_equal(d, g[f"{mode}_d"])
    if mode != "lo":                                   # the C restatement (MX and ROW)
        q, S, d = cpu.qact(g["qx"], 32, mode == "row")
        assert np.array_equal(q, g[f"{mode}_q"])
        assert np.array_equal(_words(S), _words(g[f"{mode}_S"]))
        assert np.array_equal(d, g[f"{mode}_d"])


def test_quantize_rows_matches_the_reference():
    g = np.load(GOLD_FP)
    q, S = F.quantize_rows(g["qx"])
    assert np.array_equal(q, g["quantize_q"])
    assert np.array_equal(_words(S), _words(g["quantize_S"]))


def test_int8x_and_rsc_rows_match_the_reference():
    g = np.load(GOLD_FP)
    rows, srows = Q.pack_int8x(g["w8"])
    assert np.array_equal(rows, g["int8x_rows"]) and np.array_equal(srows, g["int8x_srows"])
    rows, srows = Q.pack_rsc(g["w8"])
    assert np.array_equal(rows.view(np.int8), g["rsc_q"])
    assert np.array_equal(srows.view(np.uint32).reshape(-1), _words(g["rsc_S"]))


# ------------------------------------------------------------------------ checkpoint imports
@pytest.mark.parametrize("seed", [7, 8])
@pytest.mark.parametrize("want", [None, "nvfp4"])
def test_import_mxfp4_matches_the_reference(seed, want):
    g = np.load(GOLD_IM)
    tag = f"mx{seed}_{want or 'any'}"
    rows, srows, fmt = IM.import_mxfp4(g[f"mx{seed}_codes"], g[f"mx{seed}_e"].astype(np.int64), want=want)
    assert fmt == str(g[f"{tag}_fmt"])
    assert np.array_equal(rows, g[f"{tag}_rows"]) and np.array_equal(srows, g[f"{tag}_srows"])


@pytest.mark.parametrize("name", ["nv", "nvall"])
def test_import_nvfp4_matches_the_reference(name):
    g = np.load(GOLD_IM)
    rows, srows = IM.import_nvfp4(g[f"{name}_codes"], g[f"{name}_s"], float(g[f"{name}_ts"]))
    assert np.array_equal(rows, g[f"{name}_rows"]) and np.array_equal(srows, g[f"{name}_srows"])
