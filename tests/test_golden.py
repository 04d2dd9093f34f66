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
