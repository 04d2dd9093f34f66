"""Write the golden vectors of the functions on this path that no closed form, known answer
or scalar model pins: the reference's 4-bit weight packers, whose float64 scale searches keep
the first of equal squared errors in numpy's summation order:
  * int4x / fp4x6 (`opentpu/quant.py:325-367`, `quantize_mxu(W, "int4" | "fp4")`) ->
    `x4_packer.npz`;
  * nvfp4 with a per-row scale (`opentpu/quant.py:368-400`, `quantize_mxu(W, "nvfp4")`) ->
    `nv_packer.npz`.

Run once, in the build container (the reference is at /root/reference and never travels):
    python tests/golden/make_golden.py
It imports `opentpu.quant` from the reference and writes the files beside this one: the inputs
(seeded fp32 weights) and the packed element and scale rows for each format.
"""
import os
import sys

import numpy as np

REF = os.environ.get("OTPU_REFERENCE", "/root/reference")
HERE = os.path.dirname(os.path.abspath(__file__))


def inputs():
    rng = np.random.default_rng(2)
    # c2-shaped rows (K = 2048, N(0, 0.02)), a zero block and a zero sub-block
    c2 = (rng.standard_normal((24, 2048)) * 0.02).astype(np.float32)
    c2[3, 256:384] = 0
    c2[5, 32:64] = 0
    # rows with log-normal scales per 32 (offsets past the multiplier range), K = 640
    sp = (rng.standard_normal((16, 640)) * np.exp(3.0 * rng.standard_normal((16, 20, 1)))
          .repeat(32, 2).reshape(16, 640) * 0.02).astype(np.float32)
    sp[7, :128] = 0
    sp[9] = 0                                                   # an all-zero row: Sw = 1
    # a regular grid: exact values, where candidates give equal errors (the tie rule)
    grid = (np.arange(8 * 256).reshape(8, 256) % 15 - 7).astype(np.float32) * np.float32(0.25)
    return {"c2": c2, "spread": sp, "grid": grid}


def main():
    sys.path.insert(0, REF)
    from opentpu import quant as RQ                    # noqa: E402  (the reference)
    for fname, fmts in (("x4_packer.npz", ("int4", "fp4")), ("nv_packer.npz", ("nvfp4",))):
        out = {}
        for name, W in inputs().items():
            out[f"{name}_W"] = W
            for fmt in fmts:
                rows, srows = RQ.quantize_mxu(W, fmt)
                out[f"{name}_{fmt}_rows"] = rows
                out[f"{name}_{fmt}_srows"] = srows
        path = os.path.join(HERE, fname)
        np.savez_compressed(path, **out)
        print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
