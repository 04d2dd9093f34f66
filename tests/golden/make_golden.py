"""Write the golden vectors of the functions on this path that no closed form, known answer
or scalar model pins: the reference's 4-bit weight packers, whose float64 scale searches keep
the first of equal squared errors in numpy's summation order:
  * int4x / fp4x6 (`opentpu/quant.py:325-367`, `quantize_mxu(W, "int4" | "fp4")`) ->
    `x4_packer.npz`;
  * nvfp4 with a per-row scale (`opentpu/quant.py:368-400`, `quantize_mxu(W, "nvfp4")`) ->
    `nv_packer.npz`;
and of the sampled decode's pick, whose fp32 exp2 polynomial and sum orders no closed form
fixes: the machine's exp2 (`opentpu/fp32.py:187-202`) on a grid of inputs, and
`generate.reference_pick` (`opentpu/llm/generate.py:492-557`) over thousands of uniforms for
several Samplings, contexts and soft caps -> `sampler.npz`.

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


# (temperature, top_k, top_p, repetition_penalty, soft cap, vocabulary, masked blocks)
SAMPLER_CASES = [
    (0.7, 20, 0.8, 1.0, 0.0, 3000, 0), (0.1, 50, 1.0, 1.05, 0.0, 3000, 0),
    (1.0, 64, 0.95, 1.2, 0.0, 3000, 0), (2.0, 3, 1.0, 1.0, 0.0, 3000, 0),
    (0.7, 20, 0.0, 1.0, 0.0, 3000, 0), (1.0, 64, 1e-40, 1.2, 0.0, 3000, 0),
    (0.0, 1, 1.0, 1.1, 0.0, 3000, 0), (0.8, 40, 0.9, 1.0, 30.0, 5000, 0),
    (1.3, 64, 1.0, 1.3, 0.0, 1000, 12), (0.6, 8, 0.5, 1.0, 0.0, 151936, 0),
]


def sampler_inputs():
    rng = np.random.default_rng(5)
    x = np.concatenate([np.linspace(-130, 130, 20001), rng.uniform(-140, 140, 20000),
                        rng.standard_normal(5000) * 1e-3, [0.0, -0.0, np.inf, -np.inf, np.nan,
                                                           1e-40, -1e-40, -126.0, 128.0, 127.99999]])
    out = {"exp2_x": x.astype(np.float32)}
    for i, (T, k, P, R, cap, V, masked) in enumerate(SAMPLER_CASES):
        lg = (rng.standard_normal(V) * 3).astype(np.float32)
        if masked:                                  # whole blocks of -inf (a masked vocabulary)
            for b in rng.choice(V // 64, masked, replace=False):
                lg[64 * b:64 * (b + 1)] = -np.inf
        ctx = np.concatenate([rng.integers(0, V, 40), [int(np.argmax(lg))]]).astype(np.int64)
        out[f"s{i}_logits"], out[f"s{i}_ctx"] = lg, ctx
        out[f"s{i}_u"] = ((np.arange(4096) + 0.5) / 4096).astype(np.float32)
    return out


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
    from opentpu import fp32 as RF                     # noqa: E402
    from opentpu.llm import generate as RG             # noqa: E402
    out = sampler_inputs()
    out["exp2_y"] = RF.exp2(out["exp2_x"])
    for i, (T, k, P, R, cap, V, masked) in enumerate(SAMPLER_CASES):
        samp = RG.Sampling(T, k, P, R)
        out[f"s{i}_ids"] = RG.reference_pick(out[f"s{i}_logits"], samp, out[f"s{i}_ctx"].tolist(),
                                             out[f"s{i}_u"], 1, cap or None).astype(np.int64)
    out["cases"] = np.array(SAMPLER_CASES, np.float64)
    path = os.path.join(HERE, "sampler.npz")
    np.savez_compressed(path, **out)
    print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
