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
several Samplings, contexts and soft caps -> `sampler.npz`;
and of the magic-seed `recip` (`opentpu/fp32.py:242-261`), which is not correctly rounded, so
no closed form fixes its bits, with the quantizers built on it -> `fp32_quant.npz`:
  * `recip` on every significand of [1, 2) (a SHA-256 of the 2^23 output words, and a strided
    sample of them), on 24 significands of every exponent field of both signs, and on the
    special values (zeros, denormals, 2^126 and past it, infinities, NaNs);
  * `quantize_mx(x, 32)` in MX, ROW and LO modes and `quantize(x, axis=1)`
    (`opentpu/fp32.py:295-343`) on rows drawn like the reference's `tests/test_mx.py:52-69`;
  * `quant.quantize_mxu(W, "int8")` (int8x, `opentpu/quant.py:316-324`) and the RSC rows
    `fp32.quantize_mx(W, 128, True)` (what `runtime.quantize_rows(W, 128, row=True)` stores,
    `opentpu/runtime.py:66-76`);
and of the checkpoint imports, whose per-block dw / m choice exactness alone does not fix ->
`imports.npz`: `quant.import_mxfp4` and `quant.import_nvfp4` (`opentpu/quant.py:1084-1182`)
on the inputs of tests/test_oracle_imports.py.

Run in the build container (the reference is at /root/reference and never travels):
    python tests/golden/make_golden.py [packers] [sampler] [fp32] [imports]   (default: all)
It imports the reference's `opentpu.quant`, `opentpu.fp32` and `opentpu.llm.generate` and writes
the files beside this one: the seeded inputs and the reference's outputs, nothing else.
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


RECIP_STRIDE = 509                                  # the stored sample of the 2^23 significands


def fp32_inputs():
    rng = np.random.default_rng(11)
    f = np.arange(256, dtype=np.uint32)
    m = rng.integers(0, 1 << 23, (256, 24), dtype=np.uint32)
    m[:, 0], m[:, 1], m[:, 2] = 0, 0x7FFFFF, 1
    u = ((f[:, None] << np.uint32(23)) | m).ravel()
    special = np.array([0, 1, 0x7FFFFF, 0x00800000, 0x00800001, 0x3F800000, 0x3F800001,
                        0x3FFFFFFF, 0x7E7FFFFF, 0x7E800000, 0x7E800001, 0x7F000000, 0x7F7FFFFF,
                        0x7F800000, 0x7F800001, 0x7FC00000, 0x7FFFFFFF], np.uint32)
    u = np.concatenate([u, special])
    out = {"recip_x": np.concatenate([u, u | np.uint32(0x80000000)]).view(np.float32)}
    # rows of the reference's QACT test distribution (a scale per 8 elements, e^U(-6, 6)),
    # rows with a scale per 32-group, and edge rows
    rows, K = 192, 256
    x8 = rng.standard_normal((rows // 2, K)) * np.exp(rng.uniform(-6, 6, (rows // 2, K // 8, 1))
                                                      ).repeat(8, 2).reshape(rows // 2, K)
    x32 = rng.standard_normal((rows // 2, K)) * np.exp(rng.uniform(-9, 9, (rows // 2, K // 32, 1))
                                                       ).repeat(32, 2).reshape(rows // 2, K)
    x = np.concatenate([x8, x32]).astype(np.float32)
    x[1, 8:16] = 0                                      # a zero sub-block
    x[2, 32:64] = 0                                     # a zero group: d 0
    x[3] = 0                                            # a zero row: S 0, q 0
    x[4, :] = np.float32(1e-39) * rng.standard_normal(K).astype(np.float32)   # denormals only
    x[5, 7] = np.float32(3.0e38)                        # a huge amax: recip flushes
    x[6, :] = np.float32(0.5) * (np.arange(K) % 5 - 2)  # exact ties of x * inv
    x[7, 100] = -np.float32(2.0 ** 126)
    x[8, :] = np.ldexp(np.float32(1), (np.arange(K) % 60 - 30)).astype(np.float32)
    out["qx"] = x
    W = (rng.standard_normal((24, 1024)) * 0.02).astype(np.float32)
    W[5] *= np.exp(rng.uniform(-8, 8, (8, 1))).repeat(128, 1).reshape(1024).astype(np.float32)
    W[6, 128:256] = 0
    W[7] = 0
    out["w8"] = W
    return out


def imports_inputs():
    out = {}
    for seed in (7, 8):
        rng = np.random.default_rng(seed)
        N, K = 6, 512
        codes = rng.integers(0, 16, (N, K)).astype(np.uint8)
        codes[2, 64:96] &= 8
        base = rng.integers(100, 150, (N, 1))
        e = base + rng.integers(0, 6, (N, K // 32))
        e[2, 2] = 3
        if seed == 8:
            e[:, 1] = base[:, 0] + 17                   # a block spanning 6..17: nvfp4
        out[f"mx{seed}_codes"], out[f"mx{seed}_e"] = codes, e.astype(np.uint8)
    rng = np.random.default_rng(8)
    N, K = 5, 256
    codes = rng.integers(0, 16, (N, K)).astype(np.uint8)
    s = rng.integers(1, 127, (N, K // 16)).astype(np.uint8)
    s[0, :] = rng.integers(1, 8, K // 16)
    s[1, 0] = 0x77
    s[2, 3] = 0
    s[4, :] = 0x60
    s[4, 0], s[4, 1], s[4, 2], s[4, 3] = 0x7E, 0x01, 0x03, 0x05
    out["nv_codes"], out["nv_s"], out["nv_ts"] = codes, s, np.float32(0.0123)
    rng = np.random.default_rng(3)
    codes = rng.integers(0, 16, (127, 128)).astype(np.uint8)
    s = np.zeros((127, 8), np.uint8)
    s[:, 0] = 0x7E
    s[:, 1] = np.arange(127)
    s[:, 2] = np.arange(127)[::-1]
    out["nvall_codes"], out["nvall_s"], out["nvall_ts"] = codes, s, np.float32(1.0)
    return out


def write_fp32():
    import hashlib
    from opentpu import fp32 as RF                     # noqa: E402  (the reference)
    from opentpu import quant as RQ                    # noqa: E402
    out = fp32_inputs()
    out["recip_y"] = RF.recip(out["recip_x"])
    sig = (np.uint32(127 << 23) | np.arange(1 << 23, dtype=np.uint32)).view(np.float32)
    ys = np.ascontiguousarray(RF.recip(sig), np.float32).view(np.uint32).astype("<u4")
    out["recip_sig_sha256"] = np.array(hashlib.sha256(ys.tobytes()).hexdigest())
    out["recip_sig_sample"] = ys[::RECIP_STRIDE].copy()
    x = out["qx"]
    for name, kw in (("mx", {}), ("row", {"row_mode": True}), ("lo", {"lo": True})):
        q, S, d = RF.quantize_mx(x, 32, **kw)
        out[f"{name}_q"], out[f"{name}_S"], out[f"{name}_d"] = q, S, d
    q, S = RF.quantize(x, axis=1)
    out["quantize_q"], out["quantize_S"] = q, S
    rows, srows = RQ.quantize_mxu(out["w8"], "int8")
    out["int8x_rows"], out["int8x_srows"] = rows, srows
    q, S, _ = RF.quantize_mx(out["w8"], 128, True)
    out["rsc_q"], out["rsc_S"] = q, S
    path = os.path.join(HERE, "fp32_quant.npz")
    np.savez_compressed(path, **out)
    print(path, os.path.getsize(path), "bytes")


def write_imports():
    from opentpu import quant as RQ                    # noqa: E402  (the reference)
    out = imports_inputs()
    for seed in (7, 8):
        for want in (None, "nvfp4"):
            rows, srows, fmt = RQ.import_mxfp4(out[f"mx{seed}_codes"], out[f"mx{seed}_e"].astype(np.int64),
                                               want=want)
            tag = f"mx{seed}_{want or 'any'}"
            out[f"{tag}_rows"], out[f"{tag}_srows"], out[f"{tag}_fmt"] = rows, srows, np.array(fmt)
    for name in ("nv", "nvall"):
        rows, srows = RQ.import_nvfp4(out[f"{name}_codes"], out[f"{name}_s"], float(out[f"{name}_ts"]))
        out[f"{name}_rows"], out[f"{name}_srows"] = rows, srows
    path = os.path.join(HERE, "imports.npz")
    np.savez_compressed(path, **out)
    print(path, os.path.getsize(path), "bytes")


def write_packers():
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


def write_sampler():
    from opentpu import fp32 as RF                     # noqa: E402  (the reference)
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


def main(which):
    sys.path.insert(0, REF)
    steps = {"packers": write_packers, "sampler": write_sampler, "fp32": write_fp32,
             "imports": write_imports}
    for w in which or list(steps):
        steps[w]()


if __name__ == "__main__":
    main(sys.argv[1:])
