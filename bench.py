"""Benchmark of the quantized-linear hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Headline (the metric's quoted configuration, c2): the 4-bit group-32 decode GEMV, weights N=6144 x K=2048
int4x (opentpu/quant.py int4: nibbles + per-row Sw, per-block dw, per-32 multipliers m, from
N(0, 0.02)), one int8 MX activation row from N(0, 1).  A step is one launch of B independent
such GEMVs (B weight sets resident in HBM, > 512 MB in total, so no step is served from the
256 MB Infinity Cache); value = algorithmic bytes moved per second (GB/s, 1e9).

The same JSON line carries the other configs' figures under "extra": c1 int8 GEMV, c5 LM head
+ greedy argmax, c3 prefill GEMM (int8 TOPS), each timed with HIP events on the stream the
kernels run on; and the CPU baseline (the C oracle, OpenMP, on this host) on a bounded sample.
"""
from __future__ import annotations

import argparse
import contextlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0            # MI355X HBM3E, vendor figure
INT8_PEAK_TOPS = 5000.0          # MI355X dense int8 MFMA, vendor figure


def c2_bytes(N=6144, K=2048):
    """Algorithmic bytes of one 4-bit GEMV: elements N*K/2, scale rows 72 B/row, activation
    K int8 + K/32 offsets + Sa, output 4 B/row."""
    return N * K // 2 + N * (8 + 8 * ((K // 128 + 1) // 2)) + K + K // 32 + 4 + 4 * N


def c1_bytes(N=4096, K=1024):
    return N * K + 4 * N + K + K // 32 + 4 + 4 * N


def c5_bytes(N=262144, K=2560):
    return N * K + 4 * N + K + K // 32 + 4 + 4 * N


def timed(fn, steps, warmup, stream, graph=True):
    """ms per call of fn (which queues HIP kernels on the current stream).  With graph=True the
    `steps` calls are captured once in a HIP graph and the replay is timed with HIP events on
    the stream the kernels run on, so host launch overhead does not pad short kernels."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    if graph:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(steps):
                fn()
        g.replay()
        torch.cuda.synchronize()
        s = torch.cuda.current_stream()
        e0.record(s)
        g.replay()
        e1.record(s)
        torch.cuda.synchronize()
        del g
        return e0.elapsed_time(e1) / steps
    e0.record(stream)
    for _ in range(steps):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps          # ms per step


def make_batch(fmt, B, N, K, seed, rsc=False):
    """B independent weight sets and activation rows, generated and packed on the GPU."""
    import torch

    from opentpu_amd import fp32, quant
    gen = torch.Generator(device="cuda").manual_seed(seed)
    rows = srows = None
    for b in range(B):
        W = torch.randn((N, K), generator=gen, device="cuda") * 0.02
        r, s = quant.quantize_mxu(W, fmt, rsc=rsc)
        if rows is None:
            rows = torch.empty((B,) + tuple(r.shape), dtype=torch.uint8, device="cuda")
            srows = torch.empty((B,) + tuple(s.shape), dtype=torch.uint8, device="cuda")
        rows[b].copy_(r)
        srows[b].copy_(s)
        del W, r, s
    x = torch.randn((B, K), generator=gen, device="cuda")
    q, Sa, da = fp32.quantize_mx(x, 32)
    return rows, srows, q, Sa, da


def batched_gemv(fmt, B, N, K, seed, steps, warmup, rsc=False):
    import torch

    from opentpu_amd import _lib as X
    rows, srows, q, Sa, da = make_batch(fmt, B, N, K, seed, rsc)
    out = torch.empty((B, N), dtype=torch.float32, device="cuda")
    rs, srs = rows.shape[2], srows.shape[2]
    fl = X.RSC if rsc else 0

    def step():
        X.call("otpu_mm_batched", B, X.ptr(q), K, K, X.ptr(Sa), 1, X.ptr(da), K // 32, K // 32, 1, K,
               X.ptr(rows), rs, N * rs, X.ptr(srows), srs, N * srs, N, X.FMT[fmt], fl, 0, X.ptr(out), N, N, X.stream())
    ms = timed(step, steps, warmup, torch.cuda.current_stream())
    return ms, (rows, srows, q, Sa, da, out)


def single_gemv_ms(fmt, batch, N, K, steps, rsc=False):
    """One GEMV per launch, each launch on the next of the batch's weight sets (more than the
    Infinity Cache holds in all, so every launch streams its weights from HBM)."""
    import torch

    from opentpu_amd import _lib as X
    rows, srows, q, Sa, da = batch[:5]
    B = rows.shape[0]
    out = torch.empty((1, N), dtype=torch.float32, device="cuda")
    it = [0]

    def step():
        b = it[0] % B
        it[0] += 1
        X.call("otpu_mm", X.ptr(q[b]), K, X.ptr(Sa[b]), X.ptr(da[b]), K // 32, 1, K, X.ptr(rows[b]), rows.shape[2],
               X.ptr(srows[b]), srows.shape[2], N, X.FMT[fmt], X.RSC if rsc else 0, 0, None, X.ptr(out), N, None, X.stream())
    return timed(step, steps, 3, torch.cuda.current_stream())


def lm_head(steps, warmup):
    import torch

    from opentpu_amd import _lib as X
    from opentpu_amd import fp32, quant
    N, K = 262144, 2560
    gen = torch.Generator(device="cuda").manual_seed(5)
    W = torch.randn((N, K), generator=gen, device="cuda") * 0.02
    rows, srows = quant.quantize_mxu(W, "int8", rsc=True)
    del W
    x = torch.randn((1, K), generator=gen, device="cuda")
    q, Sa, da = fp32.quantize_mx(x, 32)
    logits = torch.empty((N,), dtype=torch.float32, device="cuda")
    best = torch.zeros((X.LM_STATE_BYTES // 8,), dtype=torch.int64, device="cuda")  # result word, maxima
    tok = torch.empty((1,), dtype=torch.int32, device="cuda")

    def step():
        X.call("otpu_lm_head_argmax", X.ptr(q), X.ptr(Sa), X.ptr(da), K, X.ptr(rows), K, X.ptr(srows), 4, N,
               X.FMT["int8"], X.RSC, 0, 0, X.ptr(logits), X.ptr(best), X.ptr(tok), X.stream())
    ms = timed(step, steps, warmup, torch.cuda.current_stream())
    # the sampled pick after the same LM head: V = 262144, top-k 50, top-p 0.9, penalty 1.1 over
    # a 64-token context, one uniform (the sampler alone, then LM head + sampler in one graph)
    from opentpu_amd import sampler as SM
    sm = SM.Sampler(N, SM.Sampling(0.8, 50, 0.9, 1.1), range(0, 64 * 4000, 4000))
    u = torch.full((1,), 0.37, dtype=torch.float32, device="cuda")

    def pick():
        sm.pick_device(logits, u)
    ms_pick = timed(pick, steps, warmup, torch.cuda.current_stream())

    def both():
        step()
        pick()
    ms_both = timed(both, steps, warmup, torch.cuda.current_stream())
    sm.check()
    step()                                          # the logits and token of the LM head alone
    sample = tuple(t.cpu().numpy() for t in (q, Sa, da, rows, srows, logits)) + (int(tok.item()),)
    return ms, int(tok.item()), ms_pick, ms_both, sample


def gemm(steps, warmup, row_mode=True, fmt="int8", generic=False):
    """The c3 prefill GEMM, RSC weights (fmt int8) or 4-bit group-quantized ones (int4x / fp4x6 / nvfp4:
    the 4-bit GEMM); activations ROW-quantized (the headline: one scale a row, a single exact
    plane) or MX (group offsets: several planes).  generic: the int8 GEMM's generic copy on the
    same operands instead of the one compiled for c3's sizes and strides (OTPU_GENERIC_COPIES
    set while the step is captured; the same work and results)."""
    import torch

    from opentpu_amd import _lib as X
    from opentpu_amd import fp32, quant
    M, K, N = 512, 2048, 8192
    gen = torch.Generator(device="cuda").manual_seed(3)
    W = torch.randn((N, K), generator=gen, device="cuda") * 0.02
    rows, srows = quant.quantize_mxu(W, "int8", rsc=True) if fmt == "int8" else quant.quantize_mxu(W, fmt)
    fl = X.RSC if fmt == "int8" else 0
    x = torch.randn((M, K), generator=gen, device="cuda")
    q, Sa, da = fp32.quantize_mx(x, 32, row_mode=row_mode)
    out = torch.empty((M, N), dtype=torch.float32, device="cuda")

    def step():
        X.call("otpu_mm", X.ptr(q), K, X.ptr(Sa), X.ptr(da), K // 32, M, K, X.ptr(rows), rows.shape[1], X.ptr(srows),
               srows.shape[1], N, X.FMT[fmt], fl, 0, None, X.ptr(out), N, None, X.stream())
    with generic_copies(generic):
        ms = timed(step, steps, warmup, torch.cuda.current_stream())
    sample = tuple(t.cpu().numpy() for t in (q, Sa, da, rows, srows, out))
    return ms, sample


@contextlib.contextmanager
def generic_copies(on):
    """OTPU_GENERIC_COPIES set inside (when on): the library then launches its generic kernel
    copies instead of the ones compiled for the c3 / c4 shapes (read per GEMM call and when a
    chain's plan is built; the same work and results)."""
    old = os.environ.get("OTPU_GENERIC_COPIES")
    if on:
        os.environ["OTPU_GENERIC_COPIES"] = "1"
    try:
        yield
    finally:
        if on:
            if old is None:
                del os.environ["OTPU_GENERIC_COPIES"]
            else:
                os.environ["OTPU_GENERIC_COPIES"] = old


def int_mm(steps, warmup):
    """Yardstick: torch._int_mm (hipBLASLt) at the c3 shape, int8 x int8 -> int32 (the same
    17.2 G ops; an int32 output of the same 16.8 MB, no MM semantics)."""
    import torch
    M, K, N = 512, 2048, 8192
    gen = torch.Generator(device="cuda").manual_seed(3)
    A = torch.randint(-127, 128, (M, K), generator=gen, device="cuda", dtype=torch.int8)
    Bw = torch.randint(-127, 128, (N, K), generator=gen, device="cuda", dtype=torch.int8)   # weight rows, as MM's
    C = torch.empty((M, N), dtype=torch.int32, device="cuda")
    return timed(lambda: torch._int_mm(A, Bw.t(), out=C), steps, warmup, torch.cuda.current_stream())


def c4_step(steps, warmup, persistent=True, generic=False, shape=None):
    """The chained decode step (28 Qwen3-0.6B-shaped layers of int4x linears, weights seeded
    100 + layer): two resident copies of the weights (474 MB, more than the Infinity Cache),
    steps alternating between them, every step's kernels replayed from one HIP graph.
    persistent: the step as one otpu_chain_step launch (the default path), else 112 launches.
    generic: the persistent kernel's generic copy instead of the one compiled for this shape.
    shape: another layer shape (chain.Shape) than Qwen3-0.6B's, 28 layers."""
    import torch

    from opentpu_amd.chain import DecodeChain, Shape
    sh = shape or Shape()
    chains = [DecodeChain.synthetic(sh, "int4", seed0=100) for _ in range(2)]
    for c in chains:
        c.persistent = persistent
    x = torch.randn((1, sh.hidden), generator=torch.Generator(device="cuda").manual_seed(4), device="cuda")
    for c in chains:
        c.x.copy_(x)
    it = [0]

    def step():
        chains[it[0] % 2].step()
        it[0] += 1
    with generic_copies(generic):                   # (the plans are built at the first step)
        ms = timed(step, steps, warmup, torch.cuda.current_stream())
    for c in chains:                    # a step whose hand-off waits gave up is no measurement
        c.check()
    wb = sh.layers * sh.layer_bytes("int4")
    launches = chains[0].kernels_per_step
    del chains
    torch.cuda.empty_cache()
    return {"us_per_step": round(ms * 1e3, 2), "weight_bytes": wb, "GBps": round(wb / (ms * 1e-3) / 1e9, 1),
            "kernels_per_step": launches}


def copy_calibration(nbytes=1 << 30, reps=3):
    """A plain streaming copy of nbytes (torch's elementwise neg: one dispatch that reads and
    writes nbytes), the yardstick the FETCH_SIZE / WRITE_SIZE counters are scaled by: what they
    read for a copy of known size.  Returns GB/s of read + write."""
    import torch
    a = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    ms = timed(lambda: torch.neg(a, out=b), reps, 1, torch.cuda.current_stream(), graph=False)
    del a, b
    torch.cuda.empty_cache()
    return {"bytes": nbytes, "ms": round(ms, 4), "GBps_rw": round(2 * nbytes / (ms * 1e-3) / 1e9, 1)}


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_c2_gemv_int4_batched.txt")


def measured_traffic():
    """HBM bytes per dispatch of the headline kernel as the committed counter summary states it
    (FETCH_SIZE and WRITE_SIZE scaled by the copy kernel's readings), or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_dispatch:"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return None


def summarize(outdir):
    """Text summary of rocprofv3 CSV output in outdir (kernel stats, and for counter runs each
    kernel's mean counter value per dispatch), for the profiles/ folder."""
    import csv
    import glob
    import collections
    for path in sorted(glob.glob(os.path.join(outdir, "**", "*kernel_stats.csv"), recursive=True)):
        print(f"# {os.path.relpath(path, outdir)}")
        with open(path) as f:
            rows = list(csv.DictReader(f))
        print(f"{'calls':>7} {'avg_us':>10} {'min_us':>10} {'max_us':>10} {'pct':>6}  kernel")
        for r in rows:
            name = r["Name"].split("(")[0]
            print(f"{int(r['Calls']):7d} {float(r['AverageNs']) / 1e3:10.3f} {float(r['MinNs']) / 1e3:10.3f} "
                  f"{float(r['MaxNs']) / 1e3:10.3f} {float(r['Percentage']):6.2f}  {name[:110]}")
    # a kernel's runs: consecutive dispatches of it with no other kernel between them (a bench
    # case's graph replays), runs of 10 or more, so that cases sharing a kernel read apart
    for path in sorted(glob.glob(os.path.join(outdir, "**", "*kernel_trace.csv"), recursive=True)):
        with open(path) as f:
            rows = sorted(csv.DictReader(f), key=lambda r: int(r["Dispatch_Id"]))
        runs, cur = [], []
        for r in rows:
            if cur and r["Kernel_Name"] != cur[-1]["Kernel_Name"]:
                runs.append(cur)
                cur = []
            cur.append(r)
        if cur:
            runs.append(cur)
        runs = [u for u in runs if len(u) >= 10]
        if not runs:
            continue
        print(f"# {os.path.relpath(path, outdir)}: runs of one kernel (10 or more dispatches in a row)")
        print(f"{'run':>4} {'calls':>6} {'avg_us':>10} {'min_us':>10} {'max_us':>10}  kernel")
        for i, u in enumerate(runs):
            d = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in u]
            print(f"{i:4d} {len(d):6d} {sum(d) / len(d):10.3f} {min(d):10.3f} {max(d):10.3f}  "
                  f"{u[0]['Kernel_Name'].split('(')[0][:110]}")
    for path in sorted(glob.glob(os.path.join(outdir, "**", "*counter_collection.csv"), recursive=True)):
        print(f"# {os.path.relpath(path, outdir)}")
        agg = collections.defaultdict(lambda: collections.defaultdict(float))
        disp = collections.defaultdict(set)
        with open(path) as f:
            for r in csv.DictReader(f):
                key = (r["Kernel_Name"].split("(")[0][:90], r.get("Grid_Size", ""))
                agg[key][r["Counter_Name"]] += float(r["Counter_Value"])
                disp[key].add(r["Dispatch_Id"])
        print(f"{'dispatches':>10}  {'grid':>10}  counter means per dispatch  kernel")
        for key, d in agg.items():
            n = len(disp[key])
            means = ", ".join(f"{c} {v / n:.1f}" for c, v in sorted(d.items()))
            print(f"{n:10d}  {key[1]:>10}  {means}  {key[0]}")


def cpu_model() -> str:
    """The host CPU's model name (lscpu's "Model name", read from /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _per_call(fn, seconds, max_reps):
    """Seconds per call of fn, over about `seconds` (at least one call after a first one)."""
    t0 = time.perf_counter()
    fn()
    one = time.perf_counter() - t0
    reps = max(1, min(max_reps, int(seconds / max(one, 1e-5))))
    t0 = time.perf_counter()
    for _ in range(reps):
        fn()
    return (time.perf_counter() - t0) / reps, reps


def _same(a, b) -> bool:
    a, b = np.ascontiguousarray(a, np.float32), np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and bool(np.array_equal(a.view(np.uint32), b.view(np.uint32)))


def c4_layer_sample():
    """One c4 layer (the decode step's first layer, weights seeded 100) on the GPU (the
    persistent step, one layer) with host copies of its weights and input, for the CPU leg."""
    import torch

    from opentpu_amd.chain import DecodeChain, Shape
    sh = Shape(layers=1)
    ch = DecodeChain.synthetic(sh, "int4", seed0=100)
    x = torch.randn((1, sh.hidden), generator=torch.Generator(device="cuda").manual_seed(4), device="cuda")
    y = ch.step(x).cpu().numpy()
    wts = {k: (r.cpu().numpy(), sr.cpu().numpy()) for k, (r, sr) in ch.layers[0].items()}
    out = (x.cpu().numpy(), wts, y, sh)
    del ch
    torch.cuda.empty_cache()
    return out


def cpu_baseline(samples, seconds=10.0):
    """The C oracle (OpenMP) on this host, timed beside each config on its own workload, each
    output checked against the GPU's bit for bit.  value: c2, the headline's problem 0 (one GEMV
    repeated for about `seconds`) on min(16, cores) threads; `also`: c2 on one thread and in the
    numpy oracle (float64 group sums, the reference simulator's method), then c1 (problem 0 of
    its timed launch), c3 ROW (the whole GEMM; one thread: its first 64 rows), one c4 layer (QACT
    and MM in the chain's order: q/k/v, o, gate/up, the 12 F-chunks of down) and c5 (the whole LM
    head and its greedy token), each on all threads and on one."""
    from oracle import chain as OCH
    from oracle import cpu as OC
    from oracle import mm as MM
    threads = min(16, os.cpu_count() or 1)
    OC.threads(threads)
    N, K = 6144, 2048
    rows, srows, q, Sa, da, gpu_out = samples["c2"]
    q, Sa, da, gpu_out = q[:1], Sa[:1], da[:1], gpu_out[:1]
    want = OC.mm(q, Sa, da, rows, srows, "int4", K)
    matches = _same(want, gpu_out)
    dt, reps = _per_call(lambda: OC.mm(q, Sa, da, rows, srows, "int4", K), seconds, 2000)
    OC.threads(1)
    dt1, _ = _per_call(lambda: OC.mm(q, Sa, da, rows, srows, "int4", K), 0.2, 20)
    OC.threads(threads)
    t0 = time.perf_counter()
    for _ in range(3):
        MM.mm(q, Sa, da, rows, srows, "int4", K)
    dtn = (time.perf_counter() - t0) / 3
    also = {"c2": {"one_core": {"GBps": round(c2_bytes() / dt1 / 1e9, 3), "ms": round(dt1 * 1e3, 2)},
                   "numpy_oracle": {"GBps": round(c2_bytes() / dtn / 1e9, 3), "ms": round(dtn * 1e3, 1)}},
            "host_cores": os.cpu_count(), "threads": threads}

    def both(name, fn, fn1, unit_of, what):
        """fn on every thread (~2 s), fn1 (a smaller sample where named) on one; unit_of(dt, one)."""
        dta, ra = _per_call(fn, 2.0, 200)
        OC.threads(1)
        dto, ro = _per_call(fn1, 1.0, 20)
        OC.threads(threads)
        also[name] = {"what": what, "all_cores": {**unit_of(dta, False), "ms": round(dta * 1e3, 3), "calls": ra},
                      "one_core": {**unit_of(dto, True), "ms": round(dto * 1e3, 3), "calls": ro}}

    if "c1" in samples:
        r1, s1, q1, S1, d1, o1 = samples["c1"]
        f1 = lambda: OC.mm(q1, S1, d1, r1, s1, "int8", 1024, flags=MM.RSC)   # noqa: E731
        both("c1", f1, f1, lambda dt, one: {"GBps": round(c1_bytes() / dt / 1e9, 3)},
             "int8 RSC GEMV 4096x1024 (problem 0 of the timed launch)")
        also["c1"]["gpu_output_matches"] = _same(f1(), o1)
    if "c3" in samples:
        q3, S3, d3, r3, s3, o3 = samples["c3"]
        f3 = lambda: OC.mm(q3, S3, d3, r3, s3, "int8", 2048, flags=MM.RSC)   # noqa: E731
        f31 = lambda: OC.mm(q3[:64], S3[:64], d3[:64], r3, s3, "int8", 2048, flags=MM.RSC)  # noqa: E731
        both("c3", f3, f31, lambda dt, one: {"TOPS": round(2 * (64 if one else 512) * 8192 * 2048 / dt / 1e12, 4)},
             "ROW x RSC GEMM 512x2048x8192 (one core: its first 64 rows)")
        also["c3"]["gpu_output_matches"] = _same(f3(), o3)
    if "c4" in samples:
        x4, wts, y4, sh = samples["c4"]
        f4 = lambda: OCH.layer(x4, wts, "int4", sh.q_dim, sh.F, mm=OC.mm)[0]    # noqa: E731
        lb = sh.layer_bytes("int4")
        both("c4", f4, f4, lambda dt, one: {"us_per_layer": round(dt * 1e6, 1), "GBps": round(lb / dt / 1e9, 3)},
             "one Qwen3-0.6B-shaped layer of int4x linears (QACT + MM each, 12 down chunks with ACC)")
        also["c4"]["gpu_output_matches"] = _same(f4(), y4)
    if "c5" in samples:
        q5, S5, d5, r5, s5, l5, t5 = samples["c5"]
        f5 = lambda: OC.mm(q5, S5, d5, r5, s5, "int8", 2560, flags=MM.RSC)   # noqa: E731
        both("c5", f5, f5, lambda dt, one: {"GBps": round(c5_bytes() / dt / 1e9, 3)},
             "LM head 262144x2560 RSC logits (greedy token checked separately)")
        lg = f5()
        also["c5"]["gpu_output_matches"] = _same(lg[0], l5) and OC.argmax(lg[0])[0] == t5
    return {"value": round(c2_bytes() / dt / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"c2 int4 GEMV 6144x2048 (problem 0 of the timed launch), {reps} calls of the C oracle "
                      f"(oracle/cpu_mm.c, OpenMP), {dt * 1e3:.2f} ms per call",
            "cpu_model": cpu_model(), "gpu_output_matches": matches, "also": also}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=80)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default="", help="comma list of c1,c2s,c3,c3r,c3m,c3q,c3g,c3blas,c4,c5,copy (default: "
                    "c1,c2s,c3,c4,c5; c3r / c3m: the ROW / the MX int8 GEMM alone; c3q: the 4-bit GEMMs alone; c3g: "
                    "the ROW GEMM's generic copy; c3blas: hipBLASLt's int8 GEMM at c3's shape, a yardstick); "
                    "the headline c2 always runs, c2s adds its single-launch figure")
    ap.add_argument("--summarize", metavar="DIR", help="print a text summary of rocprofv3 CSV output and exit")
    args = ap.parse_args()
    if args.summarize:
        summarize(args.summarize)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU only (no multi-GPU path); use --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(2)
    torch.cuda.set_device(0)
    only = set(args.only.split(",")) if args.only else {"c1", "c2s", "c3", "c4", "c5"}
    extra = {}

    N2, K2, B2 = 6144, 2048, args.batch
    ms2, single2 = batched_gemv("int4", B2, N2, K2, 2, args.steps, args.warmup)
    gbs2 = B2 * c2_bytes() / (ms2 * 1e-3) / 1e9
    print(f"[c2] batched int4 GEMV: {ms2:.4f} ms/step, {gbs2:.1f} GB/s", file=sys.stderr, flush=True)
    rows2, srows2, q2, Sa2, da2, out2 = single2
    sample2 = (rows2[0], srows2[0], q2[:1], Sa2[:1], da2[:1], out2[:1].clone())
    if "c2s" in only:
        ms2s = single_gemv_ms("int4", single2, N2, K2, 200)
        extra["c2_single_launch"] = {"us": round(ms2s * 1e3, 3),
                                     "GBps": round(c2_bytes() / (ms2s * 1e-3) / 1e9, 1)}
    samples = {"c2": tuple(t.cpu().numpy() for t in sample2)}
    del single2, rows2, srows2, q2, Sa2, da2, out2, sample2
    torch.cuda.empty_cache()

    if "copy" in only:
        extra["copy_1GiB"] = copy_calibration()
        print(f"[copy] {extra['copy_1GiB']}", file=sys.stderr, flush=True)
    if "c1" in only:
        B1 = 128
        ms1, s1 = batched_gemv("int8", B1, 4096, 1024, 1, 20, 3, rsc=True)
        extra["c1_int8_rsc_gemv"] = {"batch": B1, "ms": round(ms1, 4),
                                     "GBps": round(B1 * c1_bytes() / (ms1 * 1e-3) / 1e9, 1)}
        ms1s = single_gemv_ms("int8", s1, 4096, 1024, 200, rsc=True)
        extra["c1_single_launch"] = {"us": round(ms1s * 1e3, 3)}
        r1, sr1, q1, S1, d1, o1 = s1
        samples["c1"] = tuple(t.cpu().numpy() for t in (r1[0], sr1[0], q1[:1], S1[:1], d1[:1], o1[:1]))
        del s1, r1, sr1, q1, S1, d1, o1
        torch.cuda.empty_cache()
        print(f"[c1] {extra['c1_int8_rsc_gemv']}", file=sys.stderr, flush=True)
    if "c5" in only:
        ms5, tok, ms_pick, ms_both, samples["c5"] = lm_head(10, 2)
        extra["c5_lm_head_argmax"] = {"us": round(ms5 * 1e3, 2), "token": tok,
                                      "GBps": round(c5_bytes() / (ms5 * 1e-3) / 1e9, 1),
                                      "frac_hbm": round(c5_bytes() / (ms5 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        extra["c5_sampler"] = {"pick_us": round(ms_pick * 1e3, 2), "lm_head_plus_pick_us": round(ms_both * 1e3, 2),
                               "sampling": "top_k 50, top_p 0.9, T 0.8, penalty 1.1, V 262144"}
        torch.cuda.empty_cache()
        print(f"[c5] {extra['c5_lm_head_argmax']}", file=sys.stderr, flush=True)
    if "c4" in only:
        extra["c4_decode_step"] = c4_step(10, 2)
        print(f"[c4] {extra['c4_decode_step']}", file=sys.stderr, flush=True)
        # the same step as one launch per linear (the path the persistent step replaces)
        extra["c4_decode_step_launches"] = c4_step(10, 2, persistent=False)
        print(f"[c4 launches] {extra['c4_decode_step_launches']}", file=sys.stderr, flush=True)
        # the persistent step's generic copy (what every other shape runs) on the same weights
        extra["c4_decode_step_generic_copy"] = c4_step(10, 2, generic=True)
        print(f"[c4 generic copy] {extra['c4_decode_step_generic_copy']}", file=sys.stderr, flush=True)
        # the persistent step at Qwen3-1.7B's layer shape (hidden 2048, q_dim 2048, kv_dim 1024,
        # F 6144: 768-column down chunks), 28 layers: the chain's second set of teams
        from opentpu_amd.chain import Shape
        extra["c4_qwen3_1p7b_shape_step"] = c4_step(10, 2, shape=Shape(hidden=2048, q_dim=2048, kv_dim=1024, F=6144))
        print(f"[c4 1.7B shape] {extra['c4_qwen3_1p7b_shape_step']}", file=sys.stderr, flush=True)
        if not args.no_cpu:
            samples["c4"] = c4_layer_sample()
    if "c3" in only or "c3r" in only:
        ms3, samples["c3"] = gemm(20, 2)
        tops = 2 * 512 * 2048 * 8192 / (ms3 * 1e-3) / 1e12
        extra["c3_gemm_row_x_rsc"] = {"us": round(ms3 * 1e3, 2), "TOPS": round(tops, 2),
                                      "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4)}
        print(f"[c3] {extra['c3_gemm_row_x_rsc']}", file=sys.stderr, flush=True)
        # yardstick: writing c3's fp32 output alone (a fill kernel over the same 16.8 MB)
        o3 = torch.empty((512, 8192), dtype=torch.float32, device="cuda")
        msf = timed(lambda: o3.fill_(1.0), 20, 2, torch.cuda.current_stream())
        del o3
        extra["c3_output_write_alone"] = {"us": round(msf * 1e3, 2), "what": "torch fill_ of the 512 x 8192 fp32 output"}
    if "c3" in only or "c3g" in only:
        # the same ROW GEMM through the generic copy (every shape that is not c3's runs it)
        ms3g, _ = gemm(20, 2, generic=True)
        tops = 2 * 512 * 2048 * 8192 / (ms3g * 1e-3) / 1e12
        extra["c3_gemm_row_x_rsc_generic_copy"] = {"us": round(ms3g * 1e3, 2), "TOPS": round(tops, 2),
                                                   "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4)}
        print(f"[c3 generic copy] {extra['c3_gemm_row_x_rsc_generic_copy']}", file=sys.stderr, flush=True)
    if "c3blas" in only:
        msb = int_mm(20, 2)
        tops = 2 * 512 * 2048 * 8192 / (msb * 1e-3) / 1e12
        extra["c3_hipblaslt_int_mm"] = {"us": round(msb * 1e3, 2), "TOPS": round(tops, 2),
                                        "what": "torch._int_mm at 512 x 2048 x 8192, int32 output"}
        print(f"[c3 hipBLASLt] {extra['c3_hipblaslt_int_mm']}", file=sys.stderr, flush=True)
    if "c3" in only or "c3m" in only:
        ms3m, _ = gemm(20, 2, row_mode=False)
        tops = 2 * 512 * 2048 * 8192 / (ms3m * 1e-3) / 1e12
        extra["c3_gemm_mx_x_rsc"] = {"us": round(ms3m * 1e3, 2), "TOPS": round(tops, 2),
                                     "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4)}
        print(f"[c3 mx] {extra['c3_gemm_mx_x_rsc']}", file=sys.stderr, flush=True)
    if "c3" in only or "c3q" in only:
        # the c3 shape with 4-bit group-quantized weights (int4x, fp4x6, nvfp4): the 4-bit GEMM,
        # whose two weight planes make two int8 MFMA products of the c3 size
        for f4 in ("int4", "fp4", "nvfp4"):
            for rm, tag in ((True, "row"), (False, "mx")):
                ms4, _ = gemm(20, 2, row_mode=rm, fmt=f4)
                tops = 2 * 512 * 2048 * 8192 / (ms4 * 1e-3) / 1e12
                key = f"c3_gemm_{tag}_x_{f4}" + ("" if f4 == "nvfp4" else "x")
                extra[key] = {"us": round(ms4 * 1e3, 2), "TOPS": round(tops, 2),
                              "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4)}
                print(f"[c3 {f4} {tag}] {extra[key]}", file=sys.stderr, flush=True)

    cpu = None if args.no_cpu else cpu_baseline(samples)
    if cpu is not None:
        print(f"[cpu] {json.dumps(cpu['also'])}", file=sys.stderr, flush=True)
    line = {
        "metric": "quant GEMV GB/s (% HBM peak) + prefill int8 GEMM TOPS, 1 MI355X",
        "value": round(gbs2, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms2, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 weights x int8 activations (int32 dot, exact int64 accumulate, fp32 epilogue)",
        "data": "synthetic (seeded N(0,0.02) weights packed on the GPU, N(0,1) activations)",
        "config": {"workload": f"c2: 4-bit int4x group-32 decode GEMV N={N2} K={K2}, {B2} independent "
                               f"weight sets per launch", "batch": B2, "N": N2, "K": K2, "fmt": "int4"},
        "roofline": {"bound": "hbm", "achieved": round(gbs2, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs2 / HBM_PEAK_GBS, 4), "traffic": measured_traffic()},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
