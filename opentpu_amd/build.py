"""Build the HIP library libotpu_amd.so in-tree for gfx950 (hipcc, no JIT cache).

    python -m opentpu_amd.build          # or __graft_entry__.build()

Every .hip under csrc/ is compiled with: FMA contraction off (the epilogue and recip are
literal sequences of rounded products and sums), fp32 denormals kept (flushes are explicit),
packed-fp32 instruction selection off, -O3."""
from __future__ import annotations

import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libotpu_amd.so")
ARCH = os.environ.get("OTPU_ARCH", "gfx950")

FLAGS = ["-O3", "-std=c++17", "-fPIC", "-shared", f"--offload-arch={ARCH}",
         "-ffp-contract=off", "-fno-gpu-flush-denormals-to-zero", "-fno-fast-math",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Wno-unused-command-line-argument", "-Wall"]


def sources():
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")))


def _stale(src: str, obj: str) -> bool:
    """obj is older than src or than any header under csrc/ or include/."""
    if not os.path.exists(obj):
        return True
    t = os.path.getmtime(obj)
    deps = [src] + glob.glob(os.path.join(CSRC, "*.h")) + glob.glob(os.path.join(HERE, "..", "include", "*.h"))
    return any(os.path.getmtime(d) > t for d in deps)


STAMPS_LIB = os.path.join(HERE, "libotpu_amd_stamps.so")


def build(verbose: bool = True, incremental: bool = False, stamps: bool = False) -> str:
    """Compile every source to an object in parallel (one hipcc per file), then link.
    incremental: keep the objects in csrc/_build and recompile only those older than their
    source or a header (a developer's loop; the default compiles everything).
    stamps: the profiling build, libotpu_amd_stamps.so, with the persistent chain's phase clock
    stamps compiled in (OTPU_PHASE_STAMPS; read by python -m opentpu_amd.phases)."""
    import tempfile
    from concurrent.futures import ThreadPoolExecutor
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    inc = ["-I", os.path.join(HERE, "..", "include")]
    cflags = [f for f in FLAGS if f != "-shared"] + (["-DOTPU_PHASE_STAMPS"] if stamps else [])
    lib = STAMPS_LIB if stamps else LIB
    keep = os.path.join(CSRC, "_build_stamps" if stamps else "_build")
    if incremental:
        os.makedirs(keep, exist_ok=True)
    with tempfile.TemporaryDirectory(prefix="otpu_build_") as tmpd:
        def compile_one(src):
            obj = os.path.join(keep if incremental else tmpd, os.path.basename(src) + ".o")
            if incremental and not _stale(src, obj):
                return obj, subprocess.CompletedProcess([], 0, "", "")
            cmd = [hipcc, *cflags, *inc, "-c", src, "-o", obj]
            if verbose:
                print(" ".join(cmd), flush=True)
            return obj, subprocess.run(cmd, capture_output=True, text=True)
        with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
            results = list(ex.map(compile_one, sources()))
        warn = []
        for obj, r in results:
            if r.returncode != 0:
                sys.stderr.write(r.stdout + r.stderr)
                raise RuntimeError(f"hipcc failed on {obj}")
            warn += [l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l and l.strip()]
        tmp = lib + ".tmp"
        cmd = [hipcc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *[o for o, _ in results], "-o", tmp]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            sys.stderr.write(r.stdout + r.stderr)
            raise RuntimeError("link failed")
    if verbose and warn:
        print("\n".join(warn))
    os.replace(tmp, lib)
    return lib


if __name__ == "__main__":
    build(incremental="--incremental" in sys.argv, stamps="--stamps" in sys.argv)
