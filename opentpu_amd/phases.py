"""Phase breakdown of the persistent chained decode step (the c4 workload: 28 Qwen3-0.6B-shaped
layers of int4x linears) from per-workgroup clock stamps.

    python -m opentpu_amd.build --stamps      # libotpu_amd_stamps.so: the stamps compiled in
    python -m opentpu_amd.phases              # on a GPU: the table below

Each workgroup's first thread stamps the 100 MHz wall clock at eight points of every phase it
has rows in: phase start (0), weights issued, i.e. its wait for the input row starts (1), the
row's last entry carrying the phase's tag (7), every entry carrying it (2), QACT done, the
activation pieces in registers (3), rows stored (4), and around the QACT's first barrier: wave
0's own part done (6) and every wave's done (5). Per linear (medians over workgroups, means over
the 28 layers) the table gives the intervals 0-1, 1-2 (split into the wait for the last entry,
1-7, and the row's load and re-polls after it, 7-2), 2-3 and 3-4; the QACT interval split into
wave 0's own part (2-6), the wait at the barrier for the other waves, whose input rows can come
in later (6-5), and what follows the barrier (5-3); the hand-off (the previous phase's last
workgroup done -> this phase's median workgroup with its input in: store visibility plus
polling); and the tail (median -> last workgroup done); and the mean counts of wave 0's polls of
the last entry that missed (8) and of its rounds of re-polls of the row after it (9). Two weight
copies alternate, as in bench.py; the step is replayed from a HIP graph.
Measurement only: the stamped library is not the product's."""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
NAMES = ("qkv", "o", "gate/up", "down (fold)")
TICK_NS = 10.0                                  # s_memrealtime: 100 MHz


def breakdown(st: np.ndarray) -> dict:
    """st [phases, grid, 8] stamps -> per linear kind: the mean over layers of the medians (us)."""
    rows = {n: [] for n in NAMES}
    prev_end = None
    for i in range(st.shape[0]):
        ran = st[i, :, 4] > 0
        a = st[i][ran].astype(np.float64)
        if not len(a):
            continue
        end = a[:, 4].max()
        if i > 0:                                # layer 0's qkv reads the plain input row
            med = lambda j, k: np.median(a[:, k] - a[:, j]) * TICK_NS / 1e3
            rows[NAMES[i % 4]].append([med(0, 1), med(1, 2), med(2, 3), med(3, 4),
                                       (np.median(a[:, 2]) - prev_end) * TICK_NS / 1e3,
                                       (end - np.median(a[:, 4])) * TICK_NS / 1e3, int(ran.sum()),
                                       med(2, 6), med(6, 5), med(5, 3), med(1, 7), med(7, 2),
                                       np.mean(a[:, 8]), np.mean(a[:, 9])])
        prev_end = end
    return {n: np.mean(np.array(v), axis=0) for n, v in rows.items() if v}


def main() -> None:
    lib_path = os.path.join(HERE, "libotpu_amd_stamps.so")
    if not os.path.exists(lib_path):
        sys.exit("opentpu_amd.phases: build the stamped library first (python -m opentpu_amd.build --stamps)")
    os.environ["OTPU_LIB"] = lib_path
    import ctypes as C

    import torch

    from . import _lib as X
    from .chain import DecodeChain, Shape
    X.load(lib_path)
    sh = Shape()
    chains = [DecodeChain.synthetic(sh, "int4", seed0=100) for _ in range(2)]
    x = torch.randn((1, sh.hidden), generator=torch.Generator(device="cuda").manual_seed(4), device="cuda")
    for c in chains:
        c.x.copy_(x)
        c.capture()
    torch.cuda.synchronize()
    G = torch.cuda.get_device_properties(0).multi_processor_count
    st = torch.zeros((4 * sh.layers, G, 16), dtype=torch.int64, device="cuda")
    X.call("otpu_chain_stamps", C.c_void_p(chains[0]._plan_ptr()), C.c_void_p(st.data_ptr()))
    for _ in range(3):                              # steps alternating between the two copies
        chains[1]._graph.replay()
        chains[0]._graph.replay()
    torch.cuda.synchronize()
    X.call("otpu_chain_stamps", C.c_void_p(chains[0]._plan_ptr()), None)
    s = st.cpu().numpy()
    if chains[0].chain_error():
        sys.exit("opentpu_amd.phases: a hand-off wait ran out of polls")
    valid = s[:, :, 4] > 0
    span = (s[:, :, 4][valid].max() - s[:, :, 0][valid].min()) * TICK_NS / 1e3
    print(f"persistent c4 step (28 layers x 4 linears, {G} workgroups): {span:.1f} us in the kernel, "
          f"{span / (4 * sh.layers):.2f} us a phase")
    print(f"{'linear':12s} {'wgs':>4s} {'start->wait':>11s} {'wait':>6s} {'(last':>6s} {'row)':>6s} "
          f"{'QACT':>6s} {'(own':>6s} {'join':>6s} {'after)':>6s} {'rows':>6s} {'hand-off':>9s} {'tail':>6s}"
          f" {'polls':>6s} {'re-polls':>8s}   (us; medians over workgroups, means over layers; polls: means)")
    for n, m in breakdown(s).items():
        print(f"{n:12s} {m[6]:4.0f} {m[0]:11.2f} {m[1]:6.2f} {m[10]:6.2f} {m[11]:6.2f} {m[2]:6.2f} {m[7]:6.2f} "
              f"{m[8]:6.2f} {m[9]:6.2f} {m[3]:6.2f} {m[4]:9.2f} {m[5]:6.2f} {m[12]:6.2f} {m[13]:8.2f}")


if __name__ == "__main__":
    main()
