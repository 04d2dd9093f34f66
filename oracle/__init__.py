"""CPU oracle for the quantized-linear hot path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the bit-exact semantics of openTPU's MM / QACT / ARGMAX
(the reference's `opentpu/isasim.py`, `opentpu/fp32.py`, `opentpu/quant.py`) so that the
HIP kernels of `opentpu_amd` can be checked against it. Only `tests/`,
`__graft_entry__.smoke()` and `bench.py`'s `cpu_baseline` leg may import, call, link or run
anything in here, and only as the checker (or as the timed CPU baseline), never as the thing
measured or shipped. The product path (`opentpu_amd`) never falls back to it.

Modules
  fp32     FTZ/RNE binary32 arithmetic, recip, q8, the row/MX quantizer (QACT, QST, int8x).
  formats  MXU weight formats: DEC tables, nibble packing, row/scale-row layouts, packers
           (int8x, RSC, int4x / fp4x6 m-search, nvfp4 decode), dequantization.
  mm       MM: exact per-group int32 sums, int64 shift-accumulate, the fp32 epilogue,
           ACC / ASCALE / RMAX; ARGMAX and greedy selection.
  groups   the reference machine's grouped / channel-hashed weight images (WG lanes) and their
           inverses, built byte address by byte address from the layout's formulas.
  emulate  the reference's float64 emulation: fake_act, group offsets, mx_matmul's drops.
  imports  MXFP4 / NVFP4 checkpoint imports into fp4 / nvfp4 rows, exactly (NotExact).
  sampler  the sampled pick after the LM head: penalty, soft cap, knock-out top-k, the
           machine's exp2 softmax, top-p and the inverse-CDF pick.
  cpu      ctypes binding of `cpu_mm.c` (the same functions in C with OpenMP), the fast
           checker at full sizes and the CPU baseline timer.

Parity pinning of every function is listed in each module's header.
"""
