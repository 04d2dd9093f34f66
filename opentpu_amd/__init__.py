"""opentpu_amd: openTPU's quantized-linear hot path (MM / QACT / greedy ARGMAX) on the MI355X.

The operators run as hand-written HIP kernels for gfx950 behind the C ABI of include/otpu.h
(libotpu_amd.so, loaded with ctypes).  Python modules mirror the reference's function-level API:
  fp32.quantize_mx / quantize       (opentpu/fp32.py)        the QACT quantizer
  quant.quantize_mxu / row_bytes    (opentpu/quant.py)       weight formats and packers
  mxu.mm / dot / lm_head_argmax     (opentpu/isasim.py MM,   the operator and its callers
      / argmax / greedy / QWeight    compiler.dot, generate.Greedy)
  chain.DecodeChain                 chained decode GEMVs of a Qwen3-shaped model (linears only)
There is no CPU fallback: without the built library or a GPU the calls raise."""
from . import _lib  # noqa: F401

__version__ = "0.1.0"
