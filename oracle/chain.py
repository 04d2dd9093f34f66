"""Oracle: the chained decode step of a Qwen3-shaped stack of quantized linears (numpy).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

One layer, restated from the reference's lowering of a decoder layer's linears:
  - every linear's input is one QACT of its whole fp32 row (`fp32.quantize_mx(x, 32)`,
    `opentpu/isasim.py:913-959`), and its output is one MM (`opentpu/isasim.py:749-910`);
  - q / k / v share the layer input; o takes q's output; gate / up take o's output;
  - down takes the VOP MUL g * u (`opentpu/fp32.py:100`, here without the SiLU: linears only)
    quantized in F-chunks, one QACT and one MM per chunk, the MMs accumulated with ACC in
    chunk order (`opentpu/kernels/mlp.py:8-30`, `:87-120`; `Builder.dot`,
    `opentpu/compiler.py:2686-2720`);
  - the next layer's input is the down projection's output.

`emulated_layer` is the same layer in float64 with the quantization points but none of the
machine's rounding, the way the reference separates quantization error from kernel bugs
(`opentpu/llm/qwen3.py:830-905` emulated_logits, `opentpu/reference.py:14-17` mlp): each
linear's input through `emulate.fake_act` (its QACT ranges: the whole row, the down input in its
F-chunks), the weights through `emulate.fake_w`, each product through `emulate.mx_matmul` (the
window's drops), g * u a float64 product.

Pinning (tests/test_oracle_chain.py): `down_chunk` against the closed form of
`opentpu/kernels/mlp.py:8-30` and the chunk sizes the reference documents for F = 3072 (int8
384, 4-bit 256); the per-range ACC chain against one MM over the whole row where one range
covers it, and against independent per-range MMs added in order; the MM and QACT steps are
the pinned `oracle.mm` / `oracle.fp32` functions.
"""
from __future__ import annotations

import numpy as np

from . import emulate as EM
from . import fp32 as F
from . import mm as MM
from .formats import D, WINDOW

ACC = MM.ACC


def chunk(f_loc: int, q: int = D) -> int:
    """F-chunk size: about 8 chunks, a multiple of q, at least 2D where F allows
    (`opentpu/kernels/mlp.py:8-24`)."""
    if f_loc % q:
        raise ValueError(f"F {f_loc} is not a multiple of {q}")
    lo = min(f_loc, -(-2 * D // q) * q)
    c = max(lo, (f_loc // 8) // q * q)
    while f_loc % c and c > lo:
        c -= q
    while f_loc % c:
        c += q
    return c


def down_chunk(f_loc: int, fmt: str) -> int:
    """The columns each down MM's activations are quantized over (`opentpu/kernels/mlp.py:27-30`):
    chunks of whole D-blocks for int8, whole 2D (128-byte) chunks for the 4-bit formats."""
    return chunk(f_loc, D if fmt == "int8" else 2 * D)


def linear(x, w, fmt: str, rscale=None, cscale=None, mm=MM.mm):
    """QACT of x [M, K] (one range; with QACT's RSCALE / CSCALE factors when given) and the MM
    with packed weights w = (rows, srows).  mm: the MM restatement to use (oracle.mm.mm, or the
    C oracle's oracle.cpu.mm, which takes the same arguments)."""
    x = np.asarray(x, np.float32)
    q, Sa, da = F.qact(x, 32, rscale=rscale, cscale=cscale)
    return mm(q, Sa, da, w[0], w[1], fmt, x.shape[1])


def ranges_dot(x, w, fmt: str, width: int, mm=MM.mm):
    """x [M, K] @ w in column ranges of `width`: a QACT and an MM per range, the first MM
    writing, the rest ACC (y = add(y, mm_r)), in range order."""
    x = np.asarray(x, np.float32)
    K = x.shape[1]
    rows, srows = w
    bpb = D if fmt == "int8" else D // 2          # weight bytes per 128-column block
    y = None
    for r, c0 in enumerate(range(0, K, width)):
        q, Sa, da = F.quantize_mx(x[:, c0:c0 + width], 32)
        k0 = c0 // D
        part = rows[:, k0 * bpb:(k0 + width // D) * bpb]
        y = mm(q, Sa, da, part, srows, fmt, width, k0=k0, flags=ACC if y is not None else 0, old=y)
    return y


def layer(x, wts: dict, fmt: str = "int4", q_dim: int = 2048, F_dim: int = 3072, norm=None, mm=MM.mm):
    """One layer's linears: wts holds packed (rows, srows) for 'qkv' (q, k, v rows stacked),
    'o', 'gu' (gate, up rows stacked) and 'down'.  norm (optional): (gamma_attn, gamma_mlp,
    r_attn, r_mlp), the RMSNorm factors the qkv and gate / up QACTs apply (RSCALE r, CSCALE
    gamma).  Returns (next input, dict of the outputs)."""
    g0, g1, r0, r1 = norm if norm is not None else (None, None, None, None)
    qkv = linear(x, wts["qkv"], fmt, r0, g0, mm)
    o = linear(qkv[:, :q_dim], wts["o"], fmt, mm=mm)
    gu = linear(o, wts["gu"], fmt, r1, g1, mm)
    h = F.mul(gu[:, :F_dim], gu[:, F_dim:2 * F_dim])
    y = ranges_dot(h, wts["down"], fmt, down_chunk(F_dim, fmt), mm)
    return y, {"qkv": qkv, "o": o, "gu": gu, "h": h, "down": y}


def step(x, layers: list, fmt: str = "int4", q_dim: int = 2048, F_dim: int = 3072, norms=None, mm=MM.mm):
    """The decode step: every layer in order; returns the last layer's output (mm: the MM
    oracle, numpy's or the C restatement's)."""
    for i, wts in enumerate(layers):
        x, _ = layer(x, wts, fmt, q_dim, F_dim, norms[i] if norms is not None else None, mm=mm)
    return x


def emulated_linear(x, w, fmt: str, n: int | None = None):
    """float64: fake_act of x [M, K] (ranges of n columns) times fake_w of w = (rows, srows) with
    MM's window drops."""
    x = np.asarray(x, np.float64)
    K = x.shape[1]
    h, da = EM.fake_act(x, n=n)
    wv, dw = EM.fake_w(w[0], w[1], fmt, K)
    return EM.mx_matmul(h, wv, da, dw, WINDOW[fmt])


def emulated_layer(x, wts: dict, fmt: str = "int4", q_dim: int = 2048, F_dim: int = 3072):
    """One layer in float64 with the quantization points (see the module's header): (output,
    dict of the intermediates)."""
    qkv = emulated_linear(x, wts["qkv"], fmt)
    o = emulated_linear(qkv[:, :q_dim], wts["o"], fmt)
    gu = emulated_linear(o, wts["gu"], fmt)
    h = gu[:, :F_dim] * gu[:, F_dim:2 * F_dim]
    y = emulated_linear(h, wts["down"], fmt, down_chunk(F_dim, fmt))
    return y, {"qkv": qkv, "o": o, "gu": gu, "h": h, "down": y}
