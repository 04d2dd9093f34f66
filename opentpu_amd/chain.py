"""The chained decode step of a Qwen3-shaped stack of quantized linears, resident on the GPU.

Per layer (the reference's lowering of a decoder layer's linears: `opentpu/kernels/mlp.py`,
`Builder.dot` `opentpu/compiler.py:2686-2720`):
    QACT(x) -> MM qkv          q, k, v rows stacked: one weight, one launch
    QACT(q) -> MM o
    QACT(o) -> MM gu           gate, up rows stacked
    QACT ranges of mul(g, u)   the down input in F-chunks (one QACT each, `mlp.py:8-30`)
            -> MM down         one MM per chunk, ACC in chunk order (otpu_mm_ranges)
and the down output is the next layer's input.  Every buffer is allocated once; a step only
queues kernels, so it can be captured in a HIP graph and replayed (`capture` / `replay`).

Weights: one int4x / fp4x6 / int8x packing per linear, packed on the GPU (`quant.quantize_mxu`),
or the reference's packed bytes loaded unchanged (`from_packed`)."""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import _lib as X
from .mxu import C_ptr
from .quant import D, quantize_mxu, row_bytes, scale_bytes


def down_chunk(f_loc: int, fmt: str) -> int:
    """The F-chunk each down MM's activations are quantized over (`opentpu/kernels/mlp.py:8-30`):
    about 8 chunks, a multiple of D (int8) or 2D (4-bit), at least 2D where F allows."""
    q = D if fmt == "int8" else 2 * D
    if f_loc % q:
        raise ValueError(f"F {f_loc} is not a multiple of {q}")
    lo = min(f_loc, -(-2 * D // q) * q)
    c = max(lo, (f_loc // 8) // q * q)
    while f_loc % c and c > lo:
        c -= q
    while f_loc % c:
        c += q
    return c


@dataclass
class Shape:
    """A Qwen3-shaped layer's linears (defaults: Qwen3-0.6B: hidden 1024, 16 q heads and 8 kv
    heads of 128, intermediate 3072, 28 layers)."""
    hidden: int = 1024
    q_dim: int = 2048
    kv_dim: int = 1024
    F: int = 3072
    layers: int = 28

    def weight_shapes(self):
        """(name, N, K) of the four streamed weights of a layer."""
        h = self.hidden
        return [("qkv", self.q_dim + 2 * self.kv_dim, h), ("o", h, self.q_dim), ("gu", 2 * self.F, h),
                ("down", h, self.F)]

    def layer_bytes(self, fmt: str) -> int:
        return sum(N * (row_bytes(K, fmt) + scale_bytes(K, fmt)) for _, N, K in self.weight_shapes())


class DecodeChain:
    """`layers`: per layer a dict name -> (rows, srows) device tensors (uint8).

    persistent (default where it applies: fused and folded, int4 / fp4 / nvfp4 weights, hidden <= 2048,
    q_dim <= 2048, F <= 8192): the whole step is one launch of otpu_chain_step, its phases handing
    rows to each other on the GPU; the same bits as the four kernels a layer below.
    fused: a layer is four kernels, each linear an otpu_mm_qin (the QACT of its input
    row in the GEMV's prologue).  With 4-bit weights and 256-column down chunks the down
    projection is one otpu_mm_qin_fold, which folds its chunks' outputs in chunk order (the ACC
    chain) itself; otherwise its per-chunk outputs stay partial, the next layer's prologue folds
    them in chunk order and the step's last fold is one otpu_acc_rows.  Unfused: the nine
    kernels of `layer` (QACT, MM, .. one call each)."""

    KERNELS_PER_LAYER = 9          # unfused: 3 QACT, 3 MM, QACT ranges, per-range MM + its ACC fold
    FUSED_KERNELS_PER_LAYER = 4    # fused: one QACT + MM kernel per linear

    def __init__(self, layers: list, shape: Shape = Shape(), fmt: str = "int4", fused: bool = True,
                 norms: list | None = None, persistent: bool | None = None):
        """norms (optional): per layer (gamma_attn, gamma_mlp), the RMSNorm weights [hidden] in
        front of the qkv and of the gate / up projections.  They ride in those linears' QACT as
        CSCALE, with the row factor r of each norm (RSCALE: `self.rnorm[l, 0 | 1]`, 1 unless
        the caller sets it): x' = (x * r) * gamma (`docs/isa.md:447-452`), no extra launch."""
        self.layers = layers
        self.shape = shape
        self.fmt = fmt
        self.fused = fused
        s = shape
        self.width = down_chunk(s.F, fmt)
        self.R = s.F // self.width
        # the down projection folded in its own launch (4-bit, 256-column chunks); False keeps
        # the per-chunk partial rows folded by the next layer's prologue
        self.fold = fmt != "int8" and self.width % 256 == 0 and s.F <= 8192
        nq = s.q_dim + 2 * s.kv_dim
        T = X.torch()
        dev = "cuda"
        f32, i8, u8 = T.float32, T.int8, T.uint8
        self.x = T.zeros((1, s.hidden), dtype=f32, device=dev)
        self.y = T.zeros((1, s.hidden), dtype=f32, device=dev)           # the step's output
        self.y2 = T.zeros((1, s.hidden), dtype=f32, device=dev)
        self.qkv = T.empty((1, nq), dtype=f32, device=dev)
        self.o = T.empty((1, s.hidden), dtype=f32, device=dev)
        self.gu = T.empty((1, 2 * s.F), dtype=f32, device=dev)
        kmax = max(s.hidden, s.q_dim, s.F)
        self.qa = T.empty((1, kmax), dtype=i8, device=dev)
        self.Sa = T.empty((self.R,), dtype=f32, device=dev)
        self.da = T.empty((1, kmax // 32), dtype=u8, device=dev)
        self.part = T.empty((self.R, s.hidden), dtype=f32, device=dev)
        self.parts = [T.zeros((self.R, s.hidden), dtype=f32, device=dev) for _ in range(2)]
        self.hbuf = [T.zeros((1, s.hidden), dtype=f32, device=dev) for _ in range(2)]
        self.norms = None
        if norms is not None:
            if len(norms) != len(layers):
                raise ValueError("DecodeChain: one (gamma_attn, gamma_mlp) pair a layer")
            self.norms = [tuple(X.dev(g, np.float32).reshape(-1) for g in pair) for pair in norms]
        self.rnorm = T.ones((len(layers), 2), dtype=f32, device=dev)
        self._graph = None
        self._plan = None
        self.persistent = self.persistent_fits() if persistent is None else bool(persistent)
        if self.persistent and not self.persistent_fits():
            raise ValueError("DecodeChain: the persistent step needs fused, folded int4 / fp4 layers with "
                             "hidden <= 2048, q_dim <= 2048, F <= 8192 (and 2 kv_dim <= 2048 where o "
                             "waits for k and v)")

    @staticmethod
    def synthetic(shape: Shape = Shape(), fmt: str = "int4", seed0: int = 100, std: float = 0.02,
                  fused: bool = True) -> "DecodeChain":
        """Random-init weights N(0, std), layer l from a generator seeded seed0 + l (the weights
        of each linear drawn in the order q, k, v, o, gate, up, down), packed on the GPU."""
        T = X.torch()
        layers = []
        for l in range(shape.layers):
            g = T.Generator(device="cuda").manual_seed(seed0 + l)
            h = shape.hidden

            def rnd(n, k):
                return T.randn((n, k), generator=g, device="cuda") * std
            Wq, Wk, Wv = rnd(shape.q_dim, h), rnd(shape.kv_dim, h), rnd(shape.kv_dim, h)
            Wo = rnd(h, shape.q_dim)
            Wg, Wu = rnd(shape.F, h), rnd(shape.F, h)
            Wd = rnd(h, shape.F)
            layers.append({"qkv": quantize_mxu(T.cat([Wq, Wk, Wv]), fmt), "o": quantize_mxu(Wo, fmt),
                           "gu": quantize_mxu(T.cat([Wg, Wu]), fmt), "down": quantize_mxu(Wd, fmt)})
            del Wq, Wk, Wv, Wo, Wg, Wu, Wd
        return DecodeChain(layers, shape, fmt, fused)

    @staticmethod
    def from_packed(layers: list, shape: Shape = Shape(), fmt: str = "int4", fused: bool = True,
                    norms: list | None = None) -> "DecodeChain":
        """Packed (rows, srows) pairs per layer (numpy or tensors), e.g. the reference's
        quantize_mxu output, loaded unchanged."""
        out = []
        for wts in layers:
            out.append({k: (X.dev(r, np.uint8), X.dev(sr, np.uint8)) for k, (r, sr) in wts.items()})
        return DecodeChain(out, shape, fmt, fused, norms)

    # --- the kernels of one step ---------------------------------------------------------
    def _norm(self, l: int, i: int):
        """(rscale, cscale) pointers of layer l's norm i (0: before qkv, 1: before gate / up)."""
        if self.norms is None:
            return None, None
        return C_ptr(self.rnorm, 2 * l + i), X.ptr(self.norms[l][i])

    def _qact(self, x, K: int, norm=(None, None)) -> None:
        X.call("otpu_qact", X.ptr(x), 1, K, x.stride(0), 32, 0, norm[0], norm[1], X.ptr(self.qa), self.qa.shape[1],
               X.ptr(self.Sa), X.ptr(self.da), self.da.shape[1], None, 0, X.stream())

    def _mm(self, w, K: int, out) -> None:
        rows, srows = w
        X.call("otpu_mm", X.ptr(self.qa), self.qa.shape[1], X.ptr(self.Sa), X.ptr(self.da), self.da.shape[1],
               1, K, X.ptr(rows), rows.shape[1], X.ptr(srows), srows.shape[1], rows.shape[0],
               X.FMT[self.fmt], 0, 0, None, X.ptr(out), out.shape[1], None, X.stream())

    def layer(self, l: int, x, y) -> None:
        """Queue layer l: input x [1, hidden] -> output y [1, hidden]."""
        s, w = self.shape, self.layers[l]
        self._qact(x, s.hidden, self._norm(l, 0))
        self._mm(w["qkv"], s.hidden, self.qkv)
        self._qact(self.qkv, s.q_dim)                     # q: the first q_dim columns
        self._mm(w["o"], s.q_dim, self.o)
        self._qact(self.o, s.hidden, self._norm(l, 1))
        self._mm(w["gu"], s.hidden, self.gu)
        g, u = self.gu[:, :s.F], self.gu[:, s.F:]
        X.call("otpu_qact_ranges", X.ptr(g), X.ptr(u), 1, s.F, self.gu.shape[1], self.width, 32, 0, None, None,
               X.ptr(self.qa), self.qa.shape[1], X.ptr(self.Sa), X.ptr(self.da), self.da.shape[1], X.stream())
        rows, srows = w["down"]
        X.call("otpu_mm_ranges", X.ptr(self.qa), self.qa.shape[1], X.ptr(self.Sa), X.ptr(self.da),
               self.da.shape[1], 1, s.F, self.width, X.ptr(rows), rows.shape[1], X.ptr(srows), srows.shape[1],
               rows.shape[0], X.FMT[self.fmt], 0, 0, X.ptr(self.part), X.ptr(y), y.shape[1], X.stream())

    def _qin(self, w, x, K: int, width: int, out, part_stride: int = 0, xmul=None, nsum: int = 1,
             sum_stride: int = 0, norm=(None, None)) -> None:
        rows, srows = w
        X.call("otpu_mm_qin", X.ptr(x), X.ptr(xmul), norm[0], norm[1], nsum, sum_stride, K, width, X.ptr(rows),
               rows.shape[1], X.ptr(srows), srows.shape[1], rows.shape[0], X.FMT[self.fmt], 0, 0, X.ptr(out),
               rows.shape[0], part_stride, X.stream())

    def layer_fused(self, l: int, x, nsum: int, parts) -> None:
        """Queue layer l fused: input = the in-order fold of the nsum rows of x ([nsum, hidden]);
        output = the down projection's per-chunk rows in parts ([R, hidden], not yet folded)."""
        s, w = self.shape, self.layers[l]
        self._qin(w["qkv"], x, s.hidden, s.hidden, self.qkv, nsum=nsum, sum_stride=s.hidden, norm=self._norm(l, 0))
        self._qin(w["o"], self.qkv, s.q_dim, s.q_dim, self.o)
        self._qin(w["gu"], self.o, s.hidden, s.hidden, self.gu, norm=self._norm(l, 1))
        self._qin(w["down"], self.gu, s.F, self.width, parts, part_stride=s.hidden, xmul=self.gu[:, s.F:])

    def layer_folded(self, l: int, x, y) -> None:
        """Queue layer l fused, its down projection folded in one launch: input x [1, hidden] ->
        output y [1, hidden]."""
        s, w = self.shape, self.layers[l]
        self._qin(w["qkv"], x, s.hidden, s.hidden, self.qkv, norm=self._norm(l, 0))
        self._qin(w["o"], self.qkv, s.q_dim, s.q_dim, self.o)
        self._qin(w["gu"], self.o, s.hidden, s.hidden, self.gu, norm=self._norm(l, 1))
        rows, srows = w["down"]
        X.call("otpu_mm_qin_fold", X.ptr(self.gu), X.ptr(self.gu[:, s.F:]), None, None, s.F, self.width,
               X.ptr(rows), rows.shape[1], X.ptr(srows), srows.shape[1], rows.shape[0], X.FMT[self.fmt], 0, 0,
               X.ptr(y), X.stream())

    # --- the persistent step ---------------------------------------------------------------
    def persistent_fits(self) -> bool:
        """Whether otpu_chain_step can run this chain (its phases' teams are compiled in)."""
        s = self.shape
        # o waits for k and v as well when the q/k/v rows (16 a workgroup) span more workgroups
        # than o's (4 a workgroup); that wait holds 2048 entries.  (The plan caps both counts at
        # the CUs; without the cap this test flags a superset, so a chain it passes is never
        # refused.)
        kv_wait = -(-(s.q_dim + 2 * s.kv_dim) // 16) > -(-s.hidden // 4)
        return (self.fused and self.fold and self.fmt in ("int4", "fp4", "nvfp4") and s.hidden <= 2048
                and s.hidden % 32 == 0 and s.q_dim <= 2048 and s.q_dim % 32 == 0 and s.F <= 8192 and s.F % 256 == 0
                and not (kv_wait and 2 * s.kv_dim > 2048))

    def _use_persistent(self) -> bool:
        return self.persistent and self.fused and self.fold

    def _plan_ptr(self) -> int:
        """The plan of otpu_chain_step (built once: the weights and every row buffer are fixed)."""
        if self._plan is not None:
            return self._plan[1]
        import ctypes as C
        s, n = self.shape, len(self.layers)
        lib = X.load()
        nbytes = lib.otpu_chain_plan_bytes(n, s.hidden, s.q_dim, s.kv_dim, s.F)
        if nbytes <= 0:
            raise ValueError("DecodeChain: no persistent plan for this shape")
        T = X.torch()
        buf = T.empty((nbytes + 256,), dtype=T.uint8, device="cuda")
        ptr = (buf.data_ptr() + 255) // 256 * 256
        P = C.c_void_p * (4 * n)
        I64 = C.c_int64 * (4 * n)
        w, ws, outs = P(), P(), P()
        rs, srs = I64(), I64()
        cs = (C.c_void_p * (2 * n))() if self.norms is not None else None
        for l in range(n):
            dst = self.y if l == n - 1 else self.hbuf[l % 2]
            for k, (name, out) in enumerate((("qkv", self.qkv), ("o", self.o), ("gu", self.gu), ("down", dst))):
                rows, srows = self.layers[l][name]
                j = 4 * l + k
                w[j], ws[j], outs[j] = X.ptr(rows), X.ptr(srows), X.ptr(out)
                rs[j], srs[j] = rows.shape[1], srows.shape[1]
            if cs is not None:
                cs[2 * l], cs[2 * l + 1] = X.ptr(self.norms[l][0]), X.ptr(self.norms[l][1])
        X.call("otpu_chain_plan", n, s.hidden, s.q_dim, s.kv_dim, s.F, self.width, X.FMT[self.fmt], w, rs, ws, srs,
               X.ptr(self.rnorm) if self.norms is not None else None, cs, X.ptr(self.x), outs, ptr, nbytes)
        self._plan = (buf, ptr)
        return ptr

    def chain_error(self) -> int:
        """The persistent plan's error word (0: every hand-off of every step so far completed).
        It reads device memory: call it after the steps it covers have finished."""
        if self._plan is None:
            return 0
        import ctypes as C
        e = C.c_uint32(0)
        X.call("otpu_chain_error", self._plan[1], C.byref(e))
        return int(e.value)

    def check(self) -> None:
        """Wait for the queued steps and raise OtpuError if a hand-off wait of the persistent
        step gave up (its workgroups were not all resident, e.g. CUs held by other work): the
        outputs of that step and of every later one are then invalid.  The word is sticky: a
        chain that failed stays failed (build a new DecodeChain).  The reference's simulator
        raises on a wait that can never hold (`opentpu/isasim.py:1383-1397`)."""
        if self._plan is None:
            return
        X.torch().cuda.synchronize()
        e = self.chain_error()
        if e:
            raise X.OtpuError(X.OTPU_ETIMEOUT, f"chain step: a hand-off wait timed out (error word {e}); "
                              "the step's outputs are invalid")

    @staticmethod
    def _capturing() -> bool:
        T = X.torch()
        return bool(T.cuda.is_current_stream_capturing())

    @property
    def kernels_per_step(self) -> int:
        n = len(self.layers)
        if self.fused and self._use_persistent():
            return 1
        if not self.fused:
            return n * self.KERNELS_PER_LAYER
        return n * self.FUSED_KERNELS_PER_LAYER + (0 if self.fold else 1)  # + the last otpu_acc_rows

    def _queue(self) -> None:
        n = len(self.layers)
        if self._use_persistent():
            X.call("otpu_chain_step", self._plan_ptr(), X.stream())
            return
        if self.fused and self.fold:
            src = self.x
            for l in range(n):
                dst = self.y if l == n - 1 else self.hbuf[l % 2]
                self.layer_folded(l, src, dst)
                src = dst
            return
        if self.fused:
            src, nsum = self.x, 1
            for l in range(n):
                dst = self.parts[l % 2]
                self.layer_fused(l, src, nsum, dst)
                src, nsum = dst, self.R
            X.call("otpu_acc_rows", X.ptr(src), self.R, self.shape.hidden, self.shape.hidden, None, X.ptr(self.y),
                   X.stream())
            return
        src = self.x
        for l in range(n):                                # outputs alternate so the last is self.y
            dst = self.y if (n - 1 - l) % 2 == 0 else self.y2
            self.layer(l, src, dst)
            src = dst

    def step(self, x=None, check: bool = True):
        """One decode step on input x [1, hidden] (fp32; default: the last input set):
        returns the device tensor holding the last layer's output.  check (the persistent step,
        outside a graph capture): wait for the step and raise OtpuError if a hand-off wait gave up
        (`check`); check=False queues it without waiting, and the caller calls check() later."""
        if x is not None:
            self.x.copy_(X.dev(x, np.float32).reshape(1, -1))
        self._queue()
        if check and self._plan is not None and not self._capturing():
            self.check()
        return self.y

    def capture(self) -> None:
        """Record one step (every layer's kernels) in a HIP graph; `replay` runs it on the
        current content of self.x."""
        T = X.torch()
        self._queue()                                     # warm-up outside the capture
        T.cuda.synchronize()
        self.check()
        g = T.cuda.CUDAGraph()
        with T.cuda.graph(g):
            self._queue()
        self._graph = g

    def replay(self, x=None, check: bool = True):
        """Replay the captured step on x (default: the current self.x).  check: as in step()."""
        if self._graph is None:
            self.capture()
        if x is not None:
            self.x.copy_(X.dev(x, np.float32).reshape(1, -1))
        self._graph.replay()
        if check and self._plan is not None:
            self.check()
        return self.y
