"""The MM operator and its callers on the GPU: `mm` (one MM instruction's work), `dot` (the
operator API: QACT per range, an MM per range accumulated with ACC, as the reference's
`Builder.dot`, `opentpu/compiler.py:2622-2726`), `lm_head_argmax` and `greedy` (the LM head's
greedy sink, `opentpu/llm/generate.py:251-286`), `argmax` (VOP ARGMAX).

Arrays: numpy in -> numpy out (copied through the device); device tensors stay on the device
and every call is queued on the current torch stream."""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import _lib as X
from . import fp32 as F
from .quant import D, WINDOW, quantize_mxu, row_bytes, scale_bytes

UNIT, ACC, RMAX, ASCALE, PAIR, RSC = X.UNIT, X.ACC, X.RMAX, X.ASCALE, X.PAIR, X.RSC


def _flags(unit=False, rsc=False, acc=False, ascale=False, rmax=False) -> int:
    return (UNIT if unit else 0) | (RSC if rsc else 0) | (ACC if acc else 0) | \
        (ASCALE if ascale else 0) | (RMAX if rmax else 0)


def mm(q, Sa, da, rows, srows, fmt: str, K: int, *, rsc: bool = False, unit: bool = False,
       k0: int = 0, acc=None, alpha=None, rmax: bool = False):
    """MM of activations (q int8 [M, K], Sa [M], da uint8 [M, K/32]: one QACT range) and weight
    rows (element rows [N, rs], scale rows [N, srs]; `opentpu/isasim.py:749-910`).

    acc: the old output [M, N] (ACC: y = old + mm; with alpha [M] also ASCALE:
    y = old * alpha + mm, needs unit).  rmax: also return the row maxima.  Returns y [M, N]."""
    numpy_in = X.is_numpy(q)
    qd = X.dev(q, np.int8)
    Sad = X.dev(Sa, np.float32)
    dad = X.dev(da, np.uint8)
    wd = X.dev(rows, np.uint8)
    sd = X.dev(srows, np.uint8) if srows is not None else None
    M, N = qd.shape[0], wd.shape[0]
    out = X.empty((M, N), np.float32) if acc is None else X.dev(acc, np.float32).clone()
    al = X.dev(alpha, np.float32) if alpha is not None else None
    rm = X.empty((M,), np.float32) if rmax else None
    fl = _flags(unit, rsc, acc is not None, alpha is not None, rmax)
    X.call("otpu_mm", X.ptr(qd), qd.shape[1], X.ptr(Sad), X.ptr(dad), dad.shape[1], M, K, X.ptr(wd),
           wd.shape[1], X.ptr(sd), sd.shape[1] if sd is not None else 0, N, X.FMT[fmt], fl, k0,
           X.ptr(al), X.ptr(out), N, X.ptr(rm), X.stream())
    if numpy_in:
        return (X.host(out), X.host(rm)) if rmax else X.host(out)
    return (out, rm) if rmax else out


def mm_acc(q, da, rows, srows, fmt: str, K: int, *, rsc: bool = False, unit: bool = False, k0: int = 0):
    """The exact int64 accumulators [M, N] of MM (no epilogue)."""
    numpy_in = X.is_numpy(q)
    qd, dad = X.dev(q, np.int8), X.dev(da, np.uint8)
    wd = X.dev(rows, np.uint8)
    sd = X.dev(srows, np.uint8) if srows is not None else None
    M, N = qd.shape[0], wd.shape[0]
    acc = X.empty((M, N), np.int64)
    X.call("otpu_mm_acc", X.ptr(qd), qd.shape[1], X.ptr(dad), dad.shape[1], M, K, X.ptr(wd), wd.shape[1],
           X.ptr(sd), sd.shape[1] if sd is not None else 0, N, X.FMT[fmt], _flags(unit, rsc), k0,
           X.ptr(acc), X.stream())
    return X.host(acc) if numpy_in else acc


def mm_spl(q, Sa, da, w_hi, w_lo, Sw, nterms: int, *, acc=None):
    """MM SPL (`opentpu/isasim.py:757-770`, `docs/isa.md:414-441`): one MM over a split
    operand's terms, one 128-block of int8 RSC weights a part.  q int8 [M, 128] (2 terms) or
    [M, 256] (3 terms: hi then lo, as `fp32.qact(hl=True)` gives them side by side), Sa [M] and
    da [M, 4] the hi part's, w_hi / w_lo the weights' hi and lo rows [N, 128] (`quantize_mxu(W,
    "int8", rsc=True)` and `(..., lo=True)`), Sw [N] the hi rows' scales.  acc: ACC into it."""
    numpy_in = X.is_numpy(q)
    qd = X.dev(q, np.int8)
    Sad, dad = X.dev(Sa, np.float32), X.dev(da, np.uint8)
    wh, wl = X.dev(w_hi, np.uint8), X.dev(w_lo, np.uint8)
    M, N = qd.shape[0], wh.shape[0]
    T = X.torch()
    w = T.cat([wh[:, :D], wl[:, :D]], 1).contiguous()     # hi rows, each followed by its lo row
    ws = X.dev(np.asarray(Sw, np.float32).reshape(-1) if X.is_numpy(Sw) else Sw, np.float32)
    out = X.empty((M, N), np.float32) if acc is None else X.dev(acc, np.float32).clone()
    X.call("otpu_mm_spl", X.ptr(qd), qd.shape[1], X.ptr(Sad), X.ptr(dad), dad.shape[1], M, nterms, X.ptr(w),
           2 * D, D, X.ptr(ws), 4, N, RSC | (ACC if acc is not None else 0), X.ptr(out), N, X.stream())
    return X.host(out) if numpy_in else out


def lm_head_argmax(q, Sa, da, rows, srows, fmt: str, K: int, *, rsc: bool = False, k0: int = 0,
                   base: int = 0, logits: bool = True):
    """One activation row times the vocabulary rows, with the greedy pick fused: returns
    (token, logits or None, best) where best = max over n of key(y_n) << 32 | ~(base + n)."""
    numpy_in = X.is_numpy(q)
    qd, Sad, dad = X.dev(q, np.int8), X.dev(Sa, np.float32), X.dev(da, np.uint8)
    wd, sd = X.dev(rows, np.uint8), X.dev(srows, np.uint8)
    N = wd.shape[0]
    lg = X.empty((N,), np.float32) if logits else None
    best = X.zeros((X.LM_STATE_BYTES // 8,), np.int64)   # the result word, the running maxima (zero)
    tok = X.empty((1,), np.int32)
    X.call("otpu_lm_head_argmax", X.ptr(qd), X.ptr(Sad), X.ptr(dad), K, X.ptr(wd), wd.shape[1], X.ptr(sd),
           sd.shape[1], N, X.FMT[fmt], _flags(rsc=rsc), k0, base, X.ptr(lg), X.ptr(best), X.ptr(tok),
           X.stream())
    if numpy_in:
        return (int(X.host(tok)[0]), X.host(lg) if logits else None,
                int(X.host(best).view(np.uint64)[0]))
    return tok, lg, best[:1]


def argmax(x, base: int = 0):
    """VOP ARGMAX of each row of x [rows, cols]: (max values [rows], first index + base [rows])
    (`opentpu/isasim.py:1141-1152`; the index comes back as the i2f'd fp32 the VOP writes)."""
    numpy_in = X.is_numpy(x)
    xd = X.dev(np.atleast_2d(x) if numpy_in else x, np.float32)
    if xd.dim() == 1:
        xd = xd.reshape(1, -1)
    rows, cols = xd.shape
    pairs = X.empty((rows, 2), np.float32)
    X.call("otpu_argmax", X.ptr(xd), rows, cols, cols, base, X.ptr(pairs), 2, X.stream())
    if numpy_in:
        p = X.host(pairs)
        return p[:, 0], p[:, 1].astype(np.int64)
    return pairs[:, 0], pairs[:, 1]


@dataclass
class QWeight:
    """A streamed weight resident on the device: element rows, scale rows, format, K (the
    reference's `runtime.Weight` once placed, `opentpu/runtime.py:38-51`; the descriptor
    `compiler.QTensor`).  rsc: the scale rows are Sw alone."""
    rows: object
    srows: object
    fmt: str
    K: int
    rsc: bool = False

    @property
    def N(self) -> int:
        return self.rows.shape[0]

    @staticmethod
    def from_float(W, fmt: str = "int8", rsc: bool = False) -> "QWeight":
        """Pack W [N, K] on the GPU (quantize_mxu) and keep it there."""
        Wd = X.dev(W, np.float32)
        rows, srows = quantize_mxu(Wd, fmt, rsc=rsc)
        return QWeight(rows, srows, fmt, Wd.shape[1], rsc)

    @staticmethod
    def from_packed(rows, srows, fmt: str, K: int, rsc: bool = False) -> "QWeight":
        """Rows packed elsewhere (e.g. by the reference's quantize_mxu): loaded unchanged."""
        if rows.shape[1] < row_bytes(K, fmt) or srows.shape[1] < scale_bytes(K, fmt, rsc):
            raise ValueError("QWeight: rows or scale rows shorter than the format's")
        return QWeight(X.dev(rows, np.uint8), X.dev(srows, np.uint8), fmt, K, rsc)


def quantize_ranges(x, ranges=None, row_mode: bool = False):
    """QACT of x [M, K] in column ranges (widths summing to K, each a multiple of 128; default
    one range): the int8 operand [M, K], Sa per range [n_ranges, M], da [M, K/32]."""
    xd = X.dev(x, np.float32)
    M, K = xd.shape
    ranges = [K] if ranges is None else list(ranges)
    if sum(ranges) != K or any(r % D for r in ranges):
        raise ValueError(f"quantize_ranges: ranges {ranges} over {K} columns")
    T = X.torch()
    q = X.empty((M, K), np.int8)
    da = X.empty((M, K // 32), np.uint8)
    Sa = X.empty((len(ranges), M), np.float32)
    c0 = 0
    for i, w in enumerate(ranges):
        xs = xd[:, c0:c0 + w]
        X.call("otpu_qact", X.ptr(xs), M, w, K, 32, X.Q_ROW if row_mode else 0, None, None, C_ptr(q, c0), K,
               X.ptr(Sa[i]), C_ptr(da, c0 // 32), K // 32, None, 0, X.stream())
        c0 += w
    del T
    return q, Sa, da, ranges


def C_ptr(t, off: int):
    import ctypes
    return ctypes.c_void_p(t.data_ptr() + off * t.element_size())


def dot(x, w: QWeight, acc=None, out=None, ranges=None, row_mode: bool = False, rowmax: bool = False,
        acc_scale=None):
    """x [M, K] (fp32, quantized here, or a (q, Sa, da, ranges) operand from quantize_ranges)
    @ w^T -> [M, N] fp32, as `ol.dot` lowers it: one QACT per range, one MM per range, the
    first overwriting (or ACC into `acc`, or ASCALE with acc_scale), the rest ACC.  The
    4-bit formats need ranges that start on even blocks (a 128-byte chunk holds two blocks).
    rowmax: also return the row maxima of the final sums (MM RMAX on the last range)."""
    numpy_in = X.is_numpy(x)
    if isinstance(x, tuple):
        q, Sa, da, ranges = x
    else:
        q, Sa, da, ranges = quantize_ranges(x, ranges, row_mode)
    M, K = q.shape
    if K != w.K:
        raise ValueError(f"dot: K mismatch {K} vs {w.K}")
    if acc is not None and out is not None:
        raise ValueError("dot: give either acc= or out=")
    N = w.N
    y = X.dev(acc, np.float32) if acc is not None else (out if out is not None else X.empty((M, N), np.float32))
    unit = w.srows is None
    bpb = D if w.fmt == "int8" else D // 2
    rm = X.empty((M,), np.float32) if rowmax else None
    al = X.dev(acc_scale, np.float32) if acc_scale is not None else None
    c0 = 0
    for i, width in enumerate(ranges):
        k0 = c0 // D
        first, last = i == 0, i == len(ranges) - 1
        accf = acc is not None or not first
        fl = _flags(unit, w.rsc, accf, al is not None and first, rowmax and last)
        X.call("otpu_mm", C_ptr(q, c0), K, X.ptr(Sa[i]), C_ptr(da, c0 // 32), K // 32, M, width,
               C_ptr(w.rows, k0 * bpb), w.rows.shape[1], X.ptr(w.srows), w.srows.shape[1] if not unit else 0,
               N, X.FMT[w.fmt], fl, 0 if (unit or w.rsc) else k0, X.ptr(al) if first else None, X.ptr(y), N,
               X.ptr(rm) if (rowmax and last) else None, X.stream())
        c0 += width
    if numpy_in:
        return (X.host(y), X.host(rm)) if rowmax else X.host(y)
    return (y, rm) if rowmax else y


class Greedy:
    """The LM head's greedy sink over vocabulary chunks (`opentpu/llm/generate.py:251-286`):
    each chunk's rows run through `lm_head_argmax` with its first row as the index base, and the
    token is the best over the chunks' (key << 32 | ~index) words, ties to the lowest index."""

    def __init__(self):
        self.best = 0

    def feed(self, best_word: int) -> None:
        self.best = max(self.best, best_word)

    def token(self) -> int:
        return int(~self.best & 0xFFFFFFFF)


def greedy(x, w: QWeight, chunk: int | None = None) -> int:
    """The greedy token of x [1, K] @ w^T (w: the LM head), in vocabulary chunks (all rows at
    once by default): the argmax of the fp32 logits, the lowest index on ties."""
    q, Sa, da = F.quantize_mx(X.dev(x, np.float32).reshape(1, -1), 32)
    N = w.N
    chunk = chunk or N
    g = Greedy()
    for c0 in range(0, N, chunk):
        n = min(chunk, N - c0)
        _, _, best = lm_head_argmax(q, Sa, da, w.rows[c0:c0 + n], w.srows[c0:c0 + n], w.fmt, w.K,
                                    rsc=w.rsc, base=c0, logits=False)
        g.feed(int(X.host(best).view(np.uint64)[0]))
    return g.token()


__all__ = ["mm", "mm_acc", "mm_spl", "lm_head_argmax", "argmax", "QWeight", "quantize_ranges", "dot", "Greedy",
           "greedy", "UNIT", "ACC", "RMAX", "ASCALE", "RSC", "WINDOW"]
