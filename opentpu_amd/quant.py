"""The MXU's streamed weight formats: byte layouts (`opentpu/quant.py:287-308`) and the packers
`quantize_mxu` (`opentpu/quant.py:510-523`) run on the GPU (HIP kernels, bit-exact with the
reference's numpy: int8x, RSC rows, int4x, fp4x6, nvfp4)."""
from __future__ import annotations

import numpy as np

from . import _lib as X

D = 128
MXU_FORMATS = ("int8", "int4", "fp4", "nvfp4")
WINDOW = {"int8": 16, "int4": 11, "fp4": 11, "nvfp4": 13}


def row_bytes(K: int, fmt: str) -> int:
    """Bytes of one streamed row of K elements (4-bit rows padded to whole 128-byte chunks)."""
    return K if fmt == "int8" else -(-K // (2 * D)) * D


def scale_bytes(K: int, fmt: str, rsc: bool = False) -> int:
    """Bytes of one scale row: Sw, then int8 a byte a block, int4 / fp4 a reserved word and a
    word a block, nvfp4 three reserved words and eight bytes a block, padded (4, 8, 16)."""
    if K % D:
        raise ValueError(f"inner dimension {K} is not a multiple of D={D}")
    KB = K // D
    if rsc:
        return 4
    if fmt == "int8":
        return 4 + 4 * -(-KB // 4)
    if fmt in ("int4", "fp4"):
        return 8 + 8 * -(-KB // 2)
    if fmt == "nvfp4":
        return 16 + 16 * -(-KB // 2)
    raise ValueError(f"unknown MXU format {fmt!r}")


def quantize_mxu(W, fmt: str, D: int = D, *, rsc: bool = False, lo: bool = False):
    """W [N, K] fp32 -> (element rows uint8 [N, row_bytes], scale rows uint8 [N, scale_bytes]),
    packed on the GPU (`opentpu/quant.py:510-523`; D the MXU depth, 128 on this path).  fmt
    "int8" (int8x; with rsc=True the RSC rows of one fp32 scale each, `opentpu/runtime.py:66-76`;
    with lo=True also the split's lo rows, QST LO: q8lo bytes and Sw * 2^-8), "int4", "fp4" or
    "nvfp4" (`opentpu/quant.py:368-400`).  numpy in, numpy out; tensors stay on the device."""
    if fmt not in MXU_FORMATS:
        raise ValueError(f"quantize_mxu: unknown MXU format {fmt!r}")
    if D != 128:
        raise ValueError(f"quantize_mxu: D {D}: the MM kernels stream blocks of 128")
    if lo and fmt != "int8":
        raise ValueError("quantize_mxu: the split's lo rows are int8")
    numpy_in = X.is_numpy(W)
    Wd = X.dev(W, np.float32)
    N, K = Wd.shape
    rb, sb = row_bytes(K, fmt), scale_bytes(K, fmt, rsc)
    srs = sb if fmt == "int8" else max(8, sb)
    rows = X.empty((N, rb), np.uint8)
    srows = X.empty((N, srs), np.uint8)
    if fmt == "int8":
        fl = (X.Q_ROW if rsc else 0) | (X.Q_LO if lo else 0)
        X.call("otpu_pack_int8", X.ptr(Wd), N, K, K, fl, X.ptr(rows), rb, X.ptr(srows), srs, X.stream())
    else:
        if rsc:
            raise ValueError("quantize_mxu: RSC rows are int8")
        X.call("otpu_pack_x4", X.ptr(Wd), N, K, K, X.FMT[fmt], X.ptr(rows), rb, X.ptr(srows), srs,
               X.stream())
    return (X.host(rows), X.host(srows)) if numpy_in else (rows, srows)


# ------------------------------------------------------------------------------ weight groups
# A reference machine of WG lanes stores an [N, K] weight in groups of R rows (R = WG int8, 2 WG
# 4-bit, 1 at WG = 1), optionally with its chunks' lanes in the channel hash's order at the
# image's address (`docs/isa.md` "Weight groups"; `opentpu/quant.py:634-808`, `grouped`). The
# converters below turn such an image back into the natural rows every MM entry point streams,
# on the GPU (`otpu_ungroup_rows`, `otpu_ungroup_scales`), MM KT's pairs included (`kt=True`:
# `opentpu/quant.py:829-880`, the natural rows of the padded K).

def grp_r(fmt: str, wg: int) -> int:
    """Rows of a group on a machine of wg lanes."""
    return wg if wg == 1 or fmt == "int8" else 2 * wg


def grp_row_bytes(K: int, fmt: str, wg: int) -> int:
    """The group stride of a grouped [., K] matrix (`opentpu/quant.py:672-679`)."""
    if wg == 1 or fmt == "int8":
        return row_bytes(K, fmt) * wg
    if K % D:
        raise ValueError(f"inner dimension {K} is not a multiple of D={D}")
    return (K // D) * wg * D


def grp_scale_bytes(K: int, fmt: str, wg: int, rsc: bool = False) -> int:
    """The group scale stride (`opentpu/quant.py:682-690`)."""
    if K % D:
        raise ValueError(f"inner dimension {K} is not a multiple of D={D}")
    R = grp_r(fmt, wg)
    sb = {"int8": 1, "int4": 4, "fp4": 4, "nvfp4": 8}[fmt]
    p = 4 * R if rsc or fmt == "int8" else ((16 if R == 1 else 8 * R) if fmt == "nvfp4"
                                            else (8 if R == 1 else 4 * R))
    n = p if rsc else p + (K // D) * R * sb
    return -(-n // p) * p


def _check_image(a, G: int, width: int, what: str):
    if a.dim() != 2 or a.shape[0] < G or a.shape[1] != width or not a.is_contiguous():
        raise ValueError(f"{what}: expected a contiguous [{G}, {width}] uint8 image, got {tuple(a.shape)}")


def kt_pair_bytes(K: int, fmt: str, wg: int) -> int:
    """The pair stride of a [., K] matrix in MM KT's pairs: (2 KB - 1) P (`opentpu/quant.py:836-839`)."""
    return 2 * grp_row_bytes(K, fmt, wg) - wg * D


def ungroup_rows(data, N: int, K: int, wg: int, fmt: str, at: int | None = None, kt: bool = False):
    """A grouped element image [ceil(N / R), grp_row_bytes] (uint8; `at`: its byte address on a
    machine with the channel hash, None: unhashed; kt: in MM KT's pairs, [ceil(G / 2),
    kt_pair_bytes], K the padded K) -> natural rows [N, row_bytes] on the GPU.  numpy in, numpy
    out."""
    if fmt not in MXU_FORMATS:
        raise ValueError(f"unknown MXU format {fmt!r}")
    if kt and (wg == 1 or fmt == "nvfp4"):
        raise ValueError("ungroup_rows: KT's pairs are of groups (wg > 1) of int8, int4 or fp4")
    numpy_in = X.is_numpy(data)
    d = X.dev(data, np.uint8)
    G = -(-N // grp_r(fmt, wg))
    if kt:
        _check_image(d, -(-G // 2), kt_pair_bytes(K, fmt, wg), "ungroup_rows")
    else:
        _check_image(d, G, grp_row_bytes(K, fmt, wg), "ungroup_rows")
    rows = X.empty((N, row_bytes(K, fmt)), np.uint8)
    X.call("otpu_ungroup_rows", X.ptr(d), N, K, wg, X.FMT[fmt], int(bool(kt)), -1 if at is None else int(at),
           X.ptr(rows), rows.shape[1], X.stream())
    return X.host(rows) if numpy_in else rows


def ungroup_scales(areas, N: int, K: int, wg: int, fmt: str, rsc: bool = False, kt: bool = False):
    """Grouped scale areas [ceil(N / R), grp_scale_bytes] (kt: MM KT's, the odd groups' entries
    in chunk order) -> natural scale rows [N, scale_bytes] on the GPU (reserved words and
    padding 0). numpy in, numpy out."""
    if fmt not in MXU_FORMATS:
        raise ValueError(f"unknown MXU format {fmt!r}")
    if kt and (wg == 1 or fmt == "nvfp4"):
        raise ValueError("ungroup_scales: KT's pairs are of groups (wg > 1) of int8, int4 or fp4")
    numpy_in = X.is_numpy(areas)
    a = X.dev(areas, np.uint8)
    G = -(-N // grp_r(fmt, wg))
    _check_image(a, G, grp_scale_bytes(K, fmt, wg, rsc), "ungroup_scales")
    srows = X.empty((N, scale_bytes(K, fmt, rsc)), np.uint8)
    X.call("otpu_ungroup_scales", X.ptr(a), N, K, wg, X.FMT[fmt], int(bool(rsc)), int(bool(kt)), X.ptr(srows),
           srows.shape[1], X.stream())
    return X.host(srows) if numpy_in else srows


def ungrouped(data, areas, N: int, K: int, wg: int, fmt: str, at: int | None = None, rsc: bool = False,
              kt: bool = False):
    """The inverse of the reference's `quant.grouped(q, s, fmt, K, wg, at=at, kt=kt)`
    (`opentpu/quant.py:811-826`): an image's (data, scale areas) -> (rows, scale rows) for MM
    (with kt, K is the padded K: a whole number of blocks)."""
    return ungroup_rows(data, N, K, wg, fmt, at, kt), ungroup_scales(areas, N, K, wg, fmt, rsc, kt)


# -------------------------------------------------------------------------- checkpoint imports
class NotExact(ValueError):
    """A checkpoint's quantized weights that no MXU format holds exactly (`opentpu/quant.py:1071`)."""


def _status(st) -> int:
    return int(np.bitwise_or.reduce(X.host(st).astype(np.int64))) if st.numel() else 0


def import_mxfp4(codes, e8m0, want: str | None = None):
    """An OCP MXFP4 matrix (E2M1 codes [N, K] one a byte, E8M0 exponents [N, K / 32]) in an MXU
    format, exactly, converted on the GPU: (rows, scale rows, "fp4" | "nvfp4")
    (`opentpu/quant.py:1084-1140`). fp4 where every K-block's live exponents span at most 5, else
    nvfp4 where every row's span at most 17, else NotExact; want forces a format. numpy in,
    numpy out."""
    if want not in (None, "fp4", "nvfp4"):
        raise ValueError(f"MXFP4 into {want!r}: fp4 or nvfp4")
    numpy_in = X.is_numpy(codes)
    c = X.dev(codes, np.uint8)
    e = X.dev(e8m0, np.uint8)
    N, K = c.shape
    if K % D or tuple(e.shape) != (N, K // 32):
        raise ValueError(f"MXFP4 [{N}, {K}] with scales {tuple(e.shape)}: blocks of 32, D = 128")
    st = X.empty((N,), np.int32)
    rows = X.empty((N, row_bytes(K, "fp4")), np.uint8)

    def run(fmt):
        srows = X.empty((N, scale_bytes(K, fmt)), np.uint8)
        X.call("otpu_import_mxfp4", X.ptr(c), K, X.ptr(e), K // 32, N, K, X.FMT[fmt], X.ptr(rows), rows.shape[1],
               X.ptr(srows), srows.shape[1], X.ptr(st), X.stream())
        return srows, _status(st)

    srows, s = run("nvfp4" if want == "nvfp4" else "fp4")
    if s & 1:
        raise NotExact("MXFP4: an E8M0 NaN scale")
    fmt = "nvfp4"
    if want != "nvfp4" and not s & 2:
        if s & 4:
            raise NotExact("MXFP4: a block more than 255 octaves below its row's top")
        if s & 8:
            raise NotExact("MXFP4: a row scale outside fp32's normal range")
        fmt = "fp4"
    elif want == "fp4":
        raise NotExact("MXFP4: a K-block's exponents span more than fp4's 5 octaves")
    else:
        if want != "nvfp4":
            srows, s = run("nvfp4")
        if s & 16:
            raise NotExact("MXFP4: a row's scales span more than 17 octaves, nvfp4's E4M3 holds 17 "
                           "with mantissa 0")
        if s & 32:
            raise NotExact("MXFP4: a row scale outside fp32's normal range")
    return (X.host(rows), X.host(srows), fmt) if numpy_in else (rows, srows, fmt)


def import_nvfp4(codes, e4m3_scales, tensor_scale: float):
    """An NVFP4 matrix (E2M1 codes [N, K] one a byte, E4M3 scales [N, K / 16], the per-tensor
    fp32 scale) in the MXU's nvfp4, exactly, converted on the GPU: (rows, scale rows)
    (`opentpu/quant.py:1143-1182`). numpy in, numpy out."""
    numpy_in = X.is_numpy(codes)
    c = X.dev(codes, np.uint8)
    sc = X.dev(e4m3_scales, np.uint8)
    N, K = c.shape
    if K % D or tuple(sc.shape) != (N, K // 16):
        raise ValueError(f"NVFP4 [{N}, {K}] with scales {tuple(sc.shape)}: groups of 16, D = 128")
    st = X.empty((N,), np.int32)
    rows = X.empty((N, row_bytes(K, "nvfp4")), np.uint8)
    srows = X.empty((N, scale_bytes(K, "nvfp4")), np.uint8)
    X.call("otpu_import_nvfp4", X.ptr(c), K, X.ptr(sc), K // 16, float(np.float32(tensor_scale)), N, K,
           X.ptr(rows), rows.shape[1], X.ptr(srows), srows.shape[1], X.ptr(st), X.stream())
    s = _status(st)
    if s & 1:
        raise NotExact("NVFP4: a negative E4M3 scale")
    if s & 2:
        raise NotExact("NVFP4: an E4M3 NaN scale")
    if s & 4:
        raise NotExact("NVFP4: a scale more than 14 octaves below its row's largest whose low bits an "
                       "MXU subnormal does not hold")
    if s & 8:
        raise NotExact("NVFP4: a row scale outside fp32's normal range")
    return (X.host(rows), X.host(srows)) if numpy_in else (rows, srows)


# ---------------------------------------------------------------------------- float64 emulation
# The reference's float64 emulation of the operator (`opentpu/quant.py:895-1067`), on the GPU:
# what model code checks the machine against.  The signatures are the reference's.  numpy in,
# numpy out: MXAct / MXW are ndarray subclasses, as the reference's are, and `@` with an MXW sums
# as MM does (the GPU's mx_matmul, leaving out the 16-element groups MM's window drops).  Torch
# tensors in: DeviceMXAct / DeviceMXW hold device tensors and give the same `@`.

NVG = 8                           # drop groups a block: each of D / 8 = 16 elements
EG = D // NVG


def _check_D(D: int, what: str) -> None:
    if D != 128:
        raise ValueError(f"{what}: D {D}: the MM kernels work in blocks of 128")


class MXAct(np.ndarray):
    """Activations as QACT leaves them (float64 values) with `da`, each 16-element group's
    offset below its row's scale [..., K / 16] (`opentpu/quant.py:896-913`).  A slice, reshape or
    arithmetic result of one is a plain one again (da None): only `rows` keeps the offsets."""

    def __array_finalize__(self, obj):
        self.da = None

    @staticmethod
    def of(values, da) -> "MXAct":
        a = np.asarray(values).view(MXAct)
        a.da = None if da is None else np.asarray(da)
        return a

    def rows(self, sl) -> "MXAct":
        """The rows sl (an index or slice of the leading axes), offsets included."""
        return MXAct.of(self.view(np.ndarray)[sl], None if self.da is None else self.da[sl])


class MXW(np.ndarray):
    """A weight as the MXU holds it (`opentpu/quant.py:916-960`): float64 (or float32) values
    [N, K] with `mx` = (dw [N or 1, K / 16], the window W, D, transposed).  `h @ w.T` (h [..., K])
    and `w @ h` (h [K]) sum as MM does: mx_matmul with w's offsets and window, on the GPU.  Any
    other derived array (a slice, arithmetic) is a plain one."""

    def __array_finalize__(self, obj):
        self.mx = None

    @staticmethod
    def of(values, dw, W: int, D: int = 128) -> "MXW":
        v = np.asarray(values)
        w = (v if v.dtype in (np.float32, np.float64) else v.astype(np.float64)).view(MXW)
        w.mx = (np.asarray(dw), W, D, False)
        return w

    def astype(self, dtype, *a, **kw):
        vals = self.view(np.ndarray).astype(dtype, *a, **kw)
        if self.mx is None or self.mx[3]:
            return vals
        return MXW.of(vals, self.mx[0], self.mx[1], self.mx[2])

    @property
    def T(self):
        t = np.ndarray.transpose(self).view(MXW)
        if self.mx is not None:
            dw, W, D, tr = self.mx
            t.mx = (dw, W, D, not tr)
        return t

    def __array_ufunc__(self, ufunc, method, *inputs, **kw):
        if ufunc is np.matmul and method == "__call__" and not kw and len(inputs) == 2:
            a, b = inputs
            if isinstance(b, MXW) and b.mx is not None and b.mx[3]:            # h @ w.T
                dw, W, D, _ = b.mx
                return mx_matmul(a, b.view(np.ndarray).T, dw, W, D)
            if isinstance(a, MXW) and a.mx is not None and not a.mx[3] and np.ndim(b) == 1:
                dw, W, D, _ = a.mx                                              # w @ h
                return mx_matmul(b, a.view(np.ndarray), dw, W, D)
        plain = [x.view(np.ndarray) if isinstance(x, np.ndarray) else x for x in inputs]
        if "out" in kw:
            kw["out"] = tuple(o.view(np.ndarray) if isinstance(o, np.ndarray) else o for o in kw["out"])
        return getattr(ufunc, method)(*plain, **kw)


class DeviceMXAct:
    """MXAct's device form (torch inputs): values float64 [..., K] and da uint8 [..., K / 16],
    both device tensors; `h @ w.T` with a DeviceMXW sums as MM does."""

    def __init__(self, values, da):
        self.values, self.da = values, da

    @property
    def shape(self):
        return tuple(self.values.shape)

    def __matmul__(self, other):
        if isinstance(other, DeviceMXW) and other.transposed:
            return mx_matmul(self, other.values, other.dw, other.W, other.D)
        return NotImplemented


class DeviceMXW:
    """MXW's device form: values float64 [N, K], dw uint8 [N or 1, K / 16] (device tensors), the
    window W; `.T` marks it transposed for `h @ w.T`; `w @ h` takes a 1-D h."""

    def __init__(self, values, dw, W: int, D: int = 128, transposed: bool = False):
        self.values, self.dw, self.W, self.D, self.transposed = values, dw, W, D, transposed

    @property
    def T(self):
        return DeviceMXW(self.values, self.dw, self.W, self.D, not self.transposed)

    def __rmatmul__(self, h):
        if self.transposed:
            return mx_matmul(h, self.values, self.dw, self.W, self.D)
        return NotImplemented

    def __matmul__(self, h):
        if not self.transposed and len(getattr(h, "shape", ())) == 1:
            return mx_matmul(h, self.values, self.dw, self.W, self.D)
        return NotImplemented


def _fake_act_dev(xd, n: int, row: bool, g: int):
    """One QACT range width n over the rows of the device tensor xd [M, K] (float32 or float64)
    -> (values [M, K] float64, da [M, K / 16] uint8)."""
    M, K = xd.shape
    v = X.empty((M, K), np.float64)
    da = X.empty((M, K // EG), np.uint8)
    fn = "otpu_fake_act" if xd.dtype == X.torch().float32 else "otpu_fake_act_f64"
    X.call(fn, X.ptr(xd), M, K, K, n, g, int(bool(row)), X.ptr(v), K, X.ptr(da), K // EG, X.stream())
    return v, da


def fake_act(x, D: int = 128, n=None, row: bool = False, g: int | None = None):
    """x [..., K] quantized as QACT / QST quantize it, in float64 (`opentpu/quant.py:972-1023`):
    each row in ranges of n columns (one QACT each; None: the whole row; a sequence: the ranges'
    widths in order) has S = amax / 127, its groups of g (None: D / 4, QACT's; D: QST's) the
    offset d (0 in ROW mode) and the values rint(x 127 / amax 2^d) S 2^-d clipped to 127, a value
    within 2^-31 of a tie rounded as the device's fp32 quantizer rounds it.  Returns an MXAct
    (numpy x; da int64 per 16 elements) or a DeviceMXAct (a tensor x).  Computed on the GPU;
    float32 x is read as float32, anything else as float64 (as the reference reads it)."""
    _check_D(D, "fake_act")
    T = X.torch()
    numpy_in = not isinstance(x, T.Tensor)
    if numpy_in:
        xa = np.asarray(x)
        xa = xa if xa.dtype in (np.float32, np.float64) else xa.astype(np.float64)
        xd = X.dev(xa, xa.dtype)
    else:
        xd = x if x.dtype in (T.float32, T.float64) else x.to(T.float64)
        xd = xd.cuda().contiguous()
    sh = tuple(xd.shape)
    K = sh[-1]
    g = D // 4 if g is None else int(g)
    rows = xd.reshape(-1, K)
    if n is not None and not isinstance(n, (int, np.integer)):
        widths = [int(w) for w in n]
        if sum(widths) != K:
            raise ValueError(f"fake_act: ranges {widths} over {K} columns")
    else:
        n = K if n is None else int(n)
        if n < 1 or K % n or n % g:
            raise ValueError(f"fake_act: ranges of {n} over {K} columns, groups of {g}")
        widths = [n] * (K // n)
    if len(set(widths)) == 1:                             # equal ranges: one launch
        v, da = _fake_act_dev(rows, widths[0], row, g)
    else:
        parts, c = [], 0
        for w in widths:
            parts.append(_fake_act_dev(rows[:, c:c + w].contiguous(), w, row, g))
            c += w
        v = T.cat([p[0] for p in parts], 1)
        da = T.cat([p[1] for p in parts], 1)
    v = v.reshape(sh)
    da = da.reshape(sh[:-1] + (K // EG,))
    if not numpy_in:
        return DeviceMXAct(v, da)
    return MXAct.of(X.host(v), X.host(da).astype(np.int64))


def _dequant(rows, srows, fmt: str, K: int, rsc: bool, values: bool, offsets: bool):
    if fmt not in MXU_FORMATS:
        raise ValueError(f"unknown MXU format {fmt!r}")
    s = None if srows is None else X.dev(srows, np.uint8)
    r = X.dev(rows, np.uint8) if values else None
    N = (r if r is not None else s).shape[0]
    v = X.empty((N, K), np.float64) if values else None
    dw = X.empty((N, K // EG), np.uint8) if offsets else None
    X.call("otpu_dequant", X.ptr(r), 0 if r is None else r.shape[1], X.ptr(s), 0 if s is None else s.shape[1], N, K,
           X.FMT[fmt], int(bool(rsc)), X.ptr(v), K, X.ptr(dw), K // EG, X.stream())
    return v, dw


def dequantize_mxu(rows, srows, fmt: str, K: int, D: int = 128, rsc: bool = False):
    """The matrix [N, K] (float64) that MXU rows and their scale rows stand for, w m 2^-dw Sw
    (srows None: UNIT, the elements themselves; a denormal Sw is 0), exact, on the GPU
    (`opentpu/quant.py:460-473`).  numpy in, numpy out."""
    _check_D(D, "dequantize_mxu")
    v, _ = _dequant(rows, srows, fmt, K, rsc, True, False)
    return X.host(v) if X.is_numpy(rows) else v


def group_offsets(srows, fmt: str, K: int, D: int = 128, rsc: bool = False):
    """Each 16-element group's weight offset dw [N, K / 16] (MM's drop rule) from scale rows, on
    the GPU (`opentpu/quant.py:476-481`).  numpy in: int64 out; a tensor in: uint8 tensor out."""
    _check_D(D, "group_offsets")
    _, dw = _dequant(None, srows, fmt, K, rsc, False, True)
    return X.host(dw).astype(np.int64) if X.is_numpy(srows) else dw


def fake_w(W, fmt: str, D: int = 128, quantized: tuple | None = None, *, rsc: bool = False):
    """W [N, K] as the MXU holds it in format fmt (`opentpu/quant.py:963-969`): packed on the GPU
    (quantize_mxu, or `quantized` = its (rows, scale rows) already), dequantized, with its groups'
    offsets and the format's window.  An MXW (numpy W) or a DeviceMXW (a tensor W).  rsc: int8 RSC
    rows (one fp32 scale a row)."""
    _check_D(D, "fake_w")
    numpy_in = X.is_numpy(W)
    K = int(np.shape(W)[1]) if numpy_in else int(W.shape[1])
    rows, srows = quantize_mxu(X.dev(W, np.float32), fmt, rsc=rsc) if quantized is None else quantized
    v, dw = _dequant(rows, srows, fmt, K, rsc, True, True)
    if not numpy_in:
        return DeviceMXW(v, dw, WINDOW[fmt], D)
    return MXW.of(X.host(v), X.host(dw).astype(np.int64), WINDOW[fmt], D)


def mx_matmul(h, w, dw=None, W: int = 16, D: int = 128):
    """h @ w.T in float64 as MM sums it (`opentpu/quant.py:1042-1067`), on the GPU: w [N, K] the
    streamed matrix's values (an MXW counts as its values), dw [N or 1, K / 16] its groups'
    offsets (None: 0) and W the format's window; h [..., K] an MXAct / DeviceMXAct (a plain
    array: no offsets known, nothing dropped).  The groups whose two offsets add up to more than
    W are left out.  numpy h: numpy out ([..., N]); else a device tensor."""
    _check_D(D, "mx_matmul")
    T = X.torch()
    if isinstance(h, DeviceMXAct):
        hv, da, numpy_out = h.values, h.da, False
    elif isinstance(h, T.Tensor):
        hv, da, numpy_out = h, None, False
    else:
        da = getattr(h, "da", None)
        hv, numpy_out = np.asarray(h).view(np.ndarray), True
    hd = X.dev(hv, np.float64)
    lead = tuple(hd.shape[:-1])
    K = hd.shape[-1]
    hd = hd.reshape(-1, K)
    wv = X.dev(np.asarray(w).view(np.ndarray) if isinstance(w, np.ndarray) else w, np.float64)
    N = wv.shape[0]
    if wv.shape[1] != K:
        raise ValueError(f"mx_matmul: h has {K} columns, w {wv.shape[1]}")
    dad = None if da is None else X.dev(da, np.uint8).reshape(-1, K // EG)
    dwd = None
    if dw is not None and da is not None:
        dwd = X.dev(dw, np.uint8)
        dwd = dwd.reshape(1, -1) if dwd.dim() == 1 else dwd
    M = hd.shape[0]
    y = X.empty((M, N), np.float64)
    X.call("otpu_mx_matmul", X.ptr(hd), K, X.ptr(dad), K // EG, X.ptr(wv), wv.shape[1], X.ptr(dwd), K // EG,
           0 if dwd is None else dwd.shape[0], int(W), M, N, K, X.ptr(y), N, X.stream())
    y = y.reshape(lead + (N,))
    return X.host(y) if numpy_out else y
