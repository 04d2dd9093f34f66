"""Oracle: checkpoint imports of OCP MXFP4 and NVFP4 weights into the MXU's formats, exactly
(numpy). TEST INFRASTRUCTURE ONLY.

Restated from `opentpu/quant.py:1070-1182` (import_mxfp4, import_nvfp4) and `docs/quant.md`
"Checkpoint imports":
  * MXFP4 (E2M1 codes, one E8M0 exponent e per 32, value E2M1 x 2^(e - 127)): fp4 (fp4x6) when
    every K-block's live sub-blocks span at most 5 octaves: m = 2^(e - the block's smallest live
    e), dw = the row's top (the largest of its blocks' smallest live e) - the block's smallest,
    Sw = 2^(top - 128) (the MXU's fp4 codes are twice E2M1); else nvfp4 when each row's live
    exponents span at most 17: E4M3 bytes of mantissa 0 (exponent field 15 - span; the three
    spans past 14 the subnormals 4, 2, 1), one per 16 elements, Sw = 2^(top - 131); else
    NotExact. A sub-block whose codes are all +-0 is not live (any exponent).
  * NVFP4 (E2M1 codes, one E4M3 scale per 16, an fp32 tensor scale ts): each scale m 2^p is
    renormalized to m' in 8..15 and re-based on the row's largest (dw = top - p'); dw <= 14 is
    the byte ((15 - dw) << 3) | (m' - 8), dw 15..17 an MXU subnormal m' >> (dw - 14) when no
    set bit falls off; Sw = ts 2^(top - 1). NotExact on a negative or NaN scale, a subnormal
    that loses bits, dw > 17, or Sw outside fp32's normal range.

Pinning (tests/test_oracle_imports.py): by what exactness fixes -- the MXU's dequantization of
the imported rows equals the checkpoint's decoded values (E2M1 x 2^(e - 127), E2M1 x E4M3 x ts)
exactly for both formats -- and by the reference's own import checks (`tests/test_quant.py:
376-470`: the format chosen for spans 5 / 17 / 18, the zero sub-block, the NotExact cases, the
mantissa-7 top, the two subnormals 17 octaves down) restated with their own inputs.
"""
from __future__ import annotations

import numpy as np

from .formats import D, NSUB, NVG, pack_nibbles, pack_scales, row_bytes

DW_MAX = 255


class NotExact(ValueError):
    """A checkpoint's quantized weights that no MXU format holds exactly."""


def _pow2_f32(e, what: str) -> np.ndarray:
    e = np.asarray(e, np.int64)
    if np.any(e < -126) or np.any(e > 127):
        raise NotExact(f"{what}: a row scale 2^{int(e.min())}..2^{int(e.max())} outside fp32's normal range")
    return np.ldexp(np.float32(1.0), e.astype(np.int32)).astype(np.float32)


def _rows(codes, K):
    rows = np.zeros((codes.shape[0], row_bytes(K, "fp4")), np.uint8)
    rows[:, :K // 2] = pack_nibbles(codes)
    return rows


def import_mxfp4(codes, e8m0, want: str | None = None):
    """(rows, scale rows, format) of an OCP MXFP4 matrix: codes [N, K] uint8 (0..15, sign bit 3),
    e8m0 [N, K / 32]; want "fp4" / "nvfp4" forces that format (or NotExact)."""
    codes = np.asarray(codes, np.uint8)
    e = np.asarray(e8m0, np.int64)
    N, K = codes.shape
    if K % D or e.shape != (N, K // 32):
        raise ValueError(f"MXFP4 [{N}, {K}] with scales {e.shape}: blocks of 32, D = 128")
    if want not in (None, "fp4", "nvfp4"):
        raise ValueError(f"MXFP4 into {want!r}: fp4 or nvfp4")
    if np.any(e == 0xFF):
        raise NotExact("MXFP4: an E8M0 NaN scale")
    KB = K // D
    live = np.any(codes.reshape(N, K // 32, 32) & 7, axis=-1).reshape(N, KB, NSUB)
    eb = e.reshape(N, KB, NSUB)
    blive = live.any(-1)
    lo = np.min(np.where(live, eb, 1 << 30), axis=-1)                  # block's smallest live e
    hi = np.max(np.where(live, eb, -(1 << 30)), axis=-1)
    rows = _rows(codes, K)
    if want != "nvfp4" and not np.any(blive & (hi - lo > 5)):
        top = np.max(np.where(blive, lo, -(1 << 30)), axis=-1)         # [N]
        top = np.where(blive.any(-1), top, 129)
        dw = np.where(blive, top[:, None] - lo, 0)
        if np.any(dw > DW_MAX):
            raise NotExact("MXFP4: a block more than 255 octaves below its row's top")
        sh = np.where(live, eb - np.where(blive, lo, 0)[..., None], 0)
        m = np.left_shift(1, sh).astype(np.uint8)
        Sw = _pow2_f32(top - 128, "MXFP4")
        return rows, pack_scales("fp4", Sw, dw=dw.astype(np.uint8), m=m), "fp4"
    if want == "fp4":
        raise NotExact("MXFP4: a K-block's exponents span more than fp4's 5 octaves")
    el = live.reshape(N, K // 32)
    top = np.max(np.where(el, e, -(1 << 30)), axis=-1)
    span = np.where(el, top[:, None] - e, 0)
    if np.any(span > 17):
        raise NotExact(f"MXFP4: a row's scales span {int(span.max())} octaves, nvfp4's E4M3 "
                       f"holds 17 with mantissa 0")
    E = 15 - span
    byte = np.select([E >= 1, E == 0, E == -1], [E << 3, 4, 2], 1)
    byte = np.where(el, byte, 0)
    e4 = np.repeat(byte, 2, axis=1).reshape(N, KB, NVG).astype(np.uint8)
    top = np.where(el.any(-1), top, 131)
    return rows, pack_scales("nvfp4", _pow2_f32(top - 131, "MXFP4"), e4=e4), "nvfp4"


def import_nvfp4(codes, e4m3_scales, tensor_scale: float):
    """(rows, scale rows) of an NVFP4 matrix: codes [N, K] uint8, E4M3 scales [N, K / 16] uint8,
    the per-tensor fp32 scale."""
    codes = np.asarray(codes, np.uint8)
    s = np.asarray(e4m3_scales, np.uint8).astype(np.int64)
    N, K = codes.shape
    if K % D or s.shape != (N, K // 16):
        raise ValueError(f"NVFP4 [{N}, {K}] with scales {s.shape}: groups of 16, D = 128")
    if np.any(s & 0x80):
        raise NotExact("NVFP4: a negative E4M3 scale")
    if np.any(s == 0x7F):
        raise NotExact("NVFP4: an E4M3 NaN scale")
    E, M = s >> 3, s & 7
    m = np.where(E > 0, 8 + M, M)
    p = np.maximum(E, 1) - 10                                           # value m 2^p
    live = m > 0
    nb = np.zeros_like(m)                                               # bit length - 1 of m
    for b in range(1, 4):
        nb = np.where(m >> b > 0, b, nb)
    sh = np.where(live, 3 - nb, 0)
    mn, pn = m << sh, p - sh                                            # m' in 8..15
    top = np.max(np.where(live, pn, -(1 << 30)), axis=-1)
    top = np.where(live.any(-1), top, 1)
    dw = np.where(live, top[:, None] - pn, 0)
    drop = np.clip(dw - 14, 0, 3)
    sub = live & (dw > 14)
    ms = np.where(sub, mn >> drop, 0)
    if np.any(dw > 17) or np.any(sub & ((ms << drop) != mn)):
        raise NotExact("NVFP4: a scale more than 14 octaves below its row's largest whose low "
                       "bits an MXU subnormal does not hold")
    byte = np.where(~live, 0, np.where(dw <= 14, ((15 - dw) << 3) | (mn - 8), ms))
    sw = np.float64(np.float32(tensor_scale)) * np.exp2(top - 1.0)
    if np.any((sw != 0) & ((np.abs(sw) < 2.0 ** -126) | (np.abs(sw) >= 2.0 ** 128))):
        raise NotExact("NVFP4: a row scale outside fp32's normal range")
    return _rows(codes, K), pack_scales("nvfp4", sw.astype(np.float32),
                                        e4=byte.reshape(N, K // D, NVG).astype(np.uint8))
