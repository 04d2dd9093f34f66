"""Oracle: the reference's float64 emulation of the operator (numpy). TEST INFRASTRUCTURE ONLY.

Restated from `opentpu/quant.py:895-1067` (fake_act, group_offsets with dequantize_mxu as
fake_w's values, mx_matmul):
  * fake_act: per range of n columns s = amax / 127 (1 for a zero range); per group of g the
    offset d, the largest (<= 31) with the group's amax 2^d <= amax, from frexp (0 in row mode);
    unit = s 2^-d; q = rint(x / unit), except where x / unit lies within 2^-31 of a tie: there
    the device quantizer's q (fp32.quantize_mx of the range); values clip(q, +-127) unit; da:
    each 16-element group's d;
  * group_offsets: each 16-element group's dw from the scale rows;
  * mx_matmul: y = h @ w.T, then for every 16-element group whose offsets add up to more than W
    the group's products taken out again.

Pinning (tests/test_oracle_emulate.py): by what the emulation must equal -- the exact operator.
mx_matmul(fake_act(x), fake_w(W)) is s Sw 2^-W acc with acc the exact integer accumulator of the
pinned oracle MM (oracle/mm.py), to float64 rounding; the machine's fp32 MM agrees with it to
fp32 rounding while the undropped product does not (the reference's own check,
`tests/test_quant.py:218-241`, restated); fake_act's q equals the pinned quantizer's wherever
that is not within fp32 rounding of a tie, and its values are exact multiples of unit.
"""
from __future__ import annotations

import numpy as np

from . import formats as Q
from . import fp32 as F

EG = 16                                   # a drop group: D / 8 elements


def fake_act(x, n: int | None = None, row: bool = False, g: int = 32):
    """(values float64 [..., K], da uint8 [..., K / 16])."""
    x = np.asarray(x, np.float64)
    sh = x.shape
    K = sh[-1]
    n = K if n is None else n
    xr = x.reshape(-1, n)
    amax = np.abs(xr).max(-1, keepdims=True)
    xb = xr.reshape(len(xr), n // g, g)
    ag = np.abs(xb).max(-1)
    if row:
        d = np.zeros(ag.shape, np.int64)
    else:
        fa, ea = np.frexp(ag)
        fm, em = np.frexp(np.broadcast_to(amax, ag.shape))
        d = np.where(ag > 0, np.clip(em - ea - (fa > fm), 0, 31), 0)
    s = np.where(amax == 0, 1.0, amax / 127)
    unit = s * np.exp2(-d)
    r = xb / unit[..., None]
    q = np.rint(r)
    tie = np.abs(r - q) > 0.5 - 2.0 ** -31
    if tie.any():
        qd = F.quantize_mx(xr.astype(np.float32), g, row)[0].astype(np.float64).reshape(q.shape)
        q = np.where(tie, qd, q)
    vals = (np.clip(q, -127, 127) * unit[..., None]).reshape(sh)
    da = np.repeat(d, g // EG, axis=-1).reshape(*sh[:-1], K // EG).astype(np.uint8)
    return vals, da


def group_offsets(srows, fmt: str, K: int, rsc: bool = False) -> np.ndarray:
    """dw of every 16-element group [N, K / 16] (uint8)."""
    _, dw, _ = Q.unpack_scales(srows, fmt, K // Q.D, rsc=rsc)
    return np.repeat(dw, Q.NVG // dw.shape[2], axis=2).reshape(dw.shape[0], -1).astype(np.uint8)


def fake_w(rows, srows, fmt: str, K: int, rsc: bool = False):
    """(values float64 [N, K], dw [N, K / 16]) of packed rows."""
    return Q.dequantize(rows, srows, fmt, K, rsc=rsc), group_offsets(srows, fmt, K, rsc)


def mx_matmul(h, w, da=None, dw=None, W: int = 16) -> np.ndarray:
    """h [M, K] @ w [N, K]^T in float64, the groups with da + dw > W taken out (da None: none)."""
    h = np.asarray(h, np.float64)
    w = np.asarray(w, np.float64)
    y = h @ w.T
    if da is None:
        return y
    K = w.shape[1]
    dw = np.zeros((1, K // EG), np.int64) if dw is None else np.asarray(dw, np.int64)
    dg = np.asarray(da, np.int64).reshape(-1, K // EG)
    for gi in range(K // EG):
        m = (dg[:, gi][:, None] + dw[None, :, gi].reshape(1, -1)) > W      # [M, N or 1]
        if not m.any():
            continue
        sl = slice(EG * gi, EG * (gi + 1))
        y -= (h[:, sl] @ w[:, sl].T) * m
    return y
