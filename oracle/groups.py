"""Oracle: the reference machine's grouped weight layouts (numpy). TEST INFRASTRUCTURE ONLY.

Restated from `docs/isa.md` "Weight groups" (`docs/isa.md:319-365`) and `opentpu/quant.py:634-808`
(grp_r, swp, grp_row_bytes, grp_scale_bytes, group_rows, chunk_fold, hash_rows, ungroup_rows,
group_scales, ungroup_scales). A machine of WG lanes stores an [N, K] weight in groups of R rows
(R = WG for int8, 2 WG for a 4-bit format, 1 at WG = 1); group g's chunk c (P = WG x D bytes,
K-block c of the group's rows) lies at g * grp_row_bytes + c * P and its lane l (D bytes) at
+ l * D:
  * int8: lane l is row g R + l's block c;
  * 4-bit: lane l's byte i is element i of block c of row g R + 2l (bits 3:0) and of row
    g R + 2l + 1 (bits 7:4).
With the channel hash the chunk at byte address A keeps lane l at A + (l ^ h) * D, h the XOR
fold of A / P into log2 WG bits. Group g's scale area (grp_scale_bytes apart): row j's Sw word
at 4 j, then from SWP on block k's data of row j (SB bytes: int8 1, int4 / fp4 4, NVFP4 8, RSC
none) at SWP + (k R + j) SB.

The functions below build every map one byte address at a time from those formulas (the
reference reshapes whole arrays), so a transposed axis or a wrong stride shows up as a byte in
the wrong place. Pinning (tests/test_oracle_groups.py): the chunk fold's known answer
(0b100_011_110 at R 8 folds to 1; R 1 folds to 0) from the reference's
`tests/test_wg.py:125-137`; the scale-area offsets and 4-bit chunk layout checks of
`tests/test_wg.py:178-216` restated with their own inputs; WG = 1 the natural layout byte for
byte; group/ungroup and hash/hash round trips; area and row sizes against the closed forms.
"""
from __future__ import annotations

import numpy as np

from .formats import D, row_bytes, scale_bytes

SCALE_DATA = {"int8": 1, "int4": 4, "fp4": 4, "nvfp4": 8}


def grp_r(fmt: str, wg: int) -> int:
    """Rows of a group on a machine of wg lanes (`opentpu/quant.py:650-653`)."""
    return wg if wg == 1 or fmt == "int8" else 2 * wg


def swp(fmt: str, R: int, rsc: bool = False) -> int:
    """The Sw part of a scale area of R rows (`opentpu/quant.py:656-664`)."""
    if rsc or fmt == "int8":
        return 4 * R
    if fmt == "nvfp4":
        return 16 if R == 1 else 8 * R
    return 8 if R == 1 else 4 * R


def grp_row_bytes(K: int, fmt: str, wg: int) -> int:
    """Group stride (`opentpu/quant.py:672-679`)."""
    if wg == 1 or fmt == "int8":
        return row_bytes(K, fmt) * wg
    return (K // D) * wg * D


def grp_scale_bytes(K: int, fmt: str, wg: int, rsc: bool = False) -> int:
    """Group scale stride: Sw part plus K/D blocks of R rows' data, padded to the Sw part
    (`opentpu/quant.py:682-690`)."""
    R = grp_r(fmt, wg)
    p = swp(fmt, R, rsc)
    n = p if rsc else p + (K // D) * R * SCALE_DATA[fmt]
    return -(-n // p) * p


def chunk_fold(m: int, R: int) -> int:
    """XOR fold of chunk index m into log2 R bits, bit i into bit i mod log2 R
    (`opentpu/quant.py:718-729`)."""
    b = R.bit_length() - 1
    h = 0
    if b == 0:
        return 0
    while m:
        h ^= m & (R - 1)
        m >>= b
    return h


def _row_map(N: int, K: int, fmt: str, wg: int):
    """For every (natural row n, element e < K): (grouped byte offset, nibble shift or -1)."""
    R = grp_r(fmt, wg)
    grb = grp_row_bytes(K, fmt, wg)
    P = wg * D
    n = np.arange(N)[:, None]
    e = np.arange(K)[None, :]
    g, j = n // R, n % R
    c, i = e // D, e % D
    if fmt == "int8":
        return g * grb + c * P + j * D + i, None
    if wg == 1:                                              # natural: element e in byte e / 2
        return g * grb + e // 2, 4 * (e % 2)
    return g * grb + c * P + (j // 2) * D + i, 4 * (j % 2)


def group_rows(rows, N: int, K: int, fmt: str, wg: int) -> np.ndarray:
    """Natural rows [N, >= row_bytes] -> grouped bytes [ceil(N / R), grp_row_bytes], the pad
    rows 0 (`opentpu/quant.py:693-715`)."""
    rows = np.asarray(rows, np.uint8)
    R = grp_r(fmt, wg)
    G = -(-N // R)
    out = np.zeros(G * grp_row_bytes(K, fmt, wg), np.uint8)
    off, sh = _row_map(N, K, fmt, wg)
    if sh is None:
        out[off] = rows[:, :K]
    else:
        e = np.arange(K)[None, :]
        code = (rows[np.arange(N)[:, None], e // 2] >> (4 * (e % 2))) & 15
        np.bitwise_or.at(out, off.ravel(), (code << sh).astype(np.uint8).ravel())
    return out.reshape(G, -1)


def ungroup_rows(data, N: int, K: int, fmt: str, wg: int) -> np.ndarray:
    """Grouped bytes -> natural rows [N, row_bytes] (the 4-bit rows' pad past K / 2 zero)
    (`opentpu/quant.py:749-763`)."""
    flat = np.asarray(data, np.uint8).reshape(-1)
    off, sh = _row_map(N, K, fmt, wg)
    out = np.zeros((N, row_bytes(K, fmt)), np.uint8)
    if sh is None:
        out[:, :K] = flat[off]
        return out
    code = (flat[off] >> sh) & 15                             # [N, K]
    out[:, :K // 2] = code[:, 0::2] | (code[:, 1::2] << 4)
    return out


def hash_rows(data, at: int, wg: int) -> np.ndarray:
    """Grouped bytes as stored at byte address `at` by a machine with the channel hash: in the
    chunk at A lane l's D bytes at lane l ^ chunk_fold(A / P). Its own inverse at one address
    (`opentpu/quant.py:732-746`)."""
    data = np.asarray(data, np.uint8)
    P = wg * D
    if at % P or data.size % P:
        raise ValueError(f"grouped bytes at {at:#x} ({data.size} bytes) are not whole {P}-byte chunks")
    flat = data.reshape(-1)
    out = np.empty_like(flat)
    for m in range(flat.size // P):
        h = chunk_fold(at // P + m, wg)
        for l in range(wg):
            dst = m * P + (l ^ h) * D
            out[dst:dst + D] = flat[m * P + l * D:m * P + (l + 1) * D]
    return out.reshape(data.shape)


def _scale_map(N: int, K: int, fmt: str, wg: int, rsc: bool):
    """(area byte offsets, natural scale-row byte offsets) of every byte that moves."""
    R = grp_r(fmt, wg)
    gss = grp_scale_bytes(K, fmt, wg, rsc)
    src, dst = [], []
    for n in range(N):
        g, j = divmod(n, R)
        for b in range(4):                                   # Sw
            dst.append(g * gss + 4 * j + b)
            src.append((n, b))
        if rsc:
            continue
        sb, h, p = SCALE_DATA[fmt], swp(fmt, 1), swp(fmt, R)
        for k in range(K // D):
            for b in range(sb):
                dst.append(g * gss + p + (k * R + j) * sb + b)
                src.append((n, h + k * sb + b))
    return np.array(dst, np.int64), np.array(src, np.int64).reshape(-1, 2)


def group_scales(srows, N: int, K: int, fmt: str, wg: int, rsc: bool = False) -> np.ndarray:
    """Natural scale rows -> grouped scale areas [ceil(N / R), grp_scale_bytes], pad rows 0
    (`opentpu/quant.py:775-793`)."""
    srows = np.asarray(srows, np.uint8)
    G = -(-N // grp_r(fmt, wg))
    out = np.zeros(G * grp_scale_bytes(K, fmt, wg, rsc), np.uint8)
    dst, src = _scale_map(N, K, fmt, wg, rsc)
    out[dst] = srows[src[:, 0], src[:, 1]]
    return out.reshape(G, -1)


def ungroup_scales(areas, N: int, K: int, fmt: str, wg: int, rsc: bool = False) -> np.ndarray:
    """Grouped scale areas -> natural scale rows [N, scale_bytes], reserved words and padding 0
    (`opentpu/quant.py:796-808`)."""
    flat = np.asarray(areas, np.uint8).reshape(-1)
    out = np.zeros((N, scale_bytes(K, fmt, rsc)), np.uint8)
    dst, src = _scale_map(N, K, fmt, wg, rsc)
    out[src[:, 0], src[:, 1]] = flat[dst]
    return out
