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

MM KT's pairs (`docs/isa.md` "K tail", `opentpu/quant.py:829-880`: kt_rows, kt_scales): a
grouped matrix whose K ends in the first half of its last block (the upper half of every lane's
last chunk zero) is stored as pairs of groups, (2 KB - 1) P bytes a pair: group 2p's chunks
0 .. KB-2, the tail chunk (each lane's D bytes: group 2p's half block, then group 2p + 1's),
group 2p + 1's chunks 0 .. KB-2 (an odd group count's last pair: group 2p alone, its tail's
other half zero).  The odd groups' scale entries are stored in the order the MXU takes their
chunks: the tail block's entry first, then blocks 0 .. KB-2; a 4-bit tail entry's sub-block 0
and 1 multipliers are also copied over those of sub-blocks 2 and 3 (which meet zeros).

The functions below build every map one byte address at a time from those formulas (the
reference reshapes whole arrays), so a transposed axis or a wrong stride shows up as a byte in
the wrong place. Pinning (tests/test_oracle_groups.py): KT: the pair stride and one chunk saved
a pair (the reference's `tests/test_kt.py:115-124` and `:177-200` restated with own inputs),
every chunk of a pair against the layout's formula, refusal of a non-zero upper half, and
ungroup(kt pairs) = the natural rows, byte for byte; the chunk fold's known answer
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


def kt_rows(data, wg: int) -> np.ndarray:
    """Grouped bytes [G, KB P] whose last chunk's upper lane halves are zero -> MM KT's pairs
    [ceil(G / 2), (2 KB - 1) P] (`opentpu/quant.py:842-858`), chunk by chunk."""
    data = np.asarray(data, np.uint8)
    P = wg * D
    G = data.shape[0]
    KB = data.shape[1] // P
    ch = data.reshape(G, KB, wg, D)
    if np.any(ch[:, KB - 1, :, D // 2:]):
        raise ValueError("kt_rows: the last K-block's upper halves are not zero")
    pairs = -(-G // 2)
    out = np.zeros((pairs, (2 * KB - 1) * P), np.uint8)
    for p in range(pairs):
        for e in (0, 1):
            g = 2 * p + e
            if g >= G:
                continue
            for c in range(KB - 1):                              # whole chunks
                at = (c if e == 0 else KB + c) * P
                out[p, at:at + P] = data[g, c * P:(c + 1) * P]
            for l in range(wg):                                  # the tail chunk's lane halves
                at = (KB - 1) * P + l * D + e * (D // 2)
                out[p, at:at + D // 2] = ch[g, KB - 1, l, :D // 2]
    return out


def kt_group_chunk(g: int, c: int, KB: int) -> tuple:
    """Where group g's chunk c lies in MM KT's pairs: (chunk index from the image's start, the
    byte in each lane where its D / 2 bytes start for the tail chunk c = KB - 1, else 0)."""
    p, e = divmod(g, 2)
    if c < KB - 1:
        return p * (2 * KB - 1) + e * KB + c, 0
    return p * (2 * KB - 1) + KB - 1, e * (D // 2)


def ungroup_kt_rows(data, N: int, K: int, fmt: str, wg: int, at: int | None = None) -> np.ndarray:
    """MM KT's pairs (hashed as stored at `at` when given) -> natural rows [N, row_bytes(K)],
    K = KB D the padded K (the inverse of kt_rows, then of group_rows), byte address by byte
    address."""
    flat = np.asarray(data, np.uint8).reshape(-1)
    R = grp_r(fmt, wg)
    KB = K // D
    P = wg * D
    out = np.zeros((N, row_bytes(K, fmt)), np.uint8)
    for n in range(N):
        g, j = divmod(n, R)
        lane = j if fmt == "int8" else j // 2
        for c in range(KB):
            m, h0 = kt_group_chunk(g, c, KB)
            h = chunk_fold((at // P) + m, wg) if at is not None else 0
            base = m * P + (lane ^ h) * D + h0
            nb = D // 2 if c == KB - 1 else D                 # the tail's upper half: zeros
            src = flat[base:base + nb]
            if fmt == "int8":
                out[n, c * D:c * D + nb] = src
            else:
                nib = (src >> (4 * (j % 2))) & 15               # element c D + i in lane byte i
                e = c * D + np.arange(nb)
                np.bitwise_or.at(out[n], e // 2, (nib << (4 * (e % 2))).astype(np.uint8))
    return out


def kt_scales(areas, fmt: str, K: int, wg: int, rsc: bool = False) -> np.ndarray:
    """Grouped scale areas -> MM KT's (`opentpu/quant.py:861-880`): the odd groups' block entries
    in chunk order (the tail block's first); a 4-bit tail word's bits 8..19 (sub-blocks 0, 1)
    also into bits 20..31."""
    areas = np.array(areas, np.uint8)
    if rsc or areas.shape[0] < 2:
        return areas
    if fmt == "nvfp4":
        raise ValueError("kt_scales: nvfp4 has no K tail")
    R = grp_r(fmt, wg)
    KB = K // D
    sb, p = SCALE_DATA[fmt], swp(fmt, R)
    for g in range(1, areas.shape[0], 2):
        old = areas[g].copy()
        for j in range(R):
            for k in range(KB):
                src = p + ((KB - 1 if k == 0 else k - 1) * R + j) * sb
                dst = p + (k * R + j) * sb
                areas[g, dst:dst + sb] = old[src:src + sb]
            if fmt in ("int4", "fp4"):
                at = p + j * sb                                  # the tail entry, now first
                w = int(areas[g, at:at + 4].view("<u4")[0])
                w = (w & 0xFFFFF) | (((w >> 8) & 0xFFF) << 20)
                areas[g, at:at + 4] = np.array([w], "<u4").view(np.uint8)
    return areas


def ungroup_kt_scales(areas, N: int, K: int, fmt: str, wg: int, rsc: bool = False) -> np.ndarray:
    """MM KT's scale areas -> natural scale rows: the odd groups' entries back in block order
    (the 4-bit tail word kept as stored: its sub-block 2 and 3 multipliers meet zeros)."""
    a = np.array(areas, np.uint8)
    if not rsc and a.shape[0] >= 2:
        R = grp_r(fmt, wg)
        KB = K // D
        sb, p = SCALE_DATA[fmt], swp(fmt, R)
        for g in range(1, a.shape[0], 2):
            old = a[g].copy()
            for j in range(R):
                for k in range(KB):
                    src = p + ((0 if k == KB - 1 else k + 1) * R + j) * sb
                    dst = p + (k * R + j) * sb
                    a[g, dst:dst + sb] = old[src:src + sb]
    return ungroup_scales(a, N, K, fmt, wg, rsc)


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
