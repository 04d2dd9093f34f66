// Weight images in the reference machine's grouped layout (docs/isa.md "Weight groups",
// opentpu/quant.py:634-808) converted on the GPU to the natural rows the MM kernels stream:
// the inverse of quant.group_rows (with the channel hash of hash_rows when the image was stored
// hashed) and of quant.group_scales.  A machine of WG lanes stores a matrix in groups of R rows
// (R = WG for int8, 2 WG for the 4-bit formats), group g's chunk c (P = WG x D bytes) at
// g * (grp_row_bytes) + c P; lane l of a chunk is D bytes:
//   int8:  row g R + l's K-block c;
//   4-bit: K-block c of rows g R + 2l (low nibbles) and g R + 2l + 1 (high nibbles), element i
//          of the block in byte i;
// with the hash, the chunk at address A keeps lane l at lane l ^ fold(A / P) (the XOR fold of
// the chunk index into log2 WG bits).  Scale areas: group g's at g * grp_scale_bytes, row j's
// Sw word at 4 j, block k's data (SB bytes: int8 1, int4 / fp4 4, nvfp4 8) at SWP + (k R + j) SB.
// MM KT's pairs (docs/isa.md "K tail", opentpu/quant.py:829-880: kt_rows, kt_scales): groups 2p
// and 2p + 1 share (2 KB - 1) chunks, group 2p's chunks 0 .. KB-2, the tail chunk (each lane's
// first D/2 bytes group 2p's half of block KB-1, the next D/2 group 2p + 1's), group 2p + 1's
// chunks 0 .. KB-2; the odd groups' scale entries in chunk order (the tail block's first).  The
// natural rows come out padded: block KB-1's upper half zero.
#include "otpu_common.h"

namespace otpu {

// the XOR fold of chunk index m into log2(R) bits (bit i into bit i mod log2 R); 0 at R = 1
__device__ __forceinline__ uint32_t chunk_fold(uint64_t m, int R) {
    const int b = 31 - __builtin_clz((unsigned)R);             // log2 R (R a power of two)
    uint32_t h = 0;
    if (b == 0) return 0;
    while (m) {
        h ^= (uint32_t)(m & (uint64_t)(R - 1));
        m >>= b;
    }
    return h;
}

// one thread per 16 output bytes of a natural row (int8: 16 elements; 4-bit: 32 elements)
// four: a 4-bit format grouped two rows a lane (WG > 1); else the rows' bytes are whole lanes
// (int8, or any format at WG = 1: the natural layout, grb = the natural row bytes)
// (chunk index from the image's start, the byte a lane's data starts at in it) of group g's chunk c
__device__ __forceinline__ int64_t chunk_at(int g, int c, int KB, int kt, int64_t gch, int* h0) {
    *h0 = 0;
    if (!kt) return (int64_t)g * gch + c;                   // gch: chunks a group (KB)
    const int64_t p = g >> 1, e = g & 1;
    if (c < KB - 1) return p * (2 * KB - 1) + e * KB + c;
    *h0 = (int)e * (OTPU_D / 2);                            // the tail chunk's half of this group
    return p * (2 * KB - 1) + KB - 1;
}

__global__ __launch_bounds__(256) void ungroup_rows_kernel(const uint8_t* __restrict__ data, int N, int K, int wg,
                                                           int four, int kt, int64_t at_chunk, uint8_t* __restrict__ rows,
                                                           int64_t rs, int64_t rowb, int64_t gch) {
    const int64_t pieces = rowb / 16;                           // 16-byte pieces of an output row
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (int64_t)N * pieces) return;
    const int n = (int)(t / pieces);
    const int64_t o = (t % pieces) * 16;                        // output byte offset in the row
    const int KB = K / OTPU_D, R = four ? 2 * wg : wg;
    const int64_t P = (int64_t)wg * OTPU_D;
    const int g = n / R, j = n % R;
    uint4 outv = make_uint4(0, 0, 0, 0);
    if (!four) {
        const int c = (int)(o / OTPU_D), i0 = (int)(o % OTPU_D);
        int h0;
        const int64_t m = chunk_at(g, c, KB, kt, gch, &h0);
        if (!(kt && c == KB - 1 && i0 >= OTPU_D / 2)) {         // (KT: the tail block's upper half is 0)
            const uint32_t h = at_chunk >= 0 ? chunk_fold((uint64_t)(at_chunk + m), wg) : 0u;
            const uint8_t* src = data + m * P + (int64_t)(j ^ (int)h) * OTPU_D + h0 + i0;
            outv = *reinterpret_cast<const uint4*>(src);
        }
    } else if (o < K / 2) {                                     // (bytes past K/2: the row's zero pad)
        const int64_t e0 = 2 * o;                               // first element of the piece
        const int c = (int)(e0 / OTPU_D), i0 = (int)(e0 % OTPU_D);
        const int l = j >> 1, hb = j & 1;
        int h0;
        const int64_t m = chunk_at(g, c, KB, kt, gch, &h0);
        if (kt && c == KB - 1 && i0 >= OTPU_D / 2) {
            *reinterpret_cast<uint4*>(rows + (int64_t)n * rs + o) = outv;
            return;
        }
        const uint32_t h = at_chunk >= 0 ? chunk_fold((uint64_t)(at_chunk + m), wg) : 0u;
        const uint8_t* src = data + m * P + (int64_t)(l ^ (int)h) * OTPU_D + h0 + i0;
        const uint4 a = *reinterpret_cast<const uint4*>(src);
        const uint4 b = *reinterpret_cast<const uint4*>(src + 16);
        const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        uint32_t r[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {                           // bytes 8q .. 8q+7 -> 4 output bytes
            uint32_t v = 0;
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const uint32_t byte = (w[(8 * q + s) >> 2] >> (8 * ((8 * q + s) & 3))) & 0xFF;
                const uint32_t nib = hb ? (byte >> 4) : (byte & 15);
                v |= nib << (4 * s);                            // element 2k low, 2k + 1 high
            }
            r[q] = v;
        }
        outv = make_uint4(r[0], r[1], r[2], r[3]);
    }
    *reinterpret_cast<uint4*>(rows + (int64_t)n * rs + o) = outv;
}

// one thread per natural scale row
// (KT: an odd group's entries in chunk order, the tail block's first; a 4-bit tail word is taken
// as stored, its sub-block 2 and 3 multipliers meeting the zero half)
__global__ __launch_bounds__(256) void ungroup_scales_kernel(const uint8_t* __restrict__ areas, int N, int KB, int R,
                                                             int64_t gss, int swp_r, int hdr, int sb, int kt,
                                                             uint8_t* __restrict__ srows, int64_t srs, int64_t need) {
    const int n = blockIdx.x * blockDim.x + threadIdx.x;
    if (n >= N) return;
    const int g = n / R, j = n % R;
    const bool rot = kt && (g & 1);
    const uint8_t* a = areas + g * gss;
    uint8_t* o = srows + (int64_t)n * srs;
    for (int64_t b = 0; b < need; ++b) o[b] = 0;                // reserved words and padding
    for (int b = 0; b < 4; ++b) o[b] = a[4 * j + b];           // Sw
    for (int k = 0; k < KB && sb; ++k) {
        const int e = rot ? (k == KB - 1 ? 0 : k + 1) : k;      // the area entry of block k
        for (int b = 0; b < sb; ++b) o[hdr + k * sb + b] = a[swp_r + ((int64_t)e * R + j) * sb + b];
    }
}

}  // namespace otpu

using namespace otpu;

static int grp_r(int fmt, int wg) { return (wg == 1 || fmt == OTPU_INT8) ? wg : 2 * wg; }
static int scale_data(int fmt) { return fmt == OTPU_INT8 ? 1 : (fmt == OTPU_NVFP4 ? 8 : 4); }
static int swp(int fmt, int R, int rsc) {
    if (rsc || fmt == OTPU_INT8) return 4 * R;
    if (fmt == OTPU_NVFP4) return R == 1 ? 16 : 8 * R;
    return R == 1 ? 8 : 4 * R;
}

extern "C" int otpu_ungroup_rows(const uint8_t* data, int N, int K, int wg, int fmt, int kt, int64_t at,
                                 uint8_t* rows, int64_t rs, otpu_stream_t stream) {
    if (fmt < OTPU_INT8 || fmt > OTPU_NVFP4) return otpu_fail(OTPU_EFORMAT, "ungroup_rows: format %d", fmt);
    if (N < 1 || K < OTPU_D || K % OTPU_D || wg < 1 || wg > 64 || (wg & (wg - 1)))
        return otpu_fail(OTPU_EINVAL, "ungroup_rows: N %d, K %d, wg %d (a power of two, at most 64)", N, K, wg);
    if (kt && (wg == 1 || fmt == OTPU_NVFP4))
        return otpu_fail(OTPU_EINVAL, "ungroup_rows: KT's pairs are of groups (wg > 1) of int8, int4 or fp4");
    const int four = fmt != OTPU_INT8 && wg > 1;
    const int64_t rowb = fmt != OTPU_INT8 ? (int64_t)((K + 2 * OTPU_D - 1) / (2 * OTPU_D)) * OTPU_D : K;
    const int64_t P = (int64_t)wg * OTPU_D;
    const int64_t grb = four ? (int64_t)(K / OTPU_D) * P : rowb * wg;   // quant.grp_row_bytes
    if (!data || !rows || rs < rowb || rs % 16 || ((uintptr_t)data & 15) || ((uintptr_t)rows & 15))
        return otpu_fail(OTPU_EINVAL, "ungroup_rows: rows of %lld bytes need %lld, 16-byte aligned", (long long)rs,
                         (long long)rowb);
    if (at >= 0 && at % P) return otpu_fail(OTPU_EINVAL, "ungroup_rows: address %lld not a multiple of %lld",
                                            (long long)at, (long long)P);
    const int64_t total = (int64_t)N * (rowb / 16);
    const int64_t blocks = (total + 255) / 256;
    if (blocks > 0x7FFFFFFF) return otpu_fail(OTPU_EINVAL, "ungroup_rows: too large");
    ungroup_rows_kernel<<<(unsigned)blocks, 256, 0, (hipStream_t)stream>>>(data, N, K, wg, four, kt,
                                                                           at >= 0 ? at / P : -1, rows, rs, rowb, grb / P);
    return otpu_launch_check("ungroup_rows");
}

extern "C" int otpu_ungroup_scales(const uint8_t* areas, int N, int K, int wg, int fmt, int rsc, int kt,
                                   uint8_t* srows, int64_t srs, otpu_stream_t stream) {
    if (fmt < OTPU_INT8 || fmt > OTPU_NVFP4) return otpu_fail(OTPU_EFORMAT, "ungroup_scales: format %d", fmt);
    if (rsc && fmt == OTPU_NVFP4) return otpu_fail(OTPU_EFORMAT, "ungroup_scales: RSC does not take NVFP4");
    if (kt && (wg == 1 || fmt == OTPU_NVFP4))
        return otpu_fail(OTPU_EINVAL, "ungroup_scales: KT's pairs are of groups (wg > 1) of int8, int4 or fp4");
    if (N < 1 || K < OTPU_D || K % OTPU_D || wg < 1 || wg > 64 || (wg & (wg - 1)))
        return otpu_fail(OTPU_EINVAL, "ungroup_scales: N %d, K %d, wg %d", N, K, wg);
    const int KB = K / OTPU_D, R = grp_r(fmt, wg), sb = rsc ? 0 : scale_data(fmt);
    const int p = swp(fmt, R, rsc);
    int64_t n = rsc ? p : p + (int64_t)KB * R * sb;
    const int64_t gss = (n + p - 1) / p * p;
    const int hdr = swp(fmt, 1, rsc);
    int64_t need = rsc ? 4 : (fmt == OTPU_INT8 ? 4 + 4 * ((KB + 3) / 4)
                                               : fmt == OTPU_NVFP4 ? 16 + 16 * ((KB + 1) / 2) : 8 + 8 * ((KB + 1) / 2));
    if (!areas || !srows || srs < need)
        return otpu_fail(OTPU_EINVAL, "ungroup_scales: scale rows of %lld bytes need %lld", (long long)srs,
                         (long long)need);
    ungroup_scales_kernel<<<(N + 255) / 256, 256, 0, (hipStream_t)stream>>>(areas, N, KB, R, gss, p, hdr, sb,
                                                                           kt && !rsc, srows, srs, need);
    return otpu_launch_check("ungroup_scales");
}
