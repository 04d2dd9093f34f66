// MM for many activation rows with 4-bit weights (int4x, fp4x6, nvfp4, and their RSC / UNIT
// forms) on the int8 MFMA units: the prefill GEMM of the 4-bit formats.  Semantics:
// opentpu/isasim.py:749-910 (docs/isa.md:226-305): acc = sum over groups of [sh >= 0] m 2^sh c,
// sh = W - dw - da, c the group's integer dot product; y = (i2f(acc) * Sw) * (Sa * 2^-W).  int4x
// and fp4x6: W = 11, 32-groups with a multiplier m each and a block offset dw per 128 columns;
// nvfp4: W = 13, 16-groups with an E4M3 scale each, m its significand (8 + mantissa, or the
// mantissa at E = 0) and dw = 15 - max(E, 1).
//
// Exactness.  Every product term is folded into an integer weight before the MFMA.  For weight
// row n let R_n be the largest group offset dw <= W (a group with dw > W drops for every
// activation offset).  For the activation plane d (the 32-groups whose offset is d):
//     acc_d = 2^(W - R_n - d) * sum_i q_i w''_i,   w''_i = [dw + d <= W] m 2^(R_n - dw) w_i,
// an ordinary integer matrix product of int8 activations and the integer w'' (|w''| < 2^15 when
// the tile's offsets and multipliers allow: checked per tile).  w'' is split into two int8 planes
// in balanced base 256 (w'' = 256 h + l, l and h in [-128, 127]), each an int8 MFMA operand, so
// the K walk is a plain two-plane int8 GEMM with no rescaling inside it.  Activation planes (MX
// offsets) walk K once each, combined by Horner's rule in the int32 accumulators (acc <<= the gap
// to the next plane's d, as the int8 GEMM does; the bound is checked per tile).  The epilogue
// forms T = 256 C_h + C_l in int64 and shifts it by W - R_n - d_last (exact: the accumulator is
// an integer), then the reference's fp32 epilogue.  A tile the bounds refuse takes an exact VALU
// path.
//
// Work layout.  A workgroup of 8 waves owns a 128 x 128 output tile.  Waves 0-3 multiply (64 x 64
// each, 4 x 4 v_mfma_i32_16x16x64_i8 per 64-deep step and plane); waves 4-7 stream: they issue
// every direct-to-LDS load (the activation stage, a 3-deep ring; the 4-bit rows of a stage with
// their scale words and the activation offset words, a 4-deep ring one stage further ahead).
// Every wave turns the nibbles of the next stage into the two int8 planes, one 32-group a thread
// (a 16-entry table per group of one multiplier and plane, built with packed 16-bit products and
// read with v_perm_b32), the multiplying waves behind the current stage's MFMAs.  One workgroup
// barrier a stage.
#include <type_traits>

#include "otpu_common.h"

namespace otpu {
namespace g4 {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef short s16x2 __attribute__((ext_vector_type(2)));

constexpr int TM = 128, TN = 128, BK = 128;      // tile rows and columns, K a stage (one block)
constexpr int NA = 3;                           // activation stages in their ring
constexpr int NR = 4;                           // raw weight stages in theirs
constexpr int ATILE = TM * BK;                  // 16 KB of activations a stage
constexpr int RAWB = TN * BK / 2;               // 8 KB of nibbles a stage
constexpr int PLANE = TN * BK;                  // one int8 plane of a stage's weights: 16 KB
constexpr int OFF_RAW = NA * ATILE;
constexpr int TPS = 68;                         // the epilogue's transpose row stride (words)

// the formats' constants: MM's window; a raw stage slot's layout (nibbles, then the rows' scale
// data of the stage: 4 bytes a row, or nvfp4's 8 E4M3 bytes; then the activation rows' offset
// words; nvfp4 also a pad, below); the direct loads a streaming wave issues a raw stage
template <int FMT>
struct Fmt {
    static constexpr bool NV = FMT == OTPU_NVFP4;
    static constexpr int W = NV ? 13 : 11;
    static constexpr int SC = NV ? 1024 : 512;  // scale data of a stage's 128 rows
    static constexpr int DOFF = RAWB + SC;      // the activation offset words (128 rows)
    static constexpr int RSLOT = DOFF + 512 + (NV ? 512 : 0);
    static constexpr int OFF_PL = OFF_RAW + NR * RSLOT;
    static constexpr int LDS_BYTES = OFF_PL + 2 * 2 * PLANE;
    static constexpr int DMA_R = NV ? 4 : 3;
    static constexpr int MAGMAX = FMT == OTPU_INT4 ? 8 : 12;
    static_assert(4 * 2 * 64 * TPS * 4 <= LDS_BYTES, "the epilogue's two planes a wave fit the walk's memory");
    static_assert(LDS_BYTES <= 160 * 1024, "one workgroup a CU");
};

// nvfp4: the multiplier and the offset of an E4M3 group scale (its sign bit unused)
__device__ __forceinline__ int nv_m(uint32_t e4) {
    const int E = (int)((e4 >> 3) & 15), mt = (int)(e4 & 7);
    return E ? 8 + mt : mt;
}
__device__ __forceinline__ int nv_dw(uint32_t e4) {
    const int E = (int)((e4 >> 3) & 15);
    return 15 - (E > 1 ? E : 1);
}

struct Args {
    const int8_t* q; int64_t ldq;
    const float* Sa;
    const uint8_t* da; int64_t ldda;
    int M, K;
    const uint8_t* w; int64_t rs;
    const uint8_t* ws; int64_t srs;
    int N, flags, k0;
    const float* alpha;
    float* out; int64_t ors;
    int tiles_m, tiles_n;
    int vec4;
};

// the 16-byte slot of chunk c of row r (128-byte rows): the XOR swizzle that puts the 16 rows a
// ds_read_b128 fragment reads on distinct banks (the int8 GEMM's)
__device__ __forceinline__ int rswz(int r) { return ((r >> 1) & 7) ^ ((r & 1) << 2); }
__device__ __forceinline__ int rof(int r, int c) { return r * BK + ((c ^ rswz(r)) << 4); }

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
// direct-to-LDS loads: 16 bytes (lane L at M0 + 16 L) and 4 bytes (lane L at M0 + 4 L) a lane
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(g), "s"(lds) : "memory");
}
__device__ __forceinline__ void dma4(const void* g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" : : "v"(g), "s"(lds) : "memory");
}
template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}
// LDS reads and writes of this wave done, then the workgroup barrier
__device__ __forceinline__ void bar() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" : : : "memory"); }

// direct loads a streaming wave issues per activation stage (16 KB over 4 waves); per raw stage
// (8 KB of nibbles over 4 waves, then one dword a lane: scale words or offset words; nvfp4 two,
// below) Fmt::DMA_R
constexpr int DMA_A = 4;

// ---- the value tables of one 32-group: codes 0..15 times its integer multiplier ----
// pair k of a format: the values of codes 2k and 2k + 1 (int4 two's complement; fp4x6 twice the
// E2M1 value, sign in bit 3), as two 16-bit lanes
template <int FMT>
__device__ __forceinline__ uint32_t code_pair(int k) {
    constexpr int mag[8] = {0, 1, 2, 3, 4, 6, 8, 12};
    int v0, v1;
    if (FMT == OTPU_INT4) {
        v0 = 2 * k < 8 ? 2 * k : 2 * k - 16;
        v1 = 2 * k + 1 < 8 ? 2 * k + 1 : 2 * k + 1 - 16;
    } else {
        v0 = (2 * k) & 8 ? -mag[(2 * k) & 7] : mag[(2 * k) & 7];
        v1 = (2 * k + 1) & 8 ? -mag[(2 * k + 1) & 7] : mag[(2 * k + 1) & 7];
    }
    return ((uint32_t)v0 & 0xFFFFu) | ((uint32_t)v1 << 16);
}

__device__ __forceinline__ uint32_t as_u32(s16x2 v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ s16x2 as_s16x2(uint32_t v) { return __builtin_bit_cast(s16x2, v); }

// the l and h tables of multiplier mp (|code value * mp| <= 32256): tl[k] holds the low bytes of
// codes 4k .. 4k + 3, th[k] their high bytes (v = 256 h + l, both signed bytes)
template <int FMT>
__device__ __forceinline__ void group_tables(int mp, uint32_t (&tl)[4], uint32_t (&th)[4]) {
    const s16x2 mm = as_s16x2((uint32_t)mp * 0x00010001u);
    uint32_t p[8], h[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const s16x2 v = mm * as_s16x2(code_pair<FMT>(k));            // v_pk_mul_lo_u16
        p[k] = as_u32(v);
        h[k] = as_u32(v + as_s16x2(0x00800080u));                    // v_pk_add_u16: (v + 128)
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        tl[k] = __builtin_amdgcn_perm(p[2 * k + 1], p[2 * k], 0x06040200u);   // low bytes: l
        th[k] = __builtin_amdgcn_perm(h[2 * k + 1], h[2 * k], 0x07050301u);   // high bytes of v + 128: h
    }
}

// the table entries of the four codes in the bytes of s (each 0..15)
__device__ __forceinline__ uint32_t lookup(const uint32_t (&t)[4], uint32_t sel7, uint32_t pick) {
    const uint32_t a = __builtin_amdgcn_perm(t[1], t[0], sel7);       // codes 0..7
    const uint32_t b = __builtin_amdgcn_perm(t[3], t[2], sel7);       // codes 8..15
    return __builtin_amdgcn_perm(b, a, pick);                         // byte i: a's or b's (bit 3)
}

// one raw dword (elements 0..7 of 8, element 2i in the low nibble of byte i) -> its l and h
// bytes in element order (two dwords each)
template <bool HI>
__device__ __forceinline__ void expand8(uint32_t x, const uint32_t (&tl)[4], const uint32_t (&th)[4], uint32_t& l0,
                                        uint32_t& l1, uint32_t& h0, uint32_t& h1) {
    const uint32_t ev = x & 0x0F0F0F0Fu, od = (x >> 4) & 0x0F0F0F0Fu;   // elements 0 2 4 6, 1 3 5 7
    const uint32_t se = ev & 0x07070707u, so = od & 0x07070707u;
    const uint32_t pe = ((ev >> 1) & 0x04040404u) | 0x03020100u, po = ((od >> 1) & 0x04040404u) | 0x03020100u;
    const uint32_t le = lookup(tl, se, pe), lo = lookup(tl, so, po);
    l0 = __builtin_amdgcn_perm(lo, le, 0x05010400u);                  // elements 0 1 2 3
    l1 = __builtin_amdgcn_perm(lo, le, 0x07030602u);                  // elements 4 5 6 7
    if (HI) {
        const uint32_t he = lookup(th, se, pe), ho = lookup(th, so, po);
        h0 = __builtin_amdgcn_perm(ho, he, 0x05010400u);
        h1 = __builtin_amdgcn_perm(ho, he, 0x07030602u);
    }
}

// the exact MM integer of output (j, n), group by group (the tiles the planes' bounds refuse)
template <int FMT>
__device__ int64_t valu_acc4(const Args& a, int j, int n, bool plainw) {
    constexpr int mag[8] = {0, 1, 2, 3, 4, 6, 8, 12};
    constexpr int G = Fmt<FMT>::NV ? 2 : 1, GS = 32 / G;     // weight groups a 32-group, their size
    const int8_t* qr = a.q + (int64_t)j * a.ldq;
    const uint8_t* wr = a.w + (int64_t)n * a.rs;
    const uint8_t* srow = a.ws + (int64_t)n * a.srs;
    int64_t acc = 0;
    for (int g = 0; g < a.K / 32; ++g) {
        const int da = (int)a.da[(int64_t)j * a.ldda + g];
        for (int h = 0; h < G; ++h) {
            int c = 0;
            for (int i = GS * h; i < GS * (h + 1); ++i) {
                const int code = (wr[16 * g + i / 2] >> (4 * (i & 1))) & 15;
                const int v = FMT == OTPU_INT4 ? (code < 8 ? code : code - 16) : (code & 8 ? -mag[code & 7] : mag[code & 7]);
                c += (int)qr[32 * g + i] * v;
            }
            int dw = 0, m = 1;
            if (!plainw && Fmt<FMT>::NV) {
                const uint32_t e4 = srow[16 + 8 * (a.k0 + g / 4) + 2 * (g & 3) + h];
                dw = nv_dw(e4);
                m = nv_m(e4);
            } else if (!plainw) {
                const uint32_t word = *reinterpret_cast<const uint32_t*>(srow + 8 + 4 * (a.k0 + g / 4));
                dw = (int)(word & 0xFF);
                m = (int)((word >> (8 + 6 * (g & 3))) & 63);
            }
            const int sh = Fmt<FMT>::W - dw - da;
            if (sh >= 0) acc += ((int64_t)m * c) << sh;
        }
    }
    return acc;
}

// y = (i2f(acc) * Sw) * (Sa * 2^-11), then ACC / ASCALE (the reference's epilogue order)
__device__ __forceinline__ void store_out(const Args& a, int m, int n, int64_t acc, float sw, float sa2) {
    float y = fmul_f(fmul_f(i2f(acc), sw), sa2);
    float* o = a.out + (int64_t)m * a.ors + n;
    if (a.flags & OTPU_ASCALE) y = fadd(fmul(*o, a.alpha[m]), y);
    else if (a.flags & OTPU_ACC) y = fadd(*o, y);
    *o = y;
}

// HI: weights with scale rows (two int8 planes); false: RSC / UNIT weights (w'' = w, one plane)
template <int FMT, bool HI>
__global__ __launch_bounds__(512) void gemm4_kernel(Args a) {
    using FT = Fmt<FMT>;
    constexpr int WN = FT::W, RSLOT = FT::RSLOT, DMA_R = FT::DMA_R;
    __shared__ __align__(16) int8_t lds[FT::LDS_BYTES];
    __shared__ int sR[TN];                      // each weight row's R (the largest live dw)
    __shared__ float sSa2[TM];                  // the tile rows' Sa * 2^-W
    __shared__ uint32_t sFlag[16];              // per wave: d values present, offsets past the window, PL

    const int tid = threadIdx.x, lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool streamer = wid >= 4;
    // XCD-major tile order (workgroup b runs on XCD b % 8): the tiles of one XCD share weight panels
    int tm, tn;
    {
        const int b = blockIdx.x, ntiles = a.tiles_m * a.tiles_n;
        if (ntiles % 8 == 0 && a.tiles_n % 8 == 0) {
            const int t = (b % 8) * (ntiles / 8) + b / 8;
            tn = t / a.tiles_m;
            tm = t % a.tiles_m;
        } else {
            tn = b / a.tiles_m;
            tm = b % a.tiles_m;
        }
    }
    const int m0 = tm * TM, n0 = tn * TN;
    const bool unit = (a.flags & OTPU_UNIT) != 0;
    const bool plainw = unit || (a.flags & OTPU_RSC) != 0;
    const int KS = a.K / BK;
    constexpr int MAGMAX = FT::MAGMAX;

    // ---- the streams' sources, and the first walk's first loads (before the scan, whose
    // latency they then overlap) ----
    int8_t* const ringA = lds;
    int8_t* const ringR = lds + OFF_RAW;
    int8_t* const planes = lds + FT::OFF_PL;    // [buffer][plane][128 x 128]

    // ---- the streaming waves' sources (per lane) ----
    const int hw = wid & 3;
    const int8_t* srcA[DMA_A];
    const uint8_t* srcB[2];
    const uint8_t* srcW;                        // the dword a lane loads a raw stage (stride per stage below)
    const uint8_t* srcD = nullptr;              // nvfp4: the second (activation offset words)
    int64_t stepW = 0;
    if (streamer) {
#pragma unroll
        for (int u = 0; u < DMA_A; ++u) {
            const int blk = hw * DMA_A + u, r = blk * 8 + (lane >> 3), c = (lane & 7) ^ rswz(r);
            srcA[u] = a.q + (int64_t)min(m0 + r, a.M - 1) * a.ldq + 16 * c;
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int blk = hw * 2 + u, r = blk * 16 + (lane >> 2), c = lane & 3;
            srcB[u] = a.w + (int64_t)min(n0 + r, a.N - 1) * a.rs + 16 * c;
        }
        const int r = (hw & 1) * 64 + lane;
        if (FT::NV) {
            // every wave a quarter of the stage's 8-byte scale rows (dword s = 64 hw + lane: row
            // s / 2, half s % 2), then the offset words of rows r (waves 2-3 into their area,
            // waves 0-1 the same words into the pad: every streaming wave issues the same loads)
            const int sd = hw * 64 + lane;
            srcW = plainw ? reinterpret_cast<const uint8_t*>(a.q)
                          : a.ws + (int64_t)min(n0 + (sd >> 1), a.N - 1) * a.srs + 16 + 8 * a.k0 + 4 * (sd & 1);
            stepW = plainw ? 0 : 8;
            srcD = a.da + (int64_t)min(m0 + r, a.M - 1) * a.ldda;
        } else if (hw < 2) {                    // the weight rows' scale words (a dummy for UNIT / RSC)
            srcW = plainw ? reinterpret_cast<const uint8_t*>(a.q)
                          : a.ws + (int64_t)min(n0 + r, a.N - 1) * a.srs + 8 + 4 * a.k0;
            stepW = plainw ? 0 : 4;
        } else {                                // the activation rows' offset words
            srcW = a.da + (int64_t)min(m0 + r, a.M - 1) * a.ldda;
            stepW = 4;
        }
    }
    auto issue_a = [&](int s) {
        const uint32_t base = lds_addr(ringA + (s % NA) * ATILE) + hw * DMA_A * 1024;
#pragma unroll
        for (int u = 0; u < DMA_A; ++u) dma16(srcA[u] + s * BK, base + 1024u * u);
    };
    auto issue_r = [&](int s) {
        const uint32_t base = lds_addr(ringR + (s % NR) * RSLOT);
#pragma unroll
        for (int u = 0; u < 2; ++u) dma16(srcB[u] + s * (BK / 2), base + (uint32_t)(hw * 2 + u) * 1024u);
        dma4(srcW + s * stepW, base + (uint32_t)RAWB + (uint32_t)hw * 256u);
        if (FT::NV)
            dma4(srcD + s * 4, base + (uint32_t)(FT::DOFF + (hw < 2 ? 512 : 0) + (hw & 1) * 256));
    };
    // vmcnt(n) for the counts a walk can leave outstanding (sums of DMA_A and DMA_R, up to 16)
    auto wait_n = [&](int n) {
        switch (n) {
            case 16: wait_vm<16>(); break;
            case 14: wait_vm<14>(); break;
            case 12: wait_vm<12>(); break;
            case 11: wait_vm<11>(); break;
            case 10: wait_vm<10>(); break;
            case 8: wait_vm<8>(); break;
            case 7: wait_vm<7>(); break;
            case 4: wait_vm<4>(); break;
            case 3: wait_vm<3>(); break;
            default: wait_vm<0>(); break;
        }
    };
    // a walk's first loads: raw 0, then (A 0, raw 1), (A 1, raw 2), the waits below count them in
    // that order.  The first walk issues raw 0 and A 0 before the tile's scan and the rest after
    // it: at the start every CU's loads miss in L2 at once, and the fewer there are, the sooner
    // the scan's and stage 0's come back.
    auto prologue_first = [&] {
        issue_r(0);
        issue_a(0);
    };
    auto prologue_rest = [&] {
        if (KS > 1) issue_r(1);
        if (KS > 1) issue_a(1);
        if (KS > 2) issue_r(2);
    };
    auto prologue_issue = [&] {
        prologue_first();
        prologue_rest();
    };
    // the epilogue's column scales (region wid & 3's columns), loaded before any stream (a stream
    // wave's waits count only the loads issued after them)
    const int q = lane & 15;
    const int wm = (wid & 3) >> 1, wn = wid & 1;
    const int nc = n0 + wn * 64 + 4 * q;           // this lane's four epilogue columns
    float sw[4];
#pragma unroll
    for (int c = 0; c < 4; ++c)
        sw[c] = unit ? 1.0f : *reinterpret_cast<const float*>(a.ws + (int64_t)min(nc + c, a.N - 1) * a.srs);
    if (streamer) prologue_first();

    // ---- the tile's scan (waves 0-3): activation offsets, weight offsets and multipliers ----
    // (all of it on the waves that issue no direct loads: their loads' waits then count their own
    // loads only.  On the streaming waves the weight scan's waits, which the compiler sets
    // without counting the direct loads issued before them, waited for every stage in flight.)
    if (!streamer) {
        if (tid < TM) sSa2[tid] = m0 + tid < a.M ? fmul(a.Sa[m0 + tid], pow2f(-WN)) : 0.0f;
        // two adjacent threads a row of each operand (activation row m0 + r, weight row n0 + r),
        // a word a load (four activation offsets; a weight block's dw and multipliers), both
        // rows' loads of 8 words in flight at once (with the two scans one after the other, each
        // waited for its loads: two round trips, ~2 us each while the start's loads all miss)
        const int r = tid >> 1, h = tid & 1;
        const uint32_t* drow = reinterpret_cast<const uint32_t*>(a.da + (int64_t)min(m0 + r, a.M - 1) * a.ldda);
        const uint32_t dmask = m0 + r < a.M ? ~0u : 0u;        // (rows past M offer no offsets)
        const uint8_t* srow = a.ws + (int64_t)min(n0 + r, a.N - 1) * a.srs + (FT::NV ? 16 + 8 * a.k0 : 8 + 4 * a.k0);
        uint32_t dm = 0;
        int R = 0, T = 0;                       // (rows past N: the last row's, which they stream)
#pragma unroll 8
        for (int k = h; k < KS; k += 2) {
            const uint32_t wd = drow[k];
            uint32_t bits = 0;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint32_t d = (wd >> (8 * t)) & 0xFFu;
                bits |= 1u << (d <= WN ? d : 31);
            }
            dm |= bits & dmask;
            if (FT::NV) {                       // 8 E4M3 group scales a block: each its own dw
                const uint32_t* sp = reinterpret_cast<const uint32_t*>(srow + 8 * k);   // (4-byte aligned)
                const uint2 sc = plainw ? make_uint2(0u, 0u) : make_uint2(sp[0], sp[1]);
#pragma unroll
                for (int g = 0; g < 8; ++g) {
                    const uint32_t e4 = ((g < 4 ? sc.x : sc.y) >> (8 * (g & 3))) & 0xFFu;
                    const int dw = nv_dw(e4);
                    const bool live = !plainw && dw <= WN;
                    R = max(R, live ? dw : 0);
                    T = max(T, live ? nv_m(e4) << (WN - dw) : 0);
                }
            } else {
                const uint32_t word = plainw ? 0u : *reinterpret_cast<const uint32_t*>(srow + 4 * k);
                const int dw = (int)(word & 0xFF);
                int mx = 0;
#pragma unroll
                for (int b = 0; b < 4; ++b) mx = max(mx, (int)((word >> (8 + 6 * b)) & 63));
                const bool live = dw <= WN;                              // (dropped for every d)
                R = max(R, live ? dw : 0);
                T = max(T, live ? mx << (WN - dw) : 0);
            }
        }
        R = max(R, __shfl_xor(R, 1, 64));
        T = max(T, __shfl_xor(T, 1, 64));
        // the largest |w''| of the row: max over live groups of m 2^(R - dw) * MAGMAX
        const int need = plainw ? MAGMAX : (T >> (WN - R)) * MAGMAX;
        uint32_t bad = need > 32256 ? 1u : 0u;
        for (int o = 32; o > 0; o >>= 1) {
            dm |= __shfl_xor(dm, o, 64);
            bad |= __shfl_xor(bad, o, 64);
        }
        if (h == 0) sR[r] = R;
        if (lane == 0) {
            sFlag[wid] = dm;
            sFlag[4 + wid] = bad;
        }
    }
    __syncthreads();
    // (read into scalar registers: the compiler then knows the tile's flags are uniform, and the
    // tests on them stay scalar branches instead of per-lane ones around each use)
    const uint32_t dall = __builtin_amdgcn_readfirstlane(sFlag[0] | sFlag[1] | sFlag[2] | sFlag[3]);
    const bool wide = __builtin_amdgcn_readfirstlane(sFlag[4] | sFlag[5] | sFlag[6] | sFlag[7]) != 0;
    const uint32_t dm = dall & ((1u << (WN + 1)) - 1);
    const bool over = (dall >> 31) != 0;
    const int np = __builtin_popcount(dm);
    const int dmin = dm ? __builtin_ctz(dm) : 0, dmax = dm ? 31 - __builtin_clz(dm) : 0;
    // Horner over the planes in int32: |sum_p 2^(dmax - d_p) C_p| <= K 127 128 (2^(dmax - dmin + 1) - 1)
    const bool fits = dm && (int64_t)a.K * 127 * 128 * ((2ll << (dmax - dmin)) - 1) < (1ll << 31);
    const bool single = np == 1 && !over;

    if (dm == 0 || !fits || wide) {
        // every group drops (acc 0), or the exact VALU path
        if (streamer) wait_vm<0>();             // (the first walk's first loads, issued before the scan)
        for (int idx = tid; idx < TM * TN; idx += 512) {
            const int r = idx / TN, c = idx % TN, m = m0 + r, n = n0 + c;
            if (m >= a.M || n >= a.N) continue;
            const int64_t acc = dm ? valu_acc4<FMT>(a, m, n, plainw) : 0;
            const float sw = unit ? 1.0f : ftz(*reinterpret_cast<const float*>(a.ws + (int64_t)n * a.srs));
            store_out(a, m, n, acc, sw, sSa2[r]);
        }
        return;
    }

    // The expansion of raw stage s into plane buffer s & 1 for activation plane d.  Every thread
    // of the workgroup expands one of the stage's 512 32-groups, gi = its thread index (row
    // gi / 4, the row's group gi % 4): the multiplying waves do theirs between their MFMAs,
    // whose matrix pipe runs beside the VALU (the streaming waves alone, two groups a thread,
    // took ~1.4 us a stage, latency-bound).  A read instruction reads 1 KB of raw nibbles
    // contiguously, free of bank conflicts.
    auto expand = [&](int s, int d) {
        const int8_t* slot = ringR + (s % NR) * RSLOT;
        int8_t* pl = planes + (s & 1) * 2 * PLANE;
        {
            const int gi = tid, row = gi >> 2, b = gi & 3;
            const uint4 x = *reinterpret_cast<const uint4*>(slot + 16 * gi);
            const int R = sR[row];
            // (arithmetic, no select: as a select the compiler loaded R only where the group is
            // live, a branch per lane that split the stage's code; a dropped group's shift is
            // masked, its multiplier 0)
            auto fold = [&](int m, int dw) { return (m << ((R - dw) & 31)) & -(int)(dw + d <= WN); };
            uint32_t l[8], hv[8];
            uint32_t tl[4], th[4];
            if (FT::NV) {
                // two 16-groups, each with its own E4M3 scale: elements 0-15 (x.x, x.y) and
                // 16-31 (x.z, x.w); the second table built after the first's last use
                const uint32_t e2 = *reinterpret_cast<const uint16_t*>(slot + RAWB + 8 * row + 2 * b);
                group_tables<FMT>(HI ? fold(nv_m(e2 & 0xFFu), nv_dw(e2 & 0xFFu)) : fold(1, 0), tl, th);
                expand8<HI>(x.x, tl, th, l[0], l[1], hv[0], hv[1]);
                expand8<HI>(x.y, tl, th, l[2], l[3], hv[2], hv[3]);
                group_tables<FMT>(HI ? fold(nv_m(e2 >> 8), nv_dw(e2 >> 8)) : fold(1, 0), tl, th);
            } else {
                const uint32_t word = *reinterpret_cast<const uint32_t*>(slot + RAWB + 4 * row);
                const int dw = HI ? (int)(word & 0xFF) : 0;
                const int m = HI ? (int)((word >> (8 + 6 * b)) & 63) : 1;
                group_tables<FMT>(fold(m, dw), tl, th);
                expand8<HI>(x.x, tl, th, l[0], l[1], hv[0], hv[1]);
                expand8<HI>(x.y, tl, th, l[2], l[3], hv[2], hv[3]);
            }
            expand8<HI>(x.z, tl, th, l[4], l[5], hv[4], hv[5]);
            expand8<HI>(x.w, tl, th, l[6], l[7], hv[6], hv[7]);
            *reinterpret_cast<uint4*>(pl + rof(row, 2 * b)) = make_uint4(l[0], l[1], l[2], l[3]);
            *reinterpret_cast<uint4*>(pl + rof(row, 2 * b + 1)) = make_uint4(l[4], l[5], l[6], l[7]);
            if (HI) {
                *reinterpret_cast<uint4*>(pl + PLANE + rof(row, 2 * b)) = make_uint4(hv[0], hv[1], hv[2], hv[3]);
                *reinterpret_cast<uint4*>(pl + PLANE + rof(row, 2 * b + 1)) = make_uint4(hv[4], hv[5], hv[6], hv[7]);
            }
        }
    };

    if (streamer) {
        for (uint32_t left = dm; left; left &= left - 1) {     // the activation planes in ascending d
            const int d = __builtin_ctz(left);
            if (left != dm) prologue_issue();
            else prologue_rest();               // (the first plane's first loads: before the scan)
            // raw 0 landed: younger than it the (A 0, raw 1) and (A 1, raw 2) issued
            wait_n((KS > 1 ? DMA_A + DMA_R : DMA_A) + (KS > 2 ? DMA_A + DMA_R : (KS > 1 ? DMA_A : 0)));
            bar();                              // every stream wave's raw 0 (and the planes' last reads)
            expand(0, d);
            // raw 1 and A 0 landed: younger than raw 1 the (A 1, raw 2)
            wait_n(KS > 2 ? DMA_A + DMA_R : (KS > 1 ? DMA_A : 0));
            bar();                              // stage 0 ready
            for (int kt = 0; kt < KS; ++kt) {
                int n = 0;
                if (kt + 2 < KS) { issue_a(kt + 2); n += DMA_A; }
                if (kt + 3 < KS) { issue_r(kt + 3); n += DMA_R; }
                if (kt + 1 < KS) expand(kt + 1, d);
                wait_n(n);                      // raw kt + 2 and A kt + 1 landed
                bar();                          // stage kt + 1 ready (or the walk's end)
            }
        }
    }
    v4i accl[4][4], acch[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) accl[i][j] = acch[i][j] = v4i{0, 0, 0, 0};
    int dprev = -1;
    for (uint32_t left = streamer ? 0u : dm; left; left &= left - 1) {   // the planes in ascending d
        const int d = __builtin_ctz(left);
        if (dprev >= 0) {                       // Horner: room for this plane
            const int gap = d - dprev;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    accl[i][j] = accl[i][j] << gap;
                    acch[i][j] = acch[i][j] << gap;
                }
        }
        bar();                                  // the streamers' raw 0
        expand(0, d);
        bar();                                  // stage 0 ready
        // stage kt's MFMAs, and (EXP) the expansion of stage kt + 1 issued between them: the
        // wave's VALU work runs in the matrix pipe's shadow (after them, it ran alone while the
        // streaming wave beside it on the SIMD waited at the barrier)
        auto mstage = [&](int kt, auto exp_next) {
            constexpr bool EXP = decltype(exp_next)::value;
            const int8_t* A = ringA + (kt % NA) * ATILE;
            const int8_t* PL = planes + (kt & 1) * 2 * PLANE;
            const uint32_t* daw = reinterpret_cast<const uint32_t*>(ringR + (kt % NR) * RSLOT + FT::DOFF);
            uint32_t dwd[4] = {0u, 0u, 0u, 0u};
            if (!single) {
#pragma unroll
                for (int i = 0; i < 4; ++i) dwd[i] = daw[wm * 64 + i * 16 + (lane & 15)];
            }
            __builtin_amdgcn_sched_barrier(0);
            // every fragment of the stage read before its MFMAs (per 64-deep step, the reads and
            // the MFMAs behind them ran in series)
            v4i fa[2][4], fl[2][4], fh[2][4];
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const int c = ks * 4 + (lane >> 4);
                const int gsh = 8 * (c >> 1);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    // (the other planes' groups masked arithmetically: as a select the compiler
                    // branched per lane around each fragment, splitting the stage's schedule)
                    const int keep = single || ((dwd[i] >> gsh) & 0xFFu) == (uint32_t)d ? -1 : 0;
                    fa[ks][i] = *reinterpret_cast<const v4i*>(A + rof(wm * 64 + i * 16 + (lane & 15), c)) & keep;
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int ro = rof(wn * 64 + j * 16 + (lane & 15), c);
                    fl[ks][j] = *reinterpret_cast<const v4i*>(PL + ro);
                    if (HI) fh[ks][j] = *reinterpret_cast<const v4i*>(PL + PLANE + ro);
                }
            }
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        accl[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[ks][i], fl[ks][j], accl[i][j], 0, 0, 0);
                        if (HI) acch[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[ks][i], fh[ks][j], acch[i][j], 0, 0, 0);
                    }
            if constexpr (EXP) expand(kt + 1, d);   // (raw kt + 1 landed before this stage's barrier)
            __builtin_amdgcn_sched_barrier(0);
        };
        for (int kt = 0; kt + 1 < KS; ++kt) {
            mstage(kt, std::true_type{});
            bar();                              // stage kt + 1 ready
            __builtin_amdgcn_sched_barrier(0);
        }
        mstage(KS - 1, std::false_type{});
        bar();                                  // the walk's end
        dprev = d;
    }

    // ---- epilogue: T = 256 C_h + C_l, acc = T 2^(W - R_n - dmax), the fp32 epilogue ----
    // Each wave's two planes of sums go to LDS column-major (the four rows an MFMA lane holds
    // are contiguous: one 16-byte write each), then a rolled loop over the wave's 16 row groups
    // (lane: row 4 s + lane / 16, columns 4 (lane & 15) .. + 3) forms each output and stores 4
    // columns at once.  i2f(acc) without int64 arithmetic: acc = T 2^sh is an integer (every live
    // term is), and rounding commutes with a power-of-two scale where the result stays normal (a
    // nonzero integer is at least 1), so i2f(acc) = ldexp(RNE(T), sh): T is exact in double
    // (|T| < 2^40), cvt_f32_f64 rounds it to nearest even, the ldexp is exact.
    // (full tiles: wave w stores row groups 0-7 of region w, stream wave w + 4 groups 8-15)
    const int region = wid & 3;
    int* Tl = reinterpret_cast<int*>(lds) + region * 2 * 64 * TPS;   // [column][row], TPS apart
    int* Th = Tl + 64 * TPS;
    if (!streamer) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int o = (16 * j + (lane & 15)) * TPS + 16 * i + 4 * (lane >> 4);
                *reinterpret_cast<v4i*>(Tl + o) = accl[i][j];
                if (HI) *reinterpret_cast<v4i*>(Th + o) = acch[i][j];
            }
    }
    __syncthreads();                                // the transposes written
    int sh[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        sw[c] = ftz(sw[c]);
        sh[c] = WN - sR[min(nc + c, a.N - 1) - n0] - dmax;
    }
    const bool full = m0 + TM <= a.M && n0 + TN <= a.N && a.vec4;
    const bool asc = (a.flags & OTPU_ASCALE) != 0, accf = (a.flags & OTPU_ACC) != 0;
    const int s0 = streamer ? 8 : 0;
    // (two row groups a trip: their LDS reads and conversion chains overlap; one a trip, each
    // waited on its reads with two waves a SIMD to hide them)
#pragma unroll 2
    for (int sgrp = s0; sgrp < s0 + 8; ++sgrp) {
        const int r = 4 * sgrp + (lane >> 4);      // the region's row
        const int m = m0 + wm * 64 + r;
        const float sa = sSa2[wm * 64 + r];
        float y[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int o = (4 * q + c) * TPS + r;
            const double T = (HI ? (double)Th[o] * 256.0 : 0.0) + (double)Tl[o];   // exact: |T| < 2^40
            y[c] = fmul_f(fmul_f(__builtin_ldexpf((float)T, sh[c]), sw[c]), sa);
        }
        float* p = a.out + (int64_t)m * a.ors + nc;
        if (full) {
            if (asc || accf) {
                const float4 old = *reinterpret_cast<const float4*>(p);
                const float ov[4] = {old.x, old.y, old.z, old.w};
                const float al = asc ? a.alpha[m] : 1.0f;
#pragma unroll
                for (int c = 0; c < 4; ++c) y[c] = asc ? fadd(fmul(ov[c], al), y[c]) : fadd(ov[c], y[c]);
            }
            typedef float f32x4 __attribute__((ext_vector_type(4)));
            __builtin_nontemporal_store(f32x4{y[0], y[1], y[2], y[3]}, reinterpret_cast<f32x4*>(p));
        } else if (m < a.M) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                if (nc + c >= a.N) continue;
                float v = y[c];
                if (asc) v = fadd(fmul(p[c], a.alpha[m]), v);
                else if (accf) v = fadd(p[c], v);
                p[c] = v;
            }
        }
    }
}

}  // namespace g4
}  // namespace otpu

using namespace otpu;

// returns 1 when the call is not for this kernel (otpu_mm then streams it), else a status
int otpu_gemm4_try(const int8_t* q, int64_t ldq, const float* Sa, const uint8_t* da, int64_t ldda, int M, int K,
                   const uint8_t* w, int64_t rs, const uint8_t* ws, int64_t srs, int N, int fmt, int flags, int k0,
                   const float* alpha, float* out, int64_t ors, hipStream_t s) {
    if ((fmt != OTPU_INT4 && fmt != OTPU_FP4 && fmt != OTPU_NVFP4) || M < 16 || (flags & OTPU_RMAX)) return 1;
    if (fmt == OTPU_NVFP4 && (flags & OTPU_RSC)) return 1;     // (no RSC form: the MM checks refuse it)
    if (((uintptr_t)da & 3) || (ldda % 4) || ((uintptr_t)q & 15) || (ldq % 16) || ((uintptr_t)w & 15) || (rs % 16))
        return 1;
    if (!(flags & OTPU_UNIT) && (((uintptr_t)ws & 3) || (srs % 4))) return 1;
    g4::Args a = {};
    a.q = q; a.ldq = ldq; a.Sa = Sa; a.da = da; a.ldda = ldda; a.M = M; a.K = K;
    a.w = w; a.rs = rs; a.ws = ws; a.srs = srs; a.N = N; a.flags = flags; a.k0 = k0;
    a.alpha = alpha; a.out = out; a.ors = ors;
    a.tiles_m = (M + g4::TM - 1) / g4::TM;
    a.tiles_n = (N + g4::TN - 1) / g4::TN;
    a.vec4 = ((uintptr_t)out % 16 == 0) && (ors % 4 == 0);
    const unsigned grid = (unsigned)(a.tiles_m * a.tiles_n);
    const bool hi = !(flags & (OTPU_UNIT | OTPU_RSC));
    if (fmt == OTPU_INT4) {
        if (hi) g4::gemm4_kernel<OTPU_INT4, true><<<grid, 512, 0, s>>>(a);
        else g4::gemm4_kernel<OTPU_INT4, false><<<grid, 512, 0, s>>>(a);
    } else if (fmt == OTPU_FP4) {
        if (hi) g4::gemm4_kernel<OTPU_FP4, true><<<grid, 512, 0, s>>>(a);
        else g4::gemm4_kernel<OTPU_FP4, false><<<grid, 512, 0, s>>>(a);
    } else {
        if (hi) g4::gemm4_kernel<OTPU_NVFP4, true><<<grid, 512, 0, s>>>(a);
        else g4::gemm4_kernel<OTPU_NVFP4, false><<<grid, 512, 0, s>>>(a);
    }
    return otpu_launch_check("mm gemm4");
}
