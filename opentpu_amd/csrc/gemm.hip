// MM for many activation rows on the int8 MFMA units (prefill GEMM), int8 weights with RSC,
// UNIT or int8x scale rows.  Semantics: opentpu/isasim.py:749-910 (docs/isa.md:226-305).
//
// Exactness.  MM's integer is acc = sum over 32-groups of 2^(16 - dw - da) * c (dropped where
// the shift is negative).  The weight offset dw is constant over a 128-block of a row and the
// activation offset da over a 32-group, so the sum splits into planes (d, e): the products
// whose activation group has da = d and whose weight block has dw = e, each plane an ordinary
// integer matrix product of masked int8 operands.  With s = d + e,
//     acc = 2^(16 - smax) * sum_s 2^(smax - s) * C_s,     C_s = sum over planes with d + e = s,
// evaluated by Horner's rule in the MFMA's own int32 accumulators (shift them left by the gap
// between successive s, then accumulate the next planes).  A tile whose bound
// K * 127^2 * 2^(smax - smin) reaches 2^31 takes a VALU path instead (exact, slow; it needs
// activation offsets spread over more than 6 binades inside one 128-row tile at K = 2048).
// ROW activations (every da = 0) with RSC or UNIT weights are the single plane s = 0: a plain
// MFMA GEMM with no masking.
//
// Work layout.  A workgroup (4 waves) owns a 128 x 128 output tile and streams K in 128-byte
// stages through LDS (double-buffered via registers; 16-byte chunks XOR-swizzled by row so the
// ds_read_b128 of a 16-row fragment hits distinct banks).  Each wave computes 64 x 64 with
// 4 x 4 v_mfma_i32_16x16x64_i8.  Tiles are assigned XCD-major: the workgroups of one XCD
// share weight rows, so each weight panel is fetched from HBM once into that XCD's L2.
#include <cstdlib>

#include "otpu_common.h"

namespace otpu {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int GBM = 128, GBN = 128, GBK = 128;

struct GemmArgs {
    const int8_t* q; int64_t ldq;
    const float* Sa;
    const uint8_t* da; int64_t ldda;
    int M, K;
    const int8_t* w; int64_t rs;
    const uint8_t* ws; int64_t srs;
    int N, flags, k0;
    const float* alpha;
    float* out; int64_t ors;
    int tiles_m, tiles_n;
    int vec4;                   // out 16-byte aligned and ors a multiple of 4: float4 stores
};

// byte offset of 16-byte chunk c of tile row r (rows of 128 bytes, chunks XOR-swizzled)
// The 16-byte slot of chunk c in row r is c ^ f(r), f(r) = ((r >> 1) & 7) ^ ((r & 1) << 2): the
// 8 rows a ds_read_b128 fragment's lanes 0-7 (and 8-15) read land in 8 distinct slots of a 128-byte
// bank window, and its 16 rows in 16 distinct (row parity, slot) pairs of a 256-byte one.
__device__ __forceinline__ int rowswz(int r) { return ((r >> 1) & 7) ^ ((r & 1) << 2); }
__device__ __forceinline__ int swz(int r, int c) { return r * GBK + ((c ^ rowswz(r)) << 4); }

__device__ __forceinline__ uint4 zero4() { return make_uint4(0, 0, 0, 0); }

// the VALU path of one output: the exact sum, group by group (rare tiles only)
__device__ __forceinline__ int64_t valu_acc(const GemmArgs& a, int j, int n, bool plain) {
    const int8_t* qr = a.q + (int64_t)j * a.ldq;
    const int8_t* wr = a.w + (int64_t)n * a.rs;
    const uint8_t* srow = a.ws + (int64_t)n * a.srs;
    int64_t acc = 0;
    for (int g = 0; g < a.K / 32; ++g) {
        const int* qa = reinterpret_cast<const int*>(qr + 32 * g);
        const int* wa = reinterpret_cast<const int*>(wr + 32 * g);
        int c = 0;
#pragma unroll
        for (int t = 0; t < 8; ++t) c = __builtin_amdgcn_sdot4(qa[t], wa[t], c, false);
        const int dw = plain ? 0 : (int)srow[4 + a.k0 + g / 4];
        const int sh = 16 - dw - (int)a.da[(int64_t)j * a.ldda + g];
        if (sh >= 0) acc += (int64_t)c << sh;
    }
    return acc;
}

struct Smem {
    int8_t (*A)[GBM * GBK];
    int8_t (*B)[GBN * GBK];
    uint32_t (*Da)[GBM];
    uint8_t (*Dw)[GBN];
    int8_t* ring;               // NS stages of A | B (the masked passes use its first 64 KB)
};

// one K stage of a thread's staged operands: 4 A and 4 B chunks, its row's da word / dw byte
// (named fields, no arrays: the stage stays in registers across the MFMAs)
struct GStage {
    uint4 a0, a1, a2, a3, b0, b1, b2, b3;
    uint32_t da, dw;
};

template <bool MA, bool MB>
__device__ __forceinline__ GStage gstage_load(const int8_t* const (&ga)[4], const int8_t* const (&gb)[4],
                                              const uint8_t* gda, const uint8_t* gdw, bool hasDa, bool hasDw, int kt) {
    GStage st;
    const int o = kt * GBK;
    st.a0 = *reinterpret_cast<const uint4*>(ga[0] + o);
    st.a1 = *reinterpret_cast<const uint4*>(ga[1] + o);
    st.a2 = *reinterpret_cast<const uint4*>(ga[2] + o);
    st.a3 = *reinterpret_cast<const uint4*>(ga[3] + o);
    st.b0 = *reinterpret_cast<const uint4*>(gb[0] + o);
    st.b1 = *reinterpret_cast<const uint4*>(gb[1] + o);
    st.b2 = *reinterpret_cast<const uint4*>(gb[2] + o);
    st.b3 = *reinterpret_cast<const uint4*>(gb[3] + o);
    st.da = (MA && hasDa) ? *reinterpret_cast<const uint32_t*>(gda + 4 * kt) : 0u;
    st.dw = (MB && hasDw) ? (uint32_t)gdw[kt] : 0u;
    return st;
}

// ---- the single-plane pipeline: a ring of NS K-stages in LDS, filled by direct-to-LDS loads ----
// A stage is the A and B tiles of 128 rows x RBK bytes; NS - 1 stages are in flight while one
// is multiplied.  global_load_lds_dwordx4 writes a wave's 64 x 16 bytes to 1 KB of LDS at M0
// (lane L at M0 + 16 L), so lane L of a wave's instruction fetches the global chunk that belongs
// at LDS slot L of its 1 KB block: with CPR = RBK / 16 chunks a row, row r = block * (64 / CPR)
// + L / CPR, stored slot L % CPR, i.e. the row's chunk (L % CPR) ^ rswz(r) (the XOR swizzle
// that puts the 16 rows a ds_read_b128 fragment reads on distinct banks).
// The loads are issued from inline assembly and their completion awaited with explicit
// s_waitcnt vmcnt(n): the compiler's own accounting would wait for every stage in flight.
#ifndef OTPU_RING_BK
#define OTPU_RING_BK 128
#endif
#ifndef OTPU_RING_NS
#define OTPU_RING_NS 4
#endif
constexpr int RBK = OTPU_RING_BK;               // K bytes a stage
constexpr int NS = OTPU_RING_NS;                // stages in the ring
constexpr int CPR = RBK / 16;                   // 16-byte chunks a row
constexpr int TILE = GBM * RBK;                 // bytes of one operand tile of a stage
constexpr int STAGE = 2 * TILE;                 // A then B
constexpr int LPS = 2 * TILE / 1024 / 4;        // direct loads a wave issues per stage
constexpr int RING = NS * STAGE > 2 * 2 * GBM * GBK ? NS * STAGE : 2 * 2 * GBM * GBK;
static_assert(RBK == 64 || RBK == 128, "ring stages of 64 or 128 bytes");
static_assert(NS >= 2 && (NS - 2) * LPS <= 63, "vmcnt holds at most 63");

__device__ __forceinline__ int rswz(int r) { return RBK == 128 ? rowswz(r) : (r >> 2) & 3; }
__device__ __forceinline__ int rof(int r, int c) { return r * RBK + ((c ^ rswz(r)) << 4); }

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

__device__ __forceinline__ void dma16(const int8_t* g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(g), "s"(lds) : "memory");
}

// wait until at most n of this wave's direct loads are outstanding
template <int N>
__device__ __forceinline__ void wait_dma() {
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// wait for stage kt when `ahead` later stages have been issued (ahead <= NS - 2)
__device__ __forceinline__ void wait_stage(int ahead) {
    switch (ahead) {
#define OTPU_WAIT_CASE(x) case x: if constexpr (x <= NS - 2) wait_dma<x * LPS>(); break;
        OTPU_WAIT_CASE(7) OTPU_WAIT_CASE(6) OTPU_WAIT_CASE(5) OTPU_WAIT_CASE(4)
        OTPU_WAIT_CASE(3) OTPU_WAIT_CASE(2) OTPU_WAIT_CASE(1)
#undef OTPU_WAIT_CASE
        default: wait_dma<0>();
    }
}

// LDS reads of the workgroup done, then the barrier (no fence: the direct loads are awaited
// by each wave before it arrives)
__device__ __forceinline__ void ring_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" : : : "memory");
}

// this lane's source rows of the ring's direct loads: instruction u of a stage reads row
// ga[u] (A, u < LPS / 2) or gb[u] (B); rows past M or N read the last valid row
struct RingSrc {
    const int8_t* ga[LPS / 2];
    const int8_t* gb[LPS / 2];
    uint32_t base;                              // the wave's LDS byte address in stage 0
};

__device__ __forceinline__ RingSrc ring_src(const GemmArgs& a, const int8_t* ring, int m0, int n0) {
    // (wave w mod 4: the loader waves 4-7 of gemm_lw_kernel issue what waves 0-3 would)
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane((threadIdx.x >> 6) & 3);
    RingSrc rs;
#pragma unroll
    for (int u = 0; u < LPS / 2; ++u) {
        const int blk = w * (LPS / 2) + u;
        const int r = blk * (64 / CPR) + lane / CPR, c = (lane % CPR) ^ rswz(r);
        rs.ga[u] = a.q + (int64_t)min(m0 + r, a.M - 1) * a.ldq + 16 * c;
        rs.gb[u] = a.w + (int64_t)min(n0 + r, a.N - 1) * a.rs + 16 * c;
    }
    rs.base = lds_addr(ring) + (uint32_t)(w * (LPS / 2) * 1024);
    return rs;
}

// walk step kt into its ring slot; dk: the K stage it holds (kt, or kt rotated: see lw_rot)
__device__ __forceinline__ void ring_issue(const RingSrc& rs, int kt, int dk) {
    const uint32_t sl = rs.base + (uint32_t)((kt % NS) * STAGE);
    const int o = dk * RBK;
#pragma unroll
    for (int u = 0; u < LPS / 2; ++u) dma16(rs.ga[u] + o, sl + 1024u * u);
#pragma unroll
    for (int u = 0; u < LPS / 2; ++u) dma16(rs.gb[u] + o, sl + TILE + 1024u * u);
}

// the first NS - 1 stages (issued before the tile's offsets and constants are known; a tile
// that turns out not to be single-plane waits for them and reuses the ring's memory)
__device__ __forceinline__ void ring_prologue(const GemmArgs& a, const int8_t* ring, int m0, int n0) {
    const RingSrc rs = ring_src(a, ring, m0, n0);
    const int KS = a.K / RBK;
#pragma unroll
    for (int s = 0; s < NS - 1; ++s)
        if (s < KS) ring_issue(rs, s, s);
}

// thread t's chunk u is tile row (t + 256 u) >> 3 = (t >> 3) + 32 u, chunk t & 7
template <bool MA, bool MB>
__device__ __forceinline__ void gstage_store(const Smem& sm, const GStage& st, int buf, bool hasDa, bool hasDw, int rr) {
    const int tid = threadIdx.x, r = tid >> 3, c = tid & 7;
    int8_t* A = sm.A[buf];
    int8_t* B = sm.B[buf];
    *reinterpret_cast<uint4*>(A + swz(r, c)) = st.a0;
    *reinterpret_cast<uint4*>(A + swz(r + 32, c)) = st.a1;
    *reinterpret_cast<uint4*>(A + swz(r + 64, c)) = st.a2;
    *reinterpret_cast<uint4*>(A + swz(r + 96, c)) = st.a3;
    *reinterpret_cast<uint4*>(B + swz(r, c)) = st.b0;
    *reinterpret_cast<uint4*>(B + swz(r + 32, c)) = st.b1;
    *reinterpret_cast<uint4*>(B + swz(r + 64, c)) = st.b2;
    *reinterpret_cast<uint4*>(B + swz(r + 96, c)) = st.b3;
    if (MA && hasDa) sm.Da[buf][rr] = st.da;
    if (MB && hasDw) sm.Dw[buf][rr] = (uint8_t)st.dw;
}

// the MFMAs of one LDS stage: two 64-byte K steps of 4 x 4 16x16x64 products per wave
template <bool MA, bool MB>
__device__ __forceinline__ void mfma_stage(const Smem& sm, int cur, v4i (&acc)[4][4], int d, int e) {
    const int lane = threadIdx.x & 63, wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wid >> 1, wn = wid & 1;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        const int c = ks * 4 + (lane >> 4);
        v4i fa[4], fb[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = wm * 64 + i * 16 + (lane & 15);
            uint4 v = *reinterpret_cast<const uint4*>(&sm.A[cur][swz(r, c)]);
            if (MA) {
                const bool keep = ((sm.Da[cur][r] >> (8 * (c >> 1))) & 0xFFu) == (uint32_t)d;
                v.x = keep ? v.x : 0u; v.y = keep ? v.y : 0u; v.z = keep ? v.z : 0u; v.w = keep ? v.w : 0u;
            }
            fa[i] = v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int r = wn * 64 + j * 16 + (lane & 15);
            uint4 v = *reinterpret_cast<const uint4*>(&sm.B[cur][swz(r, c)]);
            if (MB) {
                const bool keep = sm.Dw[cur][r] == (uint8_t)e;
                v.x = keep ? v.x : 0u; v.y = keep ? v.y : 0u; v.z = keep ? v.z : 0u; v.w = keep ? v.w : 0u;
            }
            fb[j] = v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
}

// one plane (d, e) over all of K: C += mask_d(A) . mask_e(B)^T in the int32 accumulators.
// K / 128 + 1 barriers: gemm_lw_kernel's loader waves match them one for one
// (masked_barriers), so a change to their number changes masked_barriers with it.
// MA / MB: mask the activation groups by da == d / the weight blocks by dw == e (false: every
// group of the tile is in the plane).  Rows past M or N are loaded from the last valid row
// (no branches, no waits in the load path): they only reach outputs the epilogue skips.
template <bool MA, bool MB>
__device__ __forceinline__ void gemm_pass(const GemmArgs& a, const Smem& sm, v4i (&acc)[4][4], int m0, int n0,
                                          int d, int e) {
    const int tid = threadIdx.x;
    const int KT = a.K / GBK;
    // each thread stages 4 A and 4 B chunks of 16 bytes a K stage: rows p >> 3, chunks p & 7
    const int8_t* ga[4];
    const int8_t* gb[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int p = tid + 256 * u, r = p >> 3, c = p & 7;
        ga[u] = a.q + (int64_t)min(m0 + r, a.M - 1) * a.ldq + 16 * c;
        gb[u] = a.w + (int64_t)min(n0 + r, a.N - 1) * a.rs + 16 * c;
    }
    const bool hasDa = MA && tid < GBM, hasDw = MB && tid >= GBM;
    const int rr = tid & (GBM - 1);
    const uint8_t* gda = a.da + (int64_t)min(m0 + rr, a.M - 1) * a.ldda;
    const uint8_t* gdw = a.ws + (int64_t)min(n0 + rr, a.N - 1) * a.srs + 4 + a.k0;

    {
        const GStage st = gstage_load<MA, MB>(ga, gb, gda, gdw, hasDa, hasDw, 0);
        gstage_store<MA, MB>(sm, st, 0, hasDa, hasDw, rr);
    }
    __syncthreads();
    for (int kt = 0; kt + 1 < KT; ++kt) {           // stage kt + 1 loads while stage kt multiplies
        const GStage st = gstage_load<MA, MB>(ga, gb, gda, gdw, hasDa, hasDw, kt + 1);
        mfma_stage<MA, MB>(sm, kt & 1, acc, d, e);
        gstage_store<MA, MB>(sm, st, (kt & 1) ^ 1, hasDa, hasDw, rr);
        __syncthreads();
    }
    mfma_stage<MA, MB>(sm, (KT - 1) & 1, acc, d, e);
    __syncthreads();
}

// one unmasked plane over all of K through the LDS ring, whose first NS - 1 stages
// ring_prologue issued.  A stage's fragments are read from LDS up front; its MFMAs are then
// interleaved with the direct loads that refill the ring (one load every 4 MFMAs), so the
// matrix pipe and the load path work at the same time (issued in a block, the loads stall the
// wave behind the loads already in flight before its first MFMA).
__device__ __forceinline__ void gemm_pass_ring(const GemmArgs& a, int8_t* ring, v4i (&acc)[4][4], int m0, int n0) {
    const int lane = threadIdx.x & 63, wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wid >> 1, wn = wid & 1;
    const RingSrc rs = ring_src(a, ring, m0, n0);
    const int KS = a.K / RBK;
    constexpr int KSTEP = RBK / 64;                       // 64-deep MFMA steps a stage
    constexpr int EVERY = 16 * KSTEP / LPS;               // MFMAs per refill load
    for (int kt = 0; kt < KS; ++kt) {
        wait_stage(min(NS - 2, KS - 1 - kt));            // stage kt landed (this wave's part)
        ring_barrier();                                  // ... everywhere; stage kt - 1 read
        const int8_t* A = ring + (kt % NS) * STAGE;
        const int8_t* B = A + TILE;
        v4i fa[KSTEP][4], fb[KSTEP][4];
#pragma unroll
        for (int ks = 0; ks < KSTEP; ++ks) {
            const int c = ks * 4 + (lane >> 4);
#pragma unroll
            for (int i = 0; i < 4; ++i) fa[ks][i] = *reinterpret_cast<const v4i*>(A + rof(wm * 64 + i * 16 + (lane & 15), c));
#pragma unroll
            for (int j = 0; j < 4; ++j) fb[ks][j] = *reinterpret_cast<const v4i*>(B + rof(wn * 64 + j * 16 + (lane & 15), c));
        }
        const int nk = kt + NS - 1;                       // the stage the refill loads fetch
        const bool refill = nk < KS;
        const uint32_t sl = rs.base + (uint32_t)((nk % NS) * STAGE);
        const int o = nk * RBK;
#pragma unroll
        for (int ks = 0; ks < KSTEP; ++ks)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[ks][i], fb[ks][j], acc[i][j], 0, 0, 0);
                    const int x = (ks * 16 + i * 4 + j);
                    if (x % EVERY == EVERY - 1 && refill) {
                        const int u = x / EVERY;
                        __builtin_amdgcn_sched_barrier(0);
                        if (u < LPS / 2) dma16(rs.ga[u] + o, sl + 1024u * u);
                        else dma16(rs.gb[u - LPS / 2] + o, sl + TILE + 1024u * (u - LPS / 2));
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
    }
    ring_barrier();
}

// Several activation planes in one K walk (plain weights: every dw = 0, so plane s = d): the
// ring and its direct loads as in gemm_pass_ring, and each stage's A fragments multiplied once
// per plane, masked to the 32-groups whose offset is that plane's d (groups of no listed plane,
// e.g. offsets past the window, are dropped).  The planes' products go to separate int32
// accumulators, combined after the walk: acc = sum_p C_p << (smax - d_p), Horner's sum unrolled.
// The group offsets of the tile come from LDS (da_lds: row r's word of stage kt at r * DAS + kt,
// four offsets a word, staged by the offset scan).  One pass of loads serves every plane.
constexpr int MP_MAX = 3;                       // planes one walk carries (64 registers of sums each;
                                                // 4 spill)
constexpr int MP_KT = 32;                       // stages (K = 4096) the staged offsets cover
constexpr int DAS = MP_KT + 1;                  // their row stride in words (16 rows on 16 banks)

template <int NP>
__device__ __forceinline__ void gemm_pass_mp(const GemmArgs& a, int8_t* ring, const uint32_t* da_lds,
                                             v4i (&acc)[MP_MAX][4][4], const int (&dv)[MP_MAX], int m0, int n0) {
    const int lane = threadIdx.x & 63, wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wid >> 1, wn = wid & 1;
    const RingSrc rs = ring_src(a, ring, m0, n0);
    const int KS = a.K / RBK;
    constexpr int KSTEP = RBK / 64;
    constexpr int EVERY = 16 * KSTEP * NP / LPS;          // MFMAs per refill load
    static_assert(RBK == 128, "offset words cover 128-byte stages");
    for (int kt = 0; kt < KS; ++kt) {
        wait_stage(min(NS - 2, KS - 1 - kt));
        ring_barrier();
        const int8_t* A = ring + (kt % NS) * STAGE;
        const int8_t* B = A + TILE;
        v4i fa[KSTEP][4], fb[KSTEP][4];
        uint32_t dw4[4];                                   // this lane's rows' offset words
#pragma unroll
        for (int i = 0; i < 4; ++i) dw4[i] = da_lds[(wm * 64 + i * 16 + (lane & 15)) * DAS + kt];
#pragma unroll
        for (int ks = 0; ks < KSTEP; ++ks) {
            const int c = ks * 4 + (lane >> 4);
#pragma unroll
            for (int i = 0; i < 4; ++i) fa[ks][i] = *reinterpret_cast<const v4i*>(A + rof(wm * 64 + i * 16 + (lane & 15), c));
#pragma unroll
            for (int j = 0; j < 4; ++j) fb[ks][j] = *reinterpret_cast<const v4i*>(B + rof(wn * 64 + j * 16 + (lane & 15), c));
        }
        const int nk = kt + NS - 1;
        const bool refill = nk < KS;
        const uint32_t sl = rs.base + (uint32_t)((nk % NS) * STAGE);
        const int o = nk * RBK;
#pragma unroll
        for (int ks = 0; ks < KSTEP; ++ks) {
            // the 16 bytes at chunk c are 32-group c >> 1 of the stage: offset byte (c >> 1)
            const int gsh = 8 * ((ks * 4 + (lane >> 4)) >> 1);
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                v4i fm[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const bool keep = ((dw4[i] >> gsh) & 0xFFu) == (uint32_t)dv[p];
                    fm[i] = keep ? fa[ks][i] : v4i{0, 0, 0, 0};
                }
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        acc[p][i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fm[i], fb[ks][j], acc[p][i][j], 0, 0, 0);
                        const int x = (ks * NP + p) * 16 + i * 4 + j;
                        if (x % EVERY == EVERY - 1 && refill) {
                            const int u = x / EVERY;
                            __builtin_amdgcn_sched_barrier(0);
                            if (u < LPS / 2) dma16(rs.ga[u] + o, sl + 1024u * u);
                            else dma16(rs.gb[u - LPS / 2] + o, sl + TILE + 1024u * (u - LPS / 2));
                            __builtin_amdgcn_sched_barrier(0);
                        }
                    }
            }
        }
    }
    ring_barrier();
}

// The epilogue of a tile whose MM integers are acc << sh (acc the int32 sums, sh = 16 - smax >= 0):
// y = (i2f(acc << sh) * Sw[n]) * (Sa[m] * 2^-16), then ACC / ASCALE.  i2f(acc << sh) is the int32's
// RNE float times 2^sh exactly.  sa2: the tile's rows' Sa * 2^-16 in LDS (row r of the tile at r).
// A full tile leaves through LDS: each wave writes its 64 x 64 accumulators in the MFMA layout
// (rows 68 words apart: the 4 row groups of a write land on distinct banks) and reads them back
// as 4-column rows, so every store instruction writes 4 rows x 256 contiguous bytes.  The scaling
// runs after the transpose, in a loop over the 16 row groups a lane stores: the tile runs once per
// CU from a cold instruction cache, so the epilogue's code length is its latency (unrolled over
// all 64 values it was 128 rounded products of straight-line code).  `lds` is the ring's memory
// (every wave is past its last read of the ring when the epilogue starts).
constexpr int TPS = 68;                         // transpose row stride, words

// a wave's 64 x 64 accumulators into its transpose region T (rows TPS words apart)
__device__ __forceinline__ void epi_transpose(int* T, const v4i (&acc)[4][4]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int t = 0; t < 4; ++t) T[(16 * i + 4 * (lane >> 4) + t) * TPS + 16 * j + (lane & 15)] = acc[i][j][t];
}

// this lane's 4 columns' Sw in region w's epilogue rows (1 with UNIT), as loaded: epi_rows
// flushes them where it uses them, so that no wait for these loads comes before that
__device__ __forceinline__ void epi_sw(const GemmArgs& a, int n0, int w, float (&sw)[4]) {
    const bool unit = (a.flags & OTPU_UNIT) != 0;
    const int nc = n0 + (w & 1) * 64 + 4 * (threadIdx.x & 15);
#pragma unroll
    for (int c = 0; c < 4; ++c) sw[c] = unit ? 1.0f : *reinterpret_cast<const float*>(a.ws + (int64_t)(nc + c) * a.srs);
}

// row groups s0 .. s1 - 1 of region w's 16 (region w: the 64 x 64 of wave w) from T, scaled by
// sw (epi_sw) and Sa and stored as 4-row x 256-byte float4 rows
__device__ __forceinline__ void epi_rows(const GemmArgs& a, const int* T, const float* sa2, int m0, int n0, int w,
                                         int s0, int s1, int sh, const float (&sw)[4]) {
    const int lane = threadIdx.x & 63;
    const int q = lane & 15, g = lane >> 4;
    const int rt = (w >> 1) * 64 + g;                          // the tile row of group s = 0
    const int nc = n0 + (w & 1) * 64 + 4 * q;
    const float swf[4] = {ftz(sw[0]), ftz(sw[1]), ftz(sw[2]), ftz(sw[3])};
    const bool asc = (a.flags & OTPU_ASCALE) != 0, accf = (a.flags & OTPU_ACC) != 0;
#pragma unroll 2
    for (int s = s0; s < s1; ++s) {
        const int r = rt + 4 * s;
        const int4 raw = *reinterpret_cast<const int4*>(T + (g + 4 * s) * TPS + 4 * q);
        const float sa = sa2[r];
        float y[4] = {ldexpf((float)raw.x, sh), ldexpf((float)raw.y, sh), ldexpf((float)raw.z, sh),
                      ldexpf((float)raw.w, sh)};
#pragma unroll
        for (int c = 0; c < 4; ++c) y[c] = fmul_f(fmul_f(y[c], swf[c]), sa);
        float* p = a.out + (int64_t)(m0 + r) * a.ors + nc;
        if (asc || accf) {
            const float4 old = *reinterpret_cast<const float4*>(p);
            const float o[4] = {old.x, old.y, old.z, old.w};
            const float al = asc ? a.alpha[m0 + r] : 1.0f;
#pragma unroll
            for (int c = 0; c < 4; ++c) y[c] = asc ? fadd(fmul(o[c], al), y[c]) : fadd(o[c], y[c]);
        }
#ifndef OTPU_GEMM_NT_STORE
#define OTPU_GEMM_NT_STORE 1
#endif
#if OTPU_GEMM_NT_STORE
        typedef float f32x4 __attribute__((ext_vector_type(4)));
        __builtin_nontemporal_store(f32x4{y[0], y[1], y[2], y[3]}, reinterpret_cast<f32x4*>(p));
#else
        *reinterpret_cast<float4*>(p) = make_float4(y[0], y[1], y[2], y[3]);
#endif
    }
}

__device__ __forceinline__ void tile_epilogue(const GemmArgs& a, int8_t* lds, const float* sa2, int m0, int n0,
                                              const v4i (&acc)[4][4], int sh) {
    const int lane = threadIdx.x & 63, wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const bool unit = (a.flags & OTPU_UNIT) != 0;
    const bool full = m0 + GBM <= a.M && n0 + GBN <= a.N;
    if (full && a.vec4) {
        int* T = reinterpret_cast<int*>(lds) + wid * 64 * TPS;
        float sw[4];
        epi_sw(a, n0, wid, sw);
        epi_transpose(T, acc);
        epi_rows(a, T, sa2, m0, n0, wid, 0, 16, sh, sw);
        return;
    }
    // a partial tile (or an unaligned output): each lane's own values, in the MFMA layout
    const int mb = m0 + (wid >> 1) * 64 + 4 * (lane >> 4), nb = n0 + (wid & 1) * 64 + (lane & 15);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int n = nb + j * 16;
        const float sw = (unit || n >= a.N) ? 1.0f : ftz(*reinterpret_cast<const float*>(a.ws + (int64_t)n * a.srs));
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int m = mb + i * 16 + t;
                if (m >= a.M || n >= a.N) continue;
                float y = fmul_f(fmul_f(ldexpf((float)acc[i][j][t], sh), sw), sa2[m - m0]);
                float* o = a.out + (int64_t)m * a.ors + n;
                if (a.flags & OTPU_ASCALE) y = fadd(fmul(*o, a.alpha[m]), y);
                else if (a.flags & OTPU_ACC) y = fadd(*o, y);
                *o = y;
            }
    }
}

// a tile of plain weights whose activation groups hold NP offsets d (planes s = d): one K walk
// (gemm_pass_mp), the planes' sums combined, then the epilogue
template <int NP>
__device__ __forceinline__ void gemm_tile_mp(const GemmArgs& a, int8_t* ring, const uint32_t* da_lds, int m0, int n0,
                                             uint32_t dmask, int smax, const float* sa2) {
    int dv[MP_MAX];
    uint32_t left = dmask;
#pragma unroll
    for (int p = 0; p < MP_MAX; ++p) {               // the planes' d in ascending order
        dv[p] = left ? __builtin_ctz(left) : 255;
        left &= left - 1;
    }
    v4i acc[MP_MAX][4][4];
#pragma unroll
    for (int p = 0; p < MP_MAX; ++p)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[p][i][j] = v4i{0, 0, 0, 0};
    gemm_pass_mp<NP>(a, ring, da_lds, acc, dv, m0, n0);
    // sum_p C_p << (smax - d_p) = C << (16 - smax) with C an int32 (the bound checked by the caller)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            v4i t = acc[0][i][j] << (smax - dv[0]);
#pragma unroll
            for (int p = 1; p < NP; ++p) t += acc[p][i][j] << (smax - dv[p]);
            acc[0][i][j] = t;
        }
    tile_epilogue(a, ring, sa2, m0, n0, acc[0], 16 - smax);
}

// a tile's planes in ascending s (Horner in the int32 accumulators), then its epilogue (its
// (d, e) loop is masked_barriers' loop: keep the two the same)
template <bool MA, bool MB>
__device__ __forceinline__ void gemm_tile(const GemmArgs& a, const Smem& sm, int m0, int n0, uint32_t dmask,
                                          uint32_t emask, uint32_t smask, int smin, int smax, const float* sa2) {
    v4i acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = v4i{0, 0, 0, 0};
    int sprev = -1;
    for (int s = smin; s <= smax; ++s) {
        if (!(smask >> s & 1)) continue;
        if (sprev >= 0) {                                  // Horner: make room for plane s
            const int gap = s - sprev;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = acc[i][j] << gap;
        }
        sprev = s;
        for (int d = 0; d <= s; ++d) {
            const int e = s - d;
            if (!(dmask >> d & 1) || e > 16 || !(emask >> e & 1)) continue;
            if (!MA && !MB) gemm_pass_ring(a, sm.ring, acc, m0, n0);
            else gemm_pass<MA, MB>(a, sm, acc, m0, n0, d, e);
        }
    }
    // acc = C << (16 - smax) with C an int32: i2f(acc) = rne(C) * 2^(16 - smax), exactly
    tile_epilogue(a, sm.ring, sa2, m0, n0, acc, 16 - smax);
}

// The offsets present in a tile -- d over its activation rows, e over its weight rows, bit 17
// for offsets past the window -- into sMask[2 w], sMask[2 w + 1] for each wave w of threads
// 0-255, and the activation words into sDaAll (K <= 4096).  Packed offset rows (ldda = K / 32
// bytes, 16-byte aligned, the tile's rows all present) are one contiguous block, read with
// coalesced 16-byte loads: each line once.  Otherwise two threads a row read its words (each
// load instruction then touches 64 rows' lines, and the tile's 64 lines are requested ~32 times
// over: at the c3 shape that took the scan to 2.9 us, its requests queued among the ring's).
__device__ __forceinline__ void tile_offsets(const GemmArgs& a, int m0, int n0, int KT, bool plain,
                                             uint32_t* sDaAll, uint32_t* sMask) {
    const int tid = threadIdx.x & 255, lane = tid & 63, wid = tid >> 6;
    uint32_t dm = 0, em = 0;
    auto take = [&](uint32_t wd) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t d = (wd >> (8 * t)) & 0xFF;
            dm |= 1u << (d <= 16 ? d : 17);
        }
    };
    const uint8_t* blk = a.da + (int64_t)m0 * a.ldda;
    const bool packed = a.ldda == 4 * KT && (KT & 3) == 0 && ((uintptr_t)blk & 15) == 0 && m0 + GBM <= a.M;
    if (packed) {
        const uint4* v = reinterpret_cast<const uint4*>(blk);
        const int NV = GBM * KT / 4;                     // 16-byte pieces of the tile's block
        for (int i = tid; i < NV; i += 256) {
            const uint4 q = v[i];
            const int r = 4 * i / KT, k = 4 * i % KT;     // row r, words k .. k + 3
            if (KT <= MP_KT) {
                sDaAll[r * DAS + k] = q.x;
                sDaAll[r * DAS + k + 1] = q.y;
                sDaAll[r * DAS + k + 2] = q.z;
                sDaAll[r * DAS + k + 3] = q.w;
            }
            take(q.x);
            take(q.y);
            take(q.z);
            take(q.w);
        }
    } else {
        const int r = tid & (GBM - 1), h = tid >> 7;
        if (m0 + r < a.M) {
            const uint32_t* drow = reinterpret_cast<const uint32_t*>(a.da + (int64_t)(m0 + r) * a.ldda);
#pragma unroll 8
            for (int k = h; k < KT; k += 2) {             // K / 128 words of four offsets
                const uint32_t wd = drow[k];
                if (KT <= MP_KT) sDaAll[r * DAS + k] = wd;
                take(wd);
            }
        }
    }
    if (plain) {
        em = 1u;
    } else {
        const int r = tid & (GBN - 1), h = tid >> 7;
        if (n0 + r < a.N) {
            const uint8_t* wrow = a.ws + (int64_t)(n0 + r) * a.srs + 4 + a.k0;
#pragma unroll 8
            for (int k = h; k < KT; k += 2) {
                const uint32_t e = wrow[k];
                em |= 1u << (e <= 16 ? e : 17);
            }
        }
    }
    for (int o = 32; o > 0; o >>= 1) {
        dm |= __shfl_xor(dm, o, 64);
        em |= __shfl_xor(em, o, 64);
    }
    if (lane == 0) {
        sMask[2 * wid] = dm;
        sMask[2 * wid + 1] = em;
    }
}

// the barriers gemm_tile<true, MB> executes: K / 128 + 1 for each (d, e) pass it makes
__device__ __forceinline__ int masked_barriers(int KT, uint32_t dmask, uint32_t emask, uint32_t smask, int smin,
                                               int smax) {
    int passes = 0;
    for (int s = smin; s <= smax; ++s) {
        if (!(smask >> s & 1)) continue;
        for (int d = 0; d <= s; ++d) {
            const int e = s - d;
            if (!(dmask >> d & 1) || e > 16 || !(emask >> e & 1)) continue;
            ++passes;
        }
    }
    return passes * (KT + 1);
}

// ---- loader waves: workgroups of 8 waves, 4 of them streaming the ring, 4 multiplying ----
// With one wave a SIMD doing both, a direct load that finds the load path full stalls the
// wave's issue and the MFMAs behind it wait: a stage's loads and MFMAs add up instead of
// overlapping.  Here waves 4-7 issue every direct load (the first NS - 1 stages before the
// tile's offset scan) and waves 0-3 only read fragments and multiply; the two groups meet at
// one barrier a stage.  A loader arrives once its part of stage kt has landed and then refills
// the slot stage kt - 1 left; a compute wave arrives with its reads of stage kt - 1 done.
// (c3 ROW x RSC: 18.5-18.7 -> 16.3-16.6 us back to back, bit-identical.)

// The K walk of a tile starts at stage rot and wraps (the int32 sums are exact in any order).
// The workgroups of one XCD run in step, so with one common order the tiles that share an A or
// a B panel ask for each line together and all wait a miss's latency for it (L2 merges the
// requests).  Staggered starts let one tile miss a line and the others hit it in L2 stages
// later: the 8 tiles of an XCD that share A rows start 2 stages apart, the 4 that share B rows
// 4 stages apart (tn & 7 and tm: the XCD-major order gives an XCD 8 consecutive column tiles).
__device__ __forceinline__ int lw_rot(int tm, int tn, int KS) { return (2 * (tn & 7) + 4 * tm) % KS; }
__device__ __forceinline__ int lw_stage(int kt, int rot, int KS) { return kt + rot < KS ? kt + rot : kt + rot - KS; }

// a loader wave's walk (its first NS - 1 stages issued): KS + 1 barriers
__device__ __forceinline__ void lw_load_walk(const RingSrc& rs, int KS, int rot) {
    for (int kt = 0; kt < KS; ++kt) {
        wait_stage(min(NS - 2, KS - 1 - kt));
        ring_barrier();                                  // stage kt landed (this wave's part)
        const int nk = kt + NS - 1;
        if (nk < KS) ring_issue(rs, nk, lw_stage(nk, rot, KS));
    }
    ring_barrier();
}

// a compute wave's walk: NP planes into acc[p]; MASK: each stage's A fragments masked to plane
// p's 32-groups (plain weights, offsets from da_lds as in gemm_pass_mp), else the single plane.
// ALL1 (two planes covering every group): plane 1's product taken over every group instead,
// C_all, so that only plane 0 is masked (C_1 = C_all - C_0 afterwards, exactly in int32).
// KS + 1 barriers, matching lw_load_walk's.
template <int NP, bool MASK, bool ALL1 = false>
__device__ __forceinline__ void lw_mma_walk(const int8_t* ring, const uint32_t* da_lds, v4i (&acc)[NP][4][4],
                                            const int (&dv)[MP_MAX], int KS, int rot) {
    const int lane = threadIdx.x & 63, wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wid >> 1, wn = wid & 1;
    for (int kt = 0; kt < KS; ++kt) {
        ring_barrier();                                  // stage kt landed everywhere
        const int8_t* A = ring + (kt % NS) * STAGE;
        const int8_t* B = A + TILE;
        uint32_t dw4[4] = {0u, 0u, 0u, 0u};
        if constexpr (MASK) {
            const int dk = lw_stage(kt, rot, KS);
#pragma unroll
            for (int i = 0; i < 4; ++i) dw4[i] = da_lds[(wm * 64 + i * 16 + (lane & 15)) * DAS + dk];
        }
        v4i fa[2][4], fb[2][4];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int c = ks * 4 + (lane >> 4);
#pragma unroll
            for (int i = 0; i < 4; ++i) fa[ks][i] = *reinterpret_cast<const v4i*>(A + rof(wm * 64 + i * 16 + (lane & 15), c));
#pragma unroll
            for (int j = 0; j < 4; ++j) fb[ks][j] = *reinterpret_cast<const v4i*>(B + rof(wn * 64 + j * 16 + (lane & 15), c));
        }
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int gsh = 8 * ((ks * 4 + (lane >> 4)) >> 1);   // the chunk's 32-group offset byte
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                v4i fm[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const bool keep = !MASK || (ALL1 && p == 1) || ((dw4[i] >> gsh) & 0xFFu) == (uint32_t)dv[p];
                    fm[i] = keep ? fa[ks][i] : v4i{0, 0, 0, 0};
                }
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        acc[p][i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fm[i], fb[ks][j], acc[p][i][j], 0, 0, 0);
            }
        }
    }
    ring_barrier();                                      // every read of the ring done
}

// the barrier of a walk whose LDS reads the compiler tracks: its own wait for every LDS read
// (so no later wait on those reads is inserted), the barrier, and a fence that keeps the next
// stage's reads below it
__device__ __forceinline__ void ring_barrier_tracked() {
    __builtin_amdgcn_s_waitcnt(0xC07F);                  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" : : : "memory");
}

// NP planes (as lw_mma_walk's; the kernels use it for one) with the fragment reads half a stage
// ahead (for two planes it measured no faster, its accumulators spilling a few registers).  A stage's
// fragments are two halves (K chunks 0-3 and 4-7 of its 128 bytes, 8 ds_read_b128 each);
// between barriers kt + 1 and kt + 2 a wave reads half 0 of stage kt + 1, multiplies half 1 of
// stage kt, reads half 1 of stage kt + 1 and multiplies its half 0, one read issued per 2 NP
// MFMAs, so the reads run under the MFMAs (read, then multiplied, a one-plane stage took ~1000
// cycles, twice the MFMAs' 512).  Barrier j still follows every read of stage j - 1, so the
// loaders refill its slot as lw_load_walk does.  KS + 1 barriers.
struct Half {
    v4i a[4], b[4];
};

template <bool MASK>
__device__ __forceinline__ void lw_half_read(const int8_t* ring, const uint32_t* da_lds, Half& h, uint32_t (&dw)[4],
                                             int kt, int ks, int KS, int rot) {
    const int lane = threadIdx.x & 63, wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wid >> 1, wn = wid & 1;
    const int8_t* A = ring + (kt % NS) * STAGE;
    const int8_t* B = A + TILE;
    if (MASK && ks == 0) {
        const int dk = lw_stage(kt, rot, KS);
#pragma unroll
        for (int i = 0; i < 4; ++i) dw[i] = da_lds[(wm * 64 + i * 16 + (lane & 15)) * DAS + dk];
    }
    const int c = ks * 4 + (lane >> 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) h.a[i] = *reinterpret_cast<const v4i*>(A + rof(wm * 64 + i * 16 + (lane & 15), c));
#pragma unroll
    for (int j = 0; j < 4; ++j) h.b[j] = *reinterpret_cast<const v4i*>(B + rof(wn * 64 + j * 16 + (lane & 15), c));
}

template <int NP, bool MASK, bool ALL1>
__device__ __forceinline__ void lw_half_mma(const Half& h, const uint32_t (&dw)[4], v4i (&acc)[NP][4][4], int ks,
                                            const int (&dv)[MP_MAX]) {
    const int lane = threadIdx.x & 63;
    const int gsh = 8 * ((ks * 4 + (lane >> 4)) >> 1);
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        v4i fm[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const bool keep = !MASK || (ALL1 && p == 1) || ((dw[i] >> gsh) & 0xFFu) == (uint32_t)dv[p];
            fm[i] = keep ? h.a[i] : v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[p][i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fm[i], h.b[j], acc[p][i][j], 0, 0, 0);
    }
}

// (the scheduler would move the register-only MFMAs across the barriers and sink each read next
// to its use: sched_barrier closes every region, and the group barriers interleave each half's
// reads with the MFMAs that hide them)
#define OTPU_READS_UNDER_MMA(nr, np)                                                                \
    do {                                                                                           \
        if ((nr) > 8) __builtin_amdgcn_sched_group_barrier(0x100, (nr) - 8, 0);                    \
        _Pragma("unroll") for (int g_ = 0; g_ < 8; ++g_) {                                         \
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                                     \
            __builtin_amdgcn_sched_group_barrier(0x008, 2 * (np), 0);                              \
        }                                                                                          \
    } while (0)

template <int NP, bool MASK, bool ALL1 = false>
__device__ __forceinline__ void lw_mma_walk_h(const int8_t* ring, const uint32_t* da_lds, v4i (&acc)[NP][4][4],
                                              const int (&dv)[MP_MAX], int KS, int rot) {
    Half h0, h1;
    uint32_t dw[4] = {0u, 0u, 0u, 0u}, dwn[4] = {0u, 0u, 0u, 0u};
    ring_barrier_tracked();                              // stage 0 landed everywhere
    __builtin_amdgcn_sched_barrier(0);
    lw_half_read<MASK>(ring, da_lds, h0, dw, 0, 0, KS, rot);
    lw_half_read<MASK>(ring, da_lds, h1, dw, 0, 1, KS, rot);
    lw_half_mma<NP, MASK, ALL1>(h0, dw, acc, 0, dv);
    OTPU_READS_UNDER_MMA(MASK ? 20 : 16, NP);
    __builtin_amdgcn_sched_barrier(0);
    for (int kt = 0; kt + 1 < KS; ++kt) {
        ring_barrier_tracked();                          // stage kt + 1 landed, stage kt read
        __builtin_amdgcn_sched_barrier(0);
        lw_half_read<MASK>(ring, da_lds, h0, dwn, kt + 1, 0, KS, rot);
        lw_half_mma<NP, MASK, ALL1>(h1, dw, acc, 1, dv);
        OTPU_READS_UNDER_MMA(MASK ? 12 : 8, NP);
        lw_half_read<MASK>(ring, da_lds, h1, dwn, kt + 1, 1, KS, rot);
        lw_half_mma<NP, MASK, ALL1>(h0, dwn, acc, 0, dv);
        OTPU_READS_UNDER_MMA(8, NP);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 4; ++i) dw[i] = dwn[i];
    }
    ring_barrier_tracked();                              // the walk's end
    __builtin_amdgcn_sched_barrier(0);
    lw_half_mma<NP, MASK, ALL1>(h1, dw, acc, 1, dv);
}
#undef OTPU_READS_UNDER_MMA

// C3: a copy for the c3 prefill shape (M 512, N 8192, K 2048, dense rows, RSC scale words), its
// sizes and strides as constants (the kernel runs once a CU from a cold instruction cache)
#ifndef OTPU_GEMM_C3
#define OTPU_GEMM_C3 1
#endif
#ifndef OTPU_GEMM_LW
#define OTPU_GEMM_LW 1                  // loader waves (gemm_lw_kernel); 0: gemm_i8_kernel's one wave group
#endif
template <bool C3>
__global__ __launch_bounds__(256) void gemm_i8_kernel(GemmArgs a) {
    if constexpr (C3) {
        a.M = 512; a.N = 8192; a.K = 2048; a.ldq = 2048; a.rs = 2048; a.ldda = 64; a.srs = 4; a.ors = 8192;
        a.tiles_m = 4; a.tiles_n = 64; a.vec4 = 1;
    }
    __shared__ __align__(16) int8_t sRing[RING];
    __shared__ uint32_t sDa[2][GBM];       // the stage's four da bytes per activation row
    __shared__ uint8_t sDw[2][GBN];        // the stage's dw byte per weight row
    __shared__ uint32_t sMask[8];          // per wave: d values and e values present in the tile
    __shared__ uint32_t sDaAll[GBM * DAS]; // the tile's offset words (K <= 4096), for gemm_pass_mp
    __shared__ float sSa2[GBM];            // the tile rows' Sa * 2^-16

    const int tid = threadIdx.x, lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);

    // XCD-major tile order: workgroup b runs on XCD b % 8; give each XCD whole weight panels
    int b = blockIdx.x, tm, tn;
    const int ntiles = a.tiles_m * a.tiles_n;
    if (ntiles % 8 == 0 && a.tiles_n % 8 == 0) {
        const int per = ntiles / 8, x = b % 8, li = b / 8;
        const int t = x * per + li;                 // tiles of XCD x are contiguous in N
        tn = t / a.tiles_m;
        tm = t % a.tiles_m;
    } else {
        tn = b / a.tiles_m;
        tm = b % a.tiles_m;
    }
    const int m0 = tm * GBM, n0 = tn * GBN;
    const bool unit = (a.flags & OTPU_UNIT) != 0;
    const bool plain = unit || (a.flags & OTPU_RSC) != 0;
    const int KT = a.K / GBK;

    // the ring's first stages go out first: their latency overlaps the offset scan and the
    // epilogue constants (a masked tile waits for them before reusing the ring)
    ring_prologue(a, sRing, m0, n0);

    // the tile rows' Sa * 2^-16 for the epilogue (written before the scan's barrier)
    if (tid < GBM) sSa2[tid] = m0 + tid < a.M ? fmul(a.Sa[m0 + tid], pow2f(-16)) : 0.0f;
    // the offsets present in this tile
    tile_offsets(a, m0, n0, KT, plain, sDaAll, sMask);
    __syncthreads();
    uint32_t dall = 0, eall = 0;
#pragma unroll
    for (int x = 0; x < 4; ++x) {
        dall |= sMask[2 * x];
        eall |= sMask[2 * x + 1];
    }
    const uint32_t dmask = dall & 0x1FFFFu, emask = eall & 0x1FFFFu;
    // groups beyond the window exist: masking must drop them even with one live plane
    const bool over = ((dall | eall) >> 17) & 1;
    // the s = d + e values with a live plane, smin and smax
    uint32_t smask = 0;
    for (int d = 0; d <= 16; ++d)
        if (dmask >> d & 1) smask |= (emask << d) & 0x1FFFFu;

    if (smask == 0) {                               // every group drops: acc = 0
        wait_dma<0>();                              // (the ring prologue's loads end in LDS)
        ring_barrier();
        v4i z[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) z[i][j] = v4i{0, 0, 0, 0};
        tile_epilogue(a, sRing, sSa2, m0, n0, z, 0);
        return;
    }
    const int smin = __builtin_ctz(smask), smax = 31 - __builtin_clz(smask);
    // |acc| <= K * 127^2 * 2^(smax - smin) must stay below 2^31 in the int32 accumulators
    const bool fits = (int64_t)a.K * 16129 <= (((int64_t)1 << 31) - 1) >> (smax - smin);
    if (!fits) {
        wait_dma<0>();
        for (int idx = tid; idx < GBM * GBN; idx += 256) {
            const int r = idx / GBN, c = idx % GBN;
            const int m = m0 + r, n = n0 + c;
            if (m < a.M && n < a.N) {
                float y = fmul(fmul(i2f(valu_acc(a, m, n, plain)),
                                    unit ? 1.0f : *reinterpret_cast<const float*>(a.ws + (int64_t)n * a.srs)),
                               fmul(a.Sa[m], pow2f(-16)));
                float* o = a.out + (int64_t)m * a.ors + n;
                if (a.flags & OTPU_ASCALE) y = fadd(fmul(*o, a.alpha[m]), y);
                else if (a.flags & OTPU_ACC) y = fadd(*o, y);
                *o = y;
            }
        }
        return;
    }
    const bool single = !over && __builtin_popcount(dmask) == 1 && __builtin_popcount(emask) == 1;
    const Smem sm{reinterpret_cast<int8_t(*)[GBM * GBK]>(sRing),
                  reinterpret_cast<int8_t(*)[GBN * GBK]>(sRing + 2 * GBM * GBK), sDa, sDw, sRing};
    if (single) {
        gemm_tile<false, false>(a, sm, m0, n0, dmask, emask, smask, smin, smax, sSa2);
        return;
    }
    // plain weights, up to MP_MAX activation planes: one K walk through the ring for all of them
    const int np = __builtin_popcount(dmask);
    if (plain && KT <= MP_KT && np >= 1 && np <= MP_MAX) {
        switch (np) {
            case 1: gemm_tile_mp<1>(a, sRing, sDaAll, m0, n0, dmask, smax, sSa2); break;
            case 2: gemm_tile_mp<2>(a, sRing, sDaAll, m0, n0, dmask, smax, sSa2); break;
            default: gemm_tile_mp<3>(a, sRing, sDaAll, m0, n0, dmask, smax, sSa2); break;
        }
        return;
    }
    wait_dma<0>();                                  // the masked passes reuse the ring's memory
    ring_barrier();
    if (plain) gemm_tile<true, false>(a, sm, m0, n0, dmask, emask, smask, smin, smax, sSa2);
    else gemm_tile<true, true>(a, sm, m0, n0, dmask, emask, smask, smin, smax, sSa2);
}

// The GEMM with loader waves (workgroups of 8 waves; C3: the c3 shape's copy).  Waves 0-3 run everything
// gemm_i8_kernel's waves run (the offset scan, the epilogue, the masked passes); waves 4-7
// issue the ring's direct loads.  Tiles of one plane, or of one or two activation planes with
// plain weights, walk the ring with both groups; every other tile waits for the loaders' stages
// to land and runs on waves 0-3 alone, the loaders matching its barriers one for one
// (the masked passes') or leaving when none follow.
template <bool C3>
__global__ __launch_bounds__(512) void gemm_lw_kernel(GemmArgs a) {
    if constexpr (C3) {
        a.M = 512; a.N = 8192; a.K = 2048; a.ldq = 2048; a.rs = 2048; a.ldda = 64; a.srs = 4; a.ors = 8192;
        a.tiles_m = 4; a.tiles_n = 64; a.vec4 = 1;
    }
    __shared__ __align__(16) int8_t sRing[RING];
    __shared__ uint32_t sDa[2][GBM];
    __shared__ uint8_t sDw[2][GBN];
    __shared__ uint32_t sMask[8];
    __shared__ uint32_t sDaAll[GBM * DAS];
    __shared__ float sSa2[GBM];

    const int tid = threadIdx.x, lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool loader = wid >= 4;
    int b = blockIdx.x, tm, tn;
    const int ntiles = a.tiles_m * a.tiles_n;
    if (ntiles % 8 == 0 && a.tiles_n % 8 == 0) {
        const int per = ntiles / 8, x = b % 8, li = b / 8;
        const int t = x * per + li;
        tn = t / a.tiles_m;
        tm = t % a.tiles_m;
    } else {
        tn = b / a.tiles_m;
        tm = b % a.tiles_m;
    }
    const int m0 = tm * GBM, n0 = tn * GBN;
    const bool unit = (a.flags & OTPU_UNIT) != 0;
    const bool plain = unit || (a.flags & OTPU_RSC) != 0;
    const int KT = a.K / GBK, KS = a.K / RBK;
    const int rot = lw_rot(tm, tn, KS);

    const RingSrc rs = ring_src(a, sRing, m0, n0);
    // the epilogue's column scales, loaded early (a full tile's epilogue rows are shared by
    // wave w and loader w + 4, region w & 3): a loader's before its ring loads, which complete
    // in order after them (the stage waits' counts unchanged), a compute wave's after the
    // offset scan (whose waits would otherwise wait for them too)
    const bool split = m0 + GBM <= a.M && n0 + GBN <= a.N && a.vec4;
    float esw[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    if (loader) {
        if (split) epi_sw(a, n0, wid & 3, esw);
#pragma unroll
        for (int s = 0; s < NS - 1; ++s)
            if (s < KS) ring_issue(rs, s, lw_stage(s, rot, KS));
    } else {
        if (tid < GBM) sSa2[tid] = m0 + tid < a.M ? fmul(a.Sa[m0 + tid], pow2f(-16)) : 0.0f;
        tile_offsets(a, m0, n0, KT, plain, sDaAll, sMask);   // the offsets present in this tile
        if (split) epi_sw(a, n0, wid, esw);
    }
    __syncthreads();
    uint32_t dall = 0, eall = 0;
#pragma unroll
    for (int x = 0; x < 4; ++x) {
        dall |= sMask[2 * x];
        eall |= sMask[2 * x + 1];
    }
    const uint32_t dmask = dall & 0x1FFFFu, emask = eall & 0x1FFFFu;
    const bool over = ((dall | eall) >> 17) & 1;
    uint32_t smask = 0;
    for (int d = 0; d <= 16; ++d)
        if (dmask >> d & 1) smask |= (emask << d) & 0x1FFFFu;
    const int smin = smask ? __builtin_ctz(smask) : 0, smax = smask ? 31 - __builtin_clz(smask) : 0;
    const bool fits = smask && (int64_t)a.K * 16129 <= (((int64_t)1 << 31) - 1) >> (smax - smin);
    const bool single = !over && __builtin_popcount(dmask) == 1 && __builtin_popcount(emask) == 1;
    const int np = __builtin_popcount(dmask);
    const bool mp = !single && plain && KT <= MP_KT && np >= 1 && np <= 2;

    // a full tile's epilogue is shared: waves 0-3 write their transposes, then wave w and its
    // loader w + 4 store 8 row groups each (one more barrier for both groups)
    if (fits && (single || mp)) {
        if (loader) {
            lw_load_walk(rs, KS, rot);
            if (split) {
                __syncthreads();                         // the transposes written
                const int w = wid & 3;
                epi_rows(a, reinterpret_cast<const int*>(sRing) + w * 64 * TPS, sSa2, m0, n0, w, 8, 16, 16 - smax, esw);
            }
            return;
        }
        auto epilogue = [&](const v4i (&acc0)[4][4]) {
            if (split) {
                int* T = reinterpret_cast<int*>(sRing) + wid * 64 * TPS;
                epi_transpose(T, acc0);
                __syncthreads();
                epi_rows(a, T, sSa2, m0, n0, wid, 0, 8, 16 - smax, esw);
            } else {
                tile_epilogue(a, sRing, sSa2, m0, n0, acc0, 16 - smax);
            }
        };
        int dv[MP_MAX];
        uint32_t left = dmask;
#pragma unroll
        for (int p = 0; p < MP_MAX; ++p) {               // the planes' d in ascending order
            dv[p] = left ? __builtin_ctz(left) : 255;
            left &= left - 1;
        }
        if (single || np == 1) {                         // (one plane of plain weights: no masking
            v4i acc[1][4][4];                            // when its offset covers every group)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[0][i][j] = v4i{0, 0, 0, 0};
            if (single) lw_mma_walk_h<1, false>(sRing, sDaAll, acc, dv, KS, rot);
            else lw_mma_walk_h<1, true>(sRing, sDaAll, acc, dv, KS, rot);
            epilogue(acc[0]);
        } else {
            v4i acc[2][4][4];
#pragma unroll
            for (int p = 0; p < 2; ++p)
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[p][i][j] = v4i{0, 0, 0, 0};
            // (no offsets past the window: the two planes cover every group, so plane 1 is C_all)
            if (!over) lw_mma_walk<2, true, true>(sRing, sDaAll, acc, dv, KS, rot);
            else lw_mma_walk<2, true>(sRing, sDaAll, acc, dv, KS, rot);
            // sum_p C_p << (smax - d_p) (the bound checked above)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const v4i c1 = over ? acc[1][i][j] : acc[1][i][j] - acc[0][i][j];
                    acc[0][i][j] = (acc[0][i][j] << (smax - dv[0])) + (c1 << (smax - dv[1]));
                }
            epilogue(acc[0]);
        }
        return;
    }
    // every other tile: the loaders' stages land, then waves 0-3 alone
    if (loader) {
        wait_dma<0>();
        ring_barrier();
        const int nb = (smask && fits) ? masked_barriers(KT, dmask, emask, smask, smin, smax) : 0;
        for (int i = 0; i < nb; ++i) __syncthreads();    // the masked passes' barriers
        return;
    }
    ring_barrier();
    if (smask == 0) {                                    // every group drops: acc = 0
        v4i z[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) z[i][j] = v4i{0, 0, 0, 0};
        tile_epilogue(a, sRing, sSa2, m0, n0, z, 0);
        return;
    }
    if (!fits) {
        for (int idx = tid; idx < GBM * GBN; idx += 256) {
            const int r = idx / GBN, c = idx % GBN;
            const int m = m0 + r, n = n0 + c;
            if (m < a.M && n < a.N) {
                float y = fmul(fmul(i2f(valu_acc(a, m, n, plain)),
                                    unit ? 1.0f : *reinterpret_cast<const float*>(a.ws + (int64_t)n * a.srs)),
                               fmul(a.Sa[m], pow2f(-16)));
                float* o = a.out + (int64_t)m * a.ors + n;
                if (a.flags & OTPU_ASCALE) y = fadd(fmul(*o, a.alpha[m]), y);
                else if (a.flags & OTPU_ACC) y = fadd(*o, y);
                *o = y;
            }
        }
        return;
    }
    const Smem sm{reinterpret_cast<int8_t(*)[GBM * GBK]>(sRing),
                  reinterpret_cast<int8_t(*)[GBN * GBK]>(sRing + 2 * GBM * GBK), sDa, sDw, sRing};
    if (plain) gemm_tile<true, false>(a, sm, m0, n0, dmask, emask, smask, smin, smax, sSa2);
    else gemm_tile<true, true>(a, sm, m0, n0, dmask, emask, smask, smin, smax, sSa2);
}

}  // namespace otpu

using namespace otpu;

// returns 1 when the call is not for this kernel (otpu_mm then streams it), else a status
int otpu_gemm_try(const int8_t* q, int64_t ldq, const float* Sa, const uint8_t* da, int64_t ldda, int M, int K,
                  const uint8_t* w, int64_t rs, const uint8_t* ws, int64_t srs, int N, int fmt, int flags, int k0,
                  const float* alpha, float* out, int64_t ors, hipStream_t s) {
    if (fmt != OTPU_INT8 || M < 16 || (flags & OTPU_RMAX)) return 1;
    if (((uintptr_t)da & 3) || (ldda % 4) || ((uintptr_t)q & 15) || (ldq % 16) || ((uintptr_t)w & 15) || (rs % 16))
        return 1;
    GemmArgs a = {};
    a.q = q; a.ldq = ldq; a.Sa = Sa; a.da = da; a.ldda = ldda; a.M = M; a.K = K;
    a.w = reinterpret_cast<const int8_t*>(w); a.rs = rs; a.ws = ws; a.srs = srs; a.N = N;
    a.flags = flags; a.k0 = k0; a.alpha = alpha; a.out = out; a.ors = ors;
    a.tiles_m = (M + GBM - 1) / GBM;
    a.tiles_n = (N + GBN - 1) / GBN;
    a.vec4 = ((uintptr_t)out % 16 == 0) && (ors % 4 == 0);
    // (OTPU_GENERIC_COPIES set: the generic copy for every shape, the same results; for measuring
    // what the c3 copy is worth on the same operands)
    const bool c3 = OTPU_GEMM_C3 && M == 512 && N == 8192 && K == 2048 && ldq == 2048 && rs == 2048 && ldda == 64 &&
                    srs == 4 && ors == 8192 && a.vec4 && !getenv("OTPU_GENERIC_COPIES");
    if (OTPU_GEMM_LW) {
        if (c3) gemm_lw_kernel<true><<<a.tiles_m * a.tiles_n, 512, 0, s>>>(a);
        else gemm_lw_kernel<false><<<a.tiles_m * a.tiles_n, 512, 0, s>>>(a);
    } else {
        if (c3) gemm_i8_kernel<true><<<a.tiles_m * a.tiles_n, 256, 0, s>>>(a);
        else gemm_i8_kernel<false><<<a.tiles_m * a.tiles_n, 256, 0, s>>>(a);
    }
    return otpu_launch_check("mm gemm");
}
