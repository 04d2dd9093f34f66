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
};

// byte offset of 16-byte chunk c of tile row r (rows of 128 bytes, chunks XOR-swizzled)
__device__ __forceinline__ int swz(int r, int c) { return r * GBK + ((c ^ ((r >> 1) & 7)) << 4); }

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

// a wave's 64 x 64 outputs: y = (accf * Sw[n]) * (Sa[m] * 2^-16) (accf = i2f of the exact
// integer), then ACC / ASCALE.  Values are formed first and stored in a burst with no loads in
// between (the old outputs of ACC / ASCALE are all loaded before any store), so the stores
// stream instead of waiting on each other.
__device__ __forceinline__ void tile_epilogue(const GemmArgs& a, int m0, int n0, float (&v)[4][4][4],
                                              const float (&sw)[4], const float (&sa2)[4][4]) {
    const int lane = threadIdx.x & 63, wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int mb = m0 + (wid >> 1) * 64 + 4 * (lane >> 4), nb = n0 + (wid & 1) * 64 + (lane & 15);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int t = 0; t < 4; ++t) v[i][j][t] = fmul(fmul(v[i][j][t], sw[j]), sa2[i][t]);
    const bool full = m0 + GBM <= a.M && n0 + GBN <= a.N;
    if (a.flags & (OTPU_ACC | OTPU_ASCALE)) {
        float old[4][4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int m = mb + i * 16 + t, n = nb + j * 16;
                    old[i][j][t] = (m < a.M && n < a.N) ? a.out[(int64_t)m * a.ors + n] : 0.0f;
                }
        const bool asc = (a.flags & OTPU_ASCALE) != 0;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int m = mb + i * 16 + t;
                const float al = (asc && m < a.M) ? a.alpha[m] : 1.0f;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    v[i][j][t] = asc ? fadd(fmul(old[i][j][t], al), v[i][j][t]) : fadd(old[i][j][t], v[i][j][t]);
            }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int m = mb + i * 16 + t;
            float* row = a.out + (int64_t)m * a.ors;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int n = nb + j * 16;
                if (full || (m < a.M && n < a.N)) row[n] = v[i][j][t];
            }
        }
}

// a tile's planes in ascending s (Horner in the int32 accumulators), then its epilogue
template <bool MA, bool MB>
__device__ __forceinline__ void gemm_tile(const GemmArgs& a, const Smem& sm, int m0, int n0, uint32_t dmask,
                                          uint32_t emask, uint32_t smask, int smin, int smax, const float (&sw)[4],
                                          const float (&sa2)[4][4]) {
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
            gemm_pass<MA, MB>(a, sm, acc, m0, n0, d, e);
        }
    }
    // acc = C << (16 - smax) with C an int32: i2f(acc) = rne(C) * 2^(16 - smax), exactly
    float v[4][4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int t = 0; t < 4; ++t) v[i][j][t] = ldexpf((float)acc[i][j][t], 16 - smax);
    tile_epilogue(a, m0, n0, v, sw, sa2);
}

__global__ __launch_bounds__(256) void gemm_i8_kernel(GemmArgs a) {
    __shared__ __align__(16) int8_t sA[2][GBM * GBK];
    __shared__ __align__(16) int8_t sB[2][GBN * GBK];
    __shared__ uint32_t sDa[2][GBM];       // the stage's four da bytes per activation row
    __shared__ uint8_t sDw[2][GBN];        // the stage's dw byte per weight row
    __shared__ uint32_t sMask[2];          // d values and e values present in the tile

    const int tid = threadIdx.x, lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wid >> 1, wn = wid & 1;

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

    // the offsets present in this tile: d over its activation rows, e over its weight rows.
    // Two threads a row; the loads of a thread are independent (issued back to back).
    if (tid < 2) sMask[tid] = 0;
    __syncthreads();
    {
        uint32_t dm = 0, em = 0;
        const int r = tid & (GBM - 1), h = tid >> 7;
        if (m0 + r < a.M) {
            const uint32_t* drow = reinterpret_cast<const uint32_t*>(a.da + (int64_t)(m0 + r) * a.ldda);
#pragma unroll 8
            for (int k = h; k < KT; k += 2) {                 // K / 128 words of four offsets
                const uint32_t wd = drow[k];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const uint32_t d = (wd >> (8 * t)) & 0xFF;
                    dm |= 1u << (d <= 16 ? d : 17);           // bit 17: a group beyond the window
                }
            }
        }
        if (plain) {
            em = 1u;
        } else if (n0 + r < a.N) {
            const uint8_t* wrow = a.ws + (int64_t)(n0 + r) * a.srs + 4 + a.k0;
#pragma unroll 8
            for (int k = h; k < KT; k += 2) {
                const uint32_t e = wrow[k];
                em |= 1u << (e <= 16 ? e : 17);
            }
        }
        for (int o = 32; o > 0; o >>= 1) {
            dm |= __shfl_xor(dm, o, 64);
            em |= __shfl_xor(em, o, 64);
        }
        if (lane == 0) {
            atomicOr(&sMask[0], dm);
            atomicOr(&sMask[1], em);
        }
    }
    __syncthreads();
    const uint32_t dmask = sMask[0] & 0x1FFFFu, emask = sMask[1] & 0x1FFFFu;
    // groups beyond the window exist: masking must drop them even with one live plane
    const bool over = ((sMask[0] | sMask[1]) >> 17) & 1;
    // the s = d + e values with a live plane, smin and smax
    uint32_t smask = 0;
    for (int d = 0; d <= 16; ++d)
        if (dmask >> d & 1) smask |= (emask << d) & 0x1FFFFu;

    // epilogue constants of this lane's outputs
    float sw[4], sa2[4][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int n = n0 + wn * 64 + j * 16 + (lane & 15);
        sw[j] = (unit || n >= a.N) ? 1.0f : *reinterpret_cast<const float*>(a.ws + (int64_t)n * a.srs);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int m = m0 + wm * 64 + i * 16 + 4 * (lane >> 4) + t;
            sa2[i][t] = m < a.M ? fmul(a.Sa[m], pow2f(-16)) : 0.0f;
        }

    if (smask == 0) {                               // every group drops: acc = 0
        float v[4][4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int t = 0; t < 4; ++t) v[i][j][t] = 0.0f;
        tile_epilogue(a, m0, n0, v, sw, sa2);
        return;
    }
    const int smin = __builtin_ctz(smask), smax = 31 - __builtin_clz(smask);
    // |acc| <= K * 127^2 * 2^(smax - smin) must stay below 2^31 in the int32 accumulators
    const bool fits = (int64_t)a.K * 16129 <= (((int64_t)1 << 31) - 1) >> (smax - smin);
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
    const bool single = !over && __builtin_popcount(dmask) == 1 && __builtin_popcount(emask) == 1;
    const Smem sm{sA, sB, sDa, sDw};
    if (single) gemm_tile<false, false>(a, sm, m0, n0, dmask, emask, smask, smin, smax, sw, sa2);
    else if (plain) gemm_tile<true, false>(a, sm, m0, n0, dmask, emask, smask, smin, smax, sw, sa2);
    else gemm_tile<true, true>(a, sm, m0, n0, dmask, emask, smask, smin, smax, sw, sa2);
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
    gemm_i8_kernel<<<a.tiles_m * a.tiles_n, 256, 0, s>>>(a);
    return otpu_launch_check("mm gemm");
}
