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
__device__ int64_t valu_acc(const GemmArgs& a, int j, int n, bool plain) {
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

__global__ __launch_bounds__(256) void gemm_i8_kernel(GemmArgs a) {
    __shared__ __align__(16) int8_t sA[2][GBM * GBK];
    __shared__ __align__(16) int8_t sB[2][GBN * GBK];
    __shared__ uint32_t sDa[2][GBM];       // the stage's four da bytes per activation row
    __shared__ uint8_t sDw[2][GBN];        // the stage's dw byte per weight row
    __shared__ uint32_t sMask[2];          // d values and e values present in the tile

    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
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

    // the offsets present in this tile: d over its activation rows, e over its weight rows
    if (tid < 2) sMask[tid] = 0;
    __syncthreads();
    {
        uint32_t dm = 0, em = 0;
        const int groups = a.K / 32;
        for (int idx = tid; idx < GBM * groups; idx += 256) {
            const int r = idx / groups, g = idx % groups;
            if (m0 + r < a.M) {
                const int d = a.da[(int64_t)(m0 + r) * a.ldda + g];
                dm |= 1u << (d <= 16 ? d : 17);      // bit 17: some group beyond the window
            }
        }
        if (plain) {
            em = 1u;
        } else {
            for (int idx = tid; idx < GBN * KT; idx += 256) {
                const int r = idx / KT, k = idx % KT;
                if (n0 + r < a.N) {
                    const int e = a.ws[(int64_t)(n0 + r) * a.srs + 4 + a.k0 + k];
                    em |= 1u << (e <= 16 ? e : 17);
                }
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

    auto epilogue = [&](int i, int j, int t, int64_t acc) {
        const int m = m0 + wm * 64 + i * 16 + 4 * (lane >> 4) + t;
        const int n = n0 + wn * 64 + j * 16 + (lane & 15);
        if (m < a.M && n < a.N) {
            float y = fmul(fmul(i2f(acc), sw[j]), sa2[i][t]);
            float* o = a.out + (int64_t)m * a.ors + n;
            if (a.flags & OTPU_ASCALE) y = fadd(fmul(*o, a.alpha[m]), y);
            else if (a.flags & OTPU_ACC) y = fadd(*o, y);
            *o = y;
        }
    };

    if (smask == 0) {                               // every group drops: acc = 0
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int t = 0; t < 4; ++t) epilogue(i, j, t, 0);
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

    v4i acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = v4i{0, 0, 0, 0};

    // global -> register staging of one K stage: 4 A chunks and 4 B chunks per thread
    uint4 ra[4], rb[4];
    uint32_t rda = 0;
    uint8_t rdw = 0;
    auto gload = [&](int kt) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int p = tid + 256 * u, r = p >> 3, c = p & 7;
            ra[u] = m0 + r < a.M ? *reinterpret_cast<const uint4*>(a.q + (int64_t)(m0 + r) * a.ldq + kt * GBK + 16 * c) : zero4();
            rb[u] = n0 + r < a.N ? *reinterpret_cast<const uint4*>(a.w + (int64_t)(n0 + r) * a.rs + kt * GBK + 16 * c) : zero4();
        }
        if (!single) {
            if (tid < GBM) rda = m0 + tid < a.M ? *reinterpret_cast<const uint32_t*>(a.da + (int64_t)(m0 + tid) * a.ldda + 4 * kt) : 0xFFFFFFFFu;
            else if (!plain && tid < GBM + GBN)
                rdw = n0 + tid - GBM < a.N ? a.ws[(int64_t)(n0 + tid - GBM) * a.srs + 4 + a.k0 + kt] : 0xFF;
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int p = tid + 256 * u, r = p >> 3, c = p & 7;
            *reinterpret_cast<uint4*>(&sA[buf][swz(r, c)]) = ra[u];
            *reinterpret_cast<uint4*>(&sB[buf][swz(r, c)]) = rb[u];
        }
        if (!single) {
            if (tid < GBM) sDa[buf][tid] = rda;
            else if (!plain && tid < GBM + GBN) sDw[buf][tid - GBM] = rdw;
        }
    };

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
            gload(0);
            lstore(0);
            __syncthreads();
            for (int kt = 0; kt < KT; ++kt) {
                const int cur = kt & 1;
                if (kt + 1 < KT) gload(kt + 1);
#pragma unroll
                for (int ks = 0; ks < 2; ++ks) {
                    const int c = ks * 4 + (lane >> 4);
                    v4i fa[4], fb[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int r = wm * 64 + i * 16 + (lane & 15);
                        uint4 v = *reinterpret_cast<const uint4*>(&sA[cur][swz(r, c)]);
                        if (!single && ((sDa[cur][r] >> (8 * (c >> 1))) & 0xFF) != (uint32_t)d) v = zero4();
                        fa[i] = v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
                    }
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int r = wn * 64 + j * 16 + (lane & 15);
                        uint4 v = *reinterpret_cast<const uint4*>(&sB[cur][swz(r, c)]);
                        if (!single && !plain && sDw[cur][r] != (uint8_t)e) v = zero4();
                        fb[j] = v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
                    }
#pragma unroll
                    for (int i = 0; i < 4; ++i)
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
                }
                if (kt + 1 < KT) {
                    lstore(cur ^ 1);
                }
                __syncthreads();
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int t = 0; t < 4; ++t) epilogue(i, j, t, (int64_t)acc[i][j][t] << (16 - smax));
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
