// MM for few activation rows (decode GEMV, M <= 4 per launch): the weight-streaming kernel,
// the LM head with the greedy argmax fused into its epilogue, and VOP ARGMAX.
// Semantics: opentpu/isasim.py:706-910 (MM), :1141-1152 (ARGMAX), docs/isa.md:226-305.
//
// Layout of the work.  A weight row is cut into 16-byte pieces (int8: 16 elements, half a
// 32-group; 4-bit: 32 elements, one 32-group).  A wave owns R weight rows at a time and lane l
// takes pieces l, l+64, l+128, .. of each (L = ceil(pieces/64) per lane), so every load is a
// 16-byte global_load_dwordx4 and a wave's load covers 1 KB of one row.  The activation pieces
// a lane needs are the same for every row: they are loaded once, into registers (4-bit: split
// into even / odd element bytes to meet the nibbles).  Per piece:
//   int8   c = 4 x v_dot4_i32_i8
//   int4   c = 8 x v_dot4 on (nibble << 4) bytes, then >> 4 (exact)
//   fp4    E2M1 codes through two v_perm_b32 tables and a sign select, then 8 x v_dot4
// then B = m << (W - dw - da) (0 where the shift is negative) and an int64 multiply-add.  The
// wave reduces each row's int64 partials with shuffles and R*M lanes run the fp32 epilogue
// (three FTZ products) and store.  Scale rows are read per lane piece (4 lanes share a word).
#include <cstdlib>

#include "otpu_common.h"

namespace otpu {

constexpr int LMAX = 8;            // pieces per lane held in registers (K <= 128 * LMAX * 16 / elements)

struct MMArgs {
    const int8_t* q; int64_t ldq;
    const float* Sa;
    const uint8_t* da; int64_t ldda;
    int M, K;
    const uint8_t* w; int64_t rs;
    const uint8_t* ws; int64_t srs;
    int N, flags, k0;
    const float* alpha;
    float* out; int64_t ors;
    uint32_t* rmax_key;            // RMAX: total-order keys, finished by rmax_finish
    int64_t* acc_out;              // exact accumulators instead of the epilogue
    uint64_t* best;                // LM head: max of (key << 32 | ~index)
    int64_t base;                  // LM head: index of row 0
    int P, T;                      // 16-byte pieces per row, lanes per row (team)
    // batch strides (elements of each pointer's type; bytes for w / ws; blocks for k0)
    int64_t q_bs, sa_bs, da_bs, w_bs, ws_bs, out_bs;
    int k0_bs;
};

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// a streamed 16-byte weight load, marked non-temporal (the rows are read once)
__device__ __forceinline__ uint4 ld16(const uint8_t* p) {
#if OTPU_GEMV_NT
    u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
#else
    return *reinterpret_cast<const uint4*>(p);
#endif
}

// E2M1 codes (4 per dword, one per byte, 0..15) -> signed int8 values, twice the E2M1 value
__device__ __forceinline__ uint32_t dec_e2m1(uint32_t nib) {
    uint32_t sel = nib & 0x07070707u;
    uint32_t pos = __builtin_amdgcn_perm(0x0C080604u, 0x03020100u, sel);
    uint32_t neg = __builtin_amdgcn_perm(0xF4F8FAFCu, 0xFDFEFF00u, sel);
    uint32_t msk = ((nib >> 3) & 0x01010101u) * 0xFFu;
    return (neg & msk) | (pos & ~msk);
}

// piece sums: int8 (one partial 16-group of a 32-group), 4-bit (c0: whole 32-group, or with
// nvfp4 the two 16-groups c0 and c1)
template <int FMT>
__device__ __forceinline__ void piece_dot(const uint4 wv, const uint32_t* a, int& c0, int& c1) {
    if (FMT == OTPU_INT8) {
        int c = __builtin_amdgcn_sdot4((int)wv.x, (int)a[0], 0, false);
        c = __builtin_amdgcn_sdot4((int)wv.y, (int)a[1], c, false);
        c = __builtin_amdgcn_sdot4((int)wv.z, (int)a[2], c, false);
        c0 = __builtin_amdgcn_sdot4((int)wv.w, (int)a[3], c, false);
        c1 = 0;
    } else if (FMT == OTPU_INT4) {
        const uint32_t wd[4] = {wv.x, wv.y, wv.z, wv.w};
        int c = 0;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            c = __builtin_amdgcn_sdot4((int)((wd[t] << 4) & 0xF0F0F0F0u), (int)a[2 * t], c, false);
            c = __builtin_amdgcn_sdot4((int)(wd[t] & 0xF0F0F0F0u), (int)a[2 * t + 1], c, false);
        }
        c0 = c >> 4;
        c1 = 0;
    } else {
        const uint32_t wd[4] = {wv.x, wv.y, wv.z, wv.w};
        int c[2] = {0, 0};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            uint32_t ev = dec_e2m1(wd[t] & 0x0F0F0F0Fu), od = dec_e2m1((wd[t] >> 4) & 0x0F0F0F0Fu);
            c[t >> 1] = __builtin_amdgcn_sdot4((int)ev, (int)a[2 * t], c[t >> 1], false);
            c[t >> 1] = __builtin_amdgcn_sdot4((int)od, (int)a[2 * t + 1], c[t >> 1], false);
        }
        if (FMT == OTPU_NVFP4) { c0 = c[0]; c1 = c[1]; }
        else { c0 = c[0] + c[1]; c1 = 0; }
    }
}

// the scale data a piece needs, from the scale row at byte offset ro of base sb (UNIT / RSC: none)
template <int FMT>
__device__ __forceinline__ uint32_t piece_scale(const uint8_t* sb, uint32_t ro, int k0, int p, bool plain) {
    if (plain) return 0;
    if (FMT == OTPU_INT8) return sb[ro + (uint32_t)(4 + k0 + (p >> 3))];
    if (FMT == OTPU_NVFP4)
        return *reinterpret_cast<const uint16_t*>(sb + (ro + (uint32_t)(16 + 8 * (k0 + (p >> 2)) + 2 * (p & 3))));
    return *reinterpret_cast<const uint32_t*>(sb + (ro + (uint32_t)(8 + 4 * (k0 + (p >> 2)))));
}

// B * c for the piece's group(s) as an exact double; shA = W - da of the piece's 32-group
// (activation side).  |m c| < 2^22 and the shift is at most 16, so every term and every sum
// of terms of one MM (|acc| < 2^47) is an integer a double holds exactly: the accumulation
// order cannot change a bit, and cvt_f32_f64 of the sum is i2f's RNE rounding.
template <int FMT, bool PLAIN>
__device__ __forceinline__ double piece_term(int c0, int c1, uint32_t sc, int shA, int p) {
    if (FMT == OTPU_INT8) {
        const int sh = shA - (PLAIN ? 0 : (int)sc);
        return sh >= 0 ? __builtin_ldexp((double)c0, sh) : 0.0;
    }
    if (FMT == OTPU_NVFP4) {
        double t = 0.0;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int e4 = (int)((sc >> (8 * h)) & 0xFF), E = (e4 >> 3) & 15, mt = e4 & 7;
            const int m = PLAIN ? 1 : (E ? 8 + mt : mt);
            const int sh = shA - (PLAIN ? 0 : 15 - (E > 1 ? E : 1));
            const int mm = sh >= 0 ? m : 0;
            t += __builtin_ldexp((double)__mul24(mm, h ? c1 : c0), sh);
        }
        return t;
    }
    const int m = PLAIN ? 1 : (int)((sc >> (8 + 6 * (p & 3))) & 63);
    const int sh = shA - (PLAIN ? 0 : (int)(sc & 0xFF));
    const int mm = sh >= 0 ? m : 0;
    return __builtin_ldexp((double)__mul24(mm, c0), sh);
}

// ---- cross-lane exchanges of doubles (64-wide waves) ----
__device__ __forceinline__ uint2 dbits(double x) { return make_uint2(__double2loint(x), __double2hiint(x)); }
__device__ __forceinline__ double dfrom(uint32_t lo, uint32_t hi) { return __hiloint2double((int)hi, (int)lo); }

// lanes 0..31 keep a, lanes 32..63 keep b; both halves receive the other half's kept operand
// and return the sum (v_permlane32_swap exchanges a's upper half with b's lower half)
__device__ __forceinline__ double swap_add32(double a, double b) {
    const uint2 x = dbits(a), y = dbits(b);
    const auto lo = __builtin_amdgcn_permlane32_swap(x.x, y.x, false, false);
    const auto hi = __builtin_amdgcn_permlane32_swap(x.y, y.y, false, false);
    return dfrom(lo[0], hi[0]) + dfrom(lo[1], hi[1]);
}

// the same for lane bit 4 (rows of 16: v_permlane16_swap exchanges a's odd rows with b's even)
__device__ __forceinline__ double swap_add16(double a, double b) {
    const uint2 x = dbits(a), y = dbits(b);
    const auto lo = __builtin_amdgcn_permlane16_swap(x.x, y.x, false, false);
    const auto hi = __builtin_amdgcn_permlane16_swap(x.y, y.y, false, false);
    return dfrom(lo[0], hi[0]) + dfrom(lo[1], hi[1]);
}

// x from the partner lane across lane bit o (o <= 8) by DPP: row_ror:8 (bit 3),
// row_half_mirror (lane i <-> 7 - i: crosses bit 2), quad_perm (bits 1, 0)
template <int O>
__device__ __forceinline__ double dpp_partner(double x) {
    constexpr int CTRL = O == 8 ? 0x128 : O == 4 ? 0x141 : O == 2 ? 0x4E : 0xB1;
    const uint2 u = dbits(x);
    return dfrom((uint32_t)__builtin_amdgcn_update_dpp(0, (int)u.x, CTRL, 0xF, 0xF, false),
                 (uint32_t)__builtin_amdgcn_update_dpp(0, (int)u.y, CTRL, 0xF, 0xF, false));
}

// one reduce-scatter step across lane bit o: lanes with the bit clear return a + partner's a,
// lanes with it set b + partner's b
__device__ __forceinline__ double xchg_add(double a, double b, int o, int lane) {
    if (o == 32) return swap_add32(a, b);
    if (o == 16) return swap_add16(a, b);
    const bool up = (lane & o) != 0;
    const double keep = up ? b : a, give = up ? a : b;
    const double recv = o == 8 ? dpp_partner<8>(give) : o == 4 ? dpp_partner<4>(give)
                      : o == 2 ? dpp_partner<2>(give) : dpp_partner<1>(give);
    return keep + recv;
}

// x + the partner's x across lane bit o (a plain reduction step: every lane gets the sum)
__device__ __forceinline__ double xsum(double x, int o) {
    if (o == 32) return swap_add32(x, x);
    if (o == 16) return swap_add16(x, x);
    return x + (o == 8 ? dpp_partner<8>(x) : o == 4 ? dpp_partner<4>(x) : o == 2 ? dpp_partner<2>(x) : dpp_partner<1>(x));
}

// rows a team takes per iteration: with one piece a lane, 16 rows' loads in flight per wave for
// one activation row (measured best on MI355X: 8 gave 3% less, 32 no more), fewer as activation
// rows add sums to carry (R * MR stays 16)
#ifndef OTPU_GEMV_R1
#define OTPU_GEMV_R1 16
#endif
#ifndef OTPU_GEMV_NT
#define OTPU_GEMV_NT 1
#endif
#ifndef OTPU_GEMV_R2
#define OTPU_GEMV_R2 2
#endif
#ifndef OTPU_GEMV_R4
#define OTPU_GEMV_R4 2
#endif
constexpr int rows_per_team_rt(int L, int mr) {
    return L >= 4 ? OTPU_GEMV_R4 : (L == 1 ? OTPU_GEMV_R1 / mr : OTPU_GEMV_R2);
}
template <int L, int MR>
constexpr int rows_per_team() { return rows_per_team_rt(L, MR); }

// activation registers a lane holds: MR rows x L pieces x (4 int8 | 8 split 4-bit) dwords
// ... and the reduce-scatter needs the R * MR sums of an iteration to fit a team of 16 lanes
constexpr bool fits_rt(int fmt, int mr, int L) {
    return mr * L * (fmt == OTPU_INT8 ? 4 : 8) <= 64 && rows_per_team_rt(L, mr) * mr <= 16;
}
template <int FMT, int MR, int L>
constexpr bool fits() { return fits_rt(FMT, MR, L); }

// the kernel body for a team of T lanes (T a compile-time constant: the exchanges of the
// reduction are then straight-line code)
template <int FMT, int MR, int L, int T, bool PLAIN>
__device__ __forceinline__ void gemv_body(const MMArgs& a) {
    constexpr int AW = FMT == OTPU_INT8 ? 4 : 8;          // activation dwords per piece
    constexpr int R = rows_per_team<L, MR>();
    constexpr int E = R * MR;                             // sums a lane carries per iteration
    static_assert(E <= T, "a team holds its E sums after the reduce-scatter");
    const int lane = threadIdx.x & 63;
    constexpr int NT = 64 / T;                            // teams per wave
    const int tl = lane & (T - 1), team = lane / T;
    const int b = blockIdx.y;                             // batch problem
    const int8_t* q = a.q + b * a.q_bs;
    const float* Sa = a.Sa ? a.Sa + b * a.sa_bs : nullptr;
    const uint8_t* da = a.da + b * a.da_bs;
    const uint8_t* w = a.w + b * a.w_bs;
    const uint8_t* ws = a.ws + b * a.ws_bs;
    float* out = a.out ? a.out + b * a.out_bs : nullptr;
    const int k0 = a.k0 + b * a.k0_bs;
    constexpr bool plain = PLAIN;
    const bool unit = (a.flags & OTPU_UNIT) != 0;
    const int W = window_of(FMT);
    const int P = a.P;

    // activation pieces tl, tl + T, .. and their W - da, per act row, in registers
    uint32_t act[MR][L][AW];
    int shA[MR][L];
#pragma unroll
    for (int j = 0; j < MR; ++j) {
#pragma unroll
        for (int i = 0; i < L; ++i) {
            const int p = i * T + tl;
            const bool ok = p < P && j < a.M;
            if (FMT == OTPU_INT8) {
                uint4 v = ok ? *reinterpret_cast<const uint4*>(q + j * a.ldq + 16 * p) : make_uint4(0, 0, 0, 0);
                act[j][i][0] = v.x; act[j][i][1] = v.y; act[j][i][2] = v.z; act[j][i][3] = v.w;
                shA[j][i] = W - (ok ? (int)da[j * a.ldda + (p >> 1)] : 0);
            } else {
                uint4 v0 = make_uint4(0, 0, 0, 0), v1 = v0;
                if (ok) {
                    v0 = *reinterpret_cast<const uint4*>(q + j * a.ldq + 32 * p);
                    v1 = *reinterpret_cast<const uint4*>(q + j * a.ldq + 32 * p + 16);
                }
                const uint32_t d[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    act[j][i][2 * t] = __builtin_amdgcn_perm(d[2 * t + 1], d[2 * t], 0x06040200u);
                    act[j][i][2 * t + 1] = __builtin_amdgcn_perm(d[2 * t + 1], d[2 * t], 0x07050301u);
                }
                shA[j][i] = W - (ok ? (int)da[j * a.ldda + p] : 0);
            }
        }
    }
    float sa2[MR];
#pragma unroll
    for (int j = 0; j < MR; ++j) sa2[j] = (j < a.M && !a.acc_out) ? fmul(Sa[j], pow2f(-W)) : 0.0f;

    // wave-uniform by construction; readfirstlane tells the compiler (scalar loop, no exec masks)
    const int wave = __builtin_amdgcn_readfirstlane((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const int nwaves = (gridDim.x * blockDim.x) >> 6;
    const int RW = R * NT;                      // rows a wave takes per iteration
    const int stride = nwaves * RW;
    uint64_t best = 0;
    // After the reduce-scatter below, value e = r * MR + j of a team sits in the lanes
    // tl = e * (T / E) .. (e + 1) * (T / E) - 1; the first of them runs its epilogue.
    const int span = T / E;
    const int ee = tl / span;
    const int er = ee / MR, ej = ee % MR;
    const bool epilane = (tl % span) == 0;

    // one iteration's operands: weight pieces, their scale data, the epilogue row's Sw
    struct Stage {
        uint4 wv[R][L];
        uint32_t sc[R][L];
        float sw;
    };
    // operand addresses: a wave-uniform row-group base (scalar registers) plus 32-bit lane
    // offsets, so the loads take the saddr + voffset form; rows past N read the last row and
    // pieces past P the last piece (no branch around a load): the former reach no epilogue, the
    // latter meet zero activation registers
    auto load = [&](Stage& st, int n0) {
        const uint8_t* wb = w + (int64_t)n0 * a.rs;
        const uint8_t* sb = ws + (int64_t)n0 * a.srs;
        const int last = a.N - 1 - n0;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int dn = min(r * NT + team, last);
            const uint32_t roff = (uint32_t)dn * (uint32_t)a.rs;
            const uint32_t soff = (uint32_t)dn * (uint32_t)a.srs;
#pragma unroll
            for (int i = 0; i < L; ++i) {
                const int p = i * T + tl;
                const int pc = p < P ? p : P - 1;
                st.wv[r][i] = ld16(wb + (roff + 16u * (uint32_t)pc));
                st.sc[r][i] = piece_scale<FMT>(sb, soff, k0, pc, plain);
            }
        }
        st.sw = unit ? 1.0f : ftz(*reinterpret_cast<const float*>(sb + (uint32_t)min(er * NT + team, last) * (uint32_t)a.srs));
    };
    auto compute = [&](const Stage& st, int n0) {
        double v[E];
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int j = 0; j < MR; ++j) {
                double acc = 0.0;
#pragma unroll
                for (int i = 0; i < L; ++i) {
                    int c0, c1;
                    piece_dot<FMT>(st.wv[r][i], act[j][i], c0, c1);
                    acc += piece_term<FMT, PLAIN>(c0, c1, st.sc[r][i], shA[j][i], i * T + tl);
                }
                v[r * MR + j] = acc;
            }
        }
        // reduce-scatter over the team: each step halves the values a lane carries (E - 1
        // exchanges in all: permlane swaps across lane bits 5 and 4, DPP below), then plain
        // steps finish the sums over the team's T lanes
        int o = T >> 1;
#pragma unroll
        for (int h = E / 2; h >= 1; h >>= 1, o >>= 1) {
#pragma unroll
            for (int i = 0; i < h; ++i) v[i] = xchg_add(v[i], v[i + h], o, lane);
        }
        double tot = v[0];
#pragma unroll
        for (; o > 0; o >>= 1) tot = xsum(tot, o);
        const int n = n0 + er * NT + team;
        if (epilane && n < a.N && ej < a.M) {
            if (a.acc_out) {
                a.acc_out[(int64_t)ej * a.N + n] = (int64_t)tot;
            } else {
                // fmul(fmul(i2f(acc), Sw), Sa * 2^-W): the float of an integer, the flushed Sw
                // and the finished Sa * 2^-W need no operand flush
                float y = fmul_f(fmul_f((float)tot, st.sw), sa2[ej]);
                if (out) {
                    float* op = out + (int64_t)ej * a.ors + n;
                    if (a.flags & OTPU_ASCALE) y = fadd(fmul(*op, a.alpha[ej]), y);
                    else if (a.flags & OTPU_ACC) y = fadd(*op, y);
                    *op = y;
                }
                if (a.flags & OTPU_RMAX) atomicMax(a.rmax_key + ej, fkey_f(y));
                if (a.best) {
                    uint64_t cand = ((uint64_t)fkey_f(y) << 32) | (uint32_t)~(uint32_t)(a.base + n);
                    best = cand > best ? cand : best;
                }
            }
        }
    };

    // one stage per wave: the loads of an iteration go out together and the waves of the SIMD
    // (5-8 resident) overlap each other's memory latency; a second register stage per wave
    // costs occupancy and measured slower on MI355X
    for (int n0 = wave * RW; n0 < a.N; n0 += stride) {
        Stage st;
        load(st, n0);
        compute(st, n0);
    }
    if (a.best) {                               // one atomic per workgroup
        __shared__ uint64_t red[4];
        best = wave_max_u64(best);
        if (lane == 0) red[threadIdx.x >> 6] = best;
        __syncthreads();
        if (threadIdx.x == 0) {
            uint64_t m = red[0];
            for (int i = 1; i < (int)(blockDim.x >> 6); ++i) m = red[i] > m ? red[i] : m;
            if (m) atomicMax(reinterpret_cast<unsigned long long*>(a.best), (unsigned long long)m);
        }
    }
}

template <int FMT, int MR, int L, bool PLAIN>
__global__ __launch_bounds__(256) void gemv_kernel(MMArgs a) {
    if (a.T == 64) gemv_body<FMT, MR, L, 64, PLAIN>(a);
    else if (a.T == 32) gemv_body<FMT, MR, L, 32, PLAIN>(a);
    else gemv_body<FMT, MR, L, 16, PLAIN>(a);
}

// a fill kernel (graph-capture friendly, no memset nodes)
__global__ void fill_u32(uint32_t* p, int n, uint32_t v) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

__global__ void rmax_finish(uint32_t* k, int n) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) k[i] = fbits(unkey(k[i]));
}

// the ACC chain of R partial MM outputs: out = add(..add(add(old | part_0, part_1)..), part_R-1)
__global__ void sum_parts(const float* __restrict__ part, int64_t pstride, int R, int M, int N, int acc,
                          float* __restrict__ out, int64_t ors) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)M * N) return;
    const int j = (int)(i / N), n = (int)(i % N);
    const float* p = part + (int64_t)j * N + n;
    float* o = out + (int64_t)j * ors + n;
    float y = acc ? fadd(*o, p[0]) : p[0];
    for (int r = 1; r < R; ++r) y = fadd(y, p[r * pstride]);
    *o = y;
}

__global__ void best_finish(const uint64_t* best, int32_t* token) {
    if (threadIdx.x == 0) *token = (int32_t)~(uint32_t)(*best & 0xFFFFFFFFull);
}

// VOP ARGMAX: one workgroup per row; (max, i2f(index + base))
__global__ __launch_bounds__(256) void argmax_rows(const float* __restrict__ x, int cols, int64_t ldx,
                                                    int64_t base, float* pairs, int64_t drs) {
    __shared__ uint64_t red[4];
    const float* xr = x + (int64_t)blockIdx.x * ldx;
    uint64_t best = 0;
    for (int c = threadIdx.x; c < cols; c += 256) {
        uint64_t cand = ((uint64_t)fkey(xr[c]) << 32) | (uint32_t)~(uint32_t)c;
        best = cand > best ? cand : best;
    }
    best = wave_max_u64(best);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t b = red[0];
        for (int i = 1; i < 4; ++i) b = red[i] > b ? red[i] : b;
        const uint32_t idx = ~(uint32_t)(b & 0xFFFFFFFFu);
        float* o = pairs + (int64_t)blockIdx.x * drs;
        o[0] = unkey((uint32_t)(b >> 32));
        o[1] = i2f((int64_t)(int32_t)(uint32_t)((int64_t)idx + base));
    }
}

}  // namespace otpu

using namespace otpu;

static bool al(const void* p, int a) { return ((uintptr_t)p & (uintptr_t)(a - 1)) == 0; }

// the SimError-style checks of one MM (opentpu/isasim.py:767-822, the fields of isa.py:502-548)
static int check_mm(const char* who, const int8_t* q, int64_t ldq, const uint8_t* da, int64_t ldda,
                    int M, int K, const uint8_t* w, int64_t rs, const uint8_t* ws, int64_t srs,
                    int N, int fmt, int flags, int k0) {
    if (fmt < OTPU_INT8 || fmt > OTPU_NVFP4) return otpu_fail(OTPU_EFORMAT, "%s: weight format %d", who, fmt);
    if (M < 1 || N < 1 || K < OTPU_D || K % OTPU_D || k0 < 0)
        return otpu_fail(OTPU_EINVAL, "%s: M %d, N %d, K %d (a multiple of %d), k0 %d", who, M, N, K, OTPU_D, k0);
    if ((flags & OTPU_RSC) && fmt == OTPU_NVFP4) return otpu_fail(OTPU_EFORMAT, "%s: RSC does not take NVFP4", who);
    if ((flags & OTPU_ASCALE) && !((flags & OTPU_UNIT) && (flags & OTPU_ACC)))
        return otpu_fail(OTPU_EINVAL, "%s: ASCALE needs UNIT and ACC", who);
    if (flags & ~(OTPU_UNIT | OTPU_ACC | OTPU_RMAX | OTPU_ASCALE | OTPU_PAIR | OTPU_RSC))
        return otpu_fail(OTPU_EINVAL, "%s: unknown flags %#x", who, flags);
    const int KB = K / OTPU_D;
    const int64_t rowb = fmt == OTPU_INT8 ? K : K / 2;
    if (!q || !da || !w) return otpu_fail(OTPU_EINVAL, "%s: a NULL operand", who);
    if (ldq < K || ldda < K / 32 || rs < rowb)
        return otpu_fail(OTPU_EINVAL, "%s: ldq %lld, ldda %lld, rs %lld too small", who, (long long)ldq,
                         (long long)ldda, (long long)rs);
    if (!(flags & OTPU_UNIT)) {
        if (!ws) return otpu_fail(OTPU_EINVAL, "%s: NULL scale rows", who);
        int64_t need = 4;
        if (!(flags & OTPU_RSC))
            need = fmt == OTPU_INT8 ? 4 + k0 + KB : fmt == OTPU_NVFP4 ? 16 + 8 * (k0 + KB) : 8 + 4 * (k0 + KB);
        const int sal = fmt == OTPU_NVFP4 ? 16 : (fmt == OTPU_INT8 || (flags & OTPU_RSC)) ? 4 : 8;
        if (srs < need) return otpu_fail(OTPU_EINVAL, "%s: scale rows of %lld bytes, blocks k0 %d + %d need %lld",
                                         who, (long long)srs, k0, KB, (long long)need);
        if (!al(ws, 4) || srs % sal)
            return otpu_fail(OTPU_EALIGN, "%s: ssa and srs must be multiples of %d", who, sal);
    }
    if (!al(w, 16) || rs % 16 || !al(q, 16) || ldq % 16)
        return otpu_fail(OTPU_EALIGN, "%s: weight rows and activations 16-byte aligned (w, rs, q, ldq)", who);
    if (rs >= (1 << 24) || srs >= (1 << 24))
        return otpu_fail(OTPU_EINVAL, "%s: row strides of 16 MiB or more", who);
    if ((rowb / 16 + 63) / 64 > LMAX)
        return otpu_fail(OTPU_EINVAL, "%s: K %d exceeds the register-resident operand (%d 16-byte pieces a lane)",
                         who, K, LMAX);
    return OTPU_OK;
}

// resident workgroups per CU the streaming grid aims for: 16 for one piece a lane (short rows,
// more waves), else 8 (measured on MI355X); OTPU_GEMV_BLOCKS_PER_CU overrides
static int gemv_blocks_per_cu(int L) {
    static int v = -1;
    if (v < 0) {
        const char* e = getenv("OTPU_GEMV_BLOCKS_PER_CU");
        int x = e ? atoi(e) : 0;
        v = (x > 0 && x <= 64) ? x : 0;
    }
    return v ? v : (L == 1 ? 16 : 8);
}

template <int FMT, int MR, int L>
static void launch_one(const MMArgs& a, int batch, hipStream_t s) {
    static_assert(fits<FMT, 1, L>(), "one activation row always fits");
    if constexpr (fits<FMT, MR, L>()) {
        constexpr int R = rows_per_team<L, MR>();
        const int64_t waves = (a.N + (int64_t)R * (64 / a.T) - 1) / ((int64_t)R * (64 / a.T));
        // about 8 resident workgroups per CU over the whole batch; each wave then streams
        // many row groups (its activation registers are loaded once)
        int64_t blocks = (waves + 3) / 4;
        int64_t cap = (int64_t)otpu_cu_count() * gemv_blocks_per_cu(L) / batch;
        if (cap < 1) cap = 1;
        if (blocks > cap) blocks = cap;
        if (a.flags & (OTPU_UNIT | OTPU_RSC))
            gemv_kernel<FMT, MR, L, true><<<dim3((unsigned)blocks, batch), dim3(256), 0, s>>>(a);
        else
            gemv_kernel<FMT, MR, L, false><<<dim3((unsigned)blocks, batch), dim3(256), 0, s>>>(a);
    }
}

template <int FMT, int MR>
static void launch_L(const MMArgs& a, int L, int batch, hipStream_t s) {
    switch (L) {
        case 1: launch_one<FMT, MR, 1>(a, batch, s); break;
        case 2: launch_one<FMT, MR, 2>(a, batch, s); break;
        case 3: launch_one<FMT, MR, 3>(a, batch, s); break;
        case 4: launch_one<FMT, MR, 4>(a, batch, s); break;
        case 5: launch_one<FMT, MR, 5>(a, batch, s); break;
        case 6: launch_one<FMT, MR, 6>(a, batch, s); break;
        default: launch_one<FMT, MR, 8>(a, batch, s); break;
    }
}

template <int FMT>
static void launch_fmt(const MMArgs& a, int mr, int L, int batch, hipStream_t s) {
    if (mr == 1) launch_L<FMT, 1>(a, L, batch, s);
    else if (mr == 2) launch_L<FMT, 2>(a, L, batch, s);
    else launch_L<FMT, 4>(a, L, batch, s);
}

// lanes per row: the team size in {64, 32, 16} that wastes the fewest lane pieces
static void pick_team(int P, int* T, int* L) {
    int bt = 64, bl = (P + 63) / 64, bw = bl * 64 - P;
    for (int t = 32; t >= 16; t >>= 1) {
        int l = (P + t - 1) / t, w = l * t - P;
        if (l <= LMAX && w < bw) { bt = t; bl = l; bw = w; }
    }
    if (bl == 7) bl = 8;                        // (no L = 7 instantiation: the eighth is masked)
    *T = bt;
    *L = bl;
}

static int mr_max(int fmt, int L) {
    return fits_rt(fmt, 4, L) ? 4 : (fits_rt(fmt, 2, L) ? 2 : 1);
}

static int launch_gemv(MMArgs a, int fmt, int batch, hipStream_t s) {
    const int64_t rowb = fmt == OTPU_INT8 ? a.K : a.K / 2;
    a.P = (int)(rowb / 16);
    int L = 1;
    pick_team(a.P, &a.T, &L);
    const int M = a.M, cap = mr_max(fmt, L);
    for (int j0 = 0; j0 < M; j0 += cap) {        // activation rows in chunks the registers hold
        MMArgs c = a;
        c.M = M - j0 < cap ? M - j0 : cap;
        const int mr = c.M == 1 ? 1 : (c.M == 2 ? 2 : 4);
        c.q = a.q + j0 * a.ldq;
        if (a.Sa) c.Sa = a.Sa + j0;
        c.da = a.da + j0 * a.ldda;
        if (c.out) c.out = a.out + j0 * a.ors;
        if (c.alpha) c.alpha = a.alpha + j0;
        if (c.rmax_key) c.rmax_key = a.rmax_key + j0;
        if (c.acc_out) c.acc_out = a.acc_out + (int64_t)j0 * a.N;
        switch (fmt) {
            case OTPU_INT8: launch_fmt<OTPU_INT8>(c, mr, L, batch, s); break;
            case OTPU_INT4: launch_fmt<OTPU_INT4>(c, mr, L, batch, s); break;
            case OTPU_FP4: launch_fmt<OTPU_FP4>(c, mr, L, batch, s); break;
            default: launch_fmt<OTPU_NVFP4>(c, mr, L, batch, s); break;
        }
    }
    return otpu_launch_check("mm");
}

static MMArgs make_args(const int8_t* q, int64_t ldq, const float* Sa, const uint8_t* da, int64_t ldda, int M,
                        int K, const uint8_t* w, int64_t rs, const uint8_t* ws, int64_t srs, int N, int flags,
                        int k0) {
    MMArgs a = {};
    a.q = q; a.ldq = ldq; a.Sa = Sa; a.da = da; a.ldda = ldda; a.M = M; a.K = K;
    a.w = w; a.rs = rs; a.ws = ws; a.srs = srs; a.N = N; a.flags = flags & ~OTPU_PAIR; a.k0 = k0;
    return a;
}

int otpu_gemm_try(const int8_t* q, int64_t ldq, const float* Sa, const uint8_t* da, int64_t ldda, int M, int K,
                  const uint8_t* w, int64_t rs, const uint8_t* ws, int64_t srs, int N, int fmt, int flags, int k0,
                  const float* alpha, float* out, int64_t ors, hipStream_t s);

extern "C" int otpu_mm(const int8_t* q, int64_t ldq, const float* Sa, const uint8_t* da, int64_t ldda,
                       int M, int K, const uint8_t* w, int64_t rs, const uint8_t* ws, int64_t srs, int N,
                       int fmt, int flags, int k0, const float* alpha, float* out, int64_t ors,
                       float* rowmax, otpu_stream_t stream) {
    int rc = check_mm("mm", q, ldq, da, ldda, M, K, w, rs, ws, srs, N, fmt, flags, k0);
    if (rc) return rc;
    if (!Sa || !out || ors < N) return otpu_fail(OTPU_EINVAL, "mm: Sa / out NULL or ors < N");
    if ((flags & OTPU_ASCALE) && !alpha) return otpu_fail(OTPU_EINVAL, "mm: ASCALE without alpha");
    if ((flags & OTPU_RMAX) && !rowmax) return otpu_fail(OTPU_EINVAL, "mm: RMAX without rowmax");
    hipStream_t s = (hipStream_t)stream;
    if (M > 4) {
        rc = otpu_gemm_try(q, ldq, Sa, da, ldda, M, K, w, rs, ws, srs, N, fmt, flags & ~OTPU_PAIR, k0, alpha,
                           out, ors, s);
        if (rc <= 0) return rc;                       // handled (or failed); > 0: not this path
    }
    MMArgs a = make_args(q, ldq, Sa, da, ldda, M, K, w, rs, ws, srs, N, flags, k0);
    a.alpha = alpha; a.out = out; a.ors = ors;
    if (flags & OTPU_RMAX) {
        a.rmax_key = reinterpret_cast<uint32_t*>(rowmax);
        fill_u32<<<(M + 255) / 256, 256, 0, s>>>(a.rmax_key, M, 0u);
    }
    rc = launch_gemv(a, fmt, 1, s);
    if (rc) return rc;
    if (flags & OTPU_RMAX) {
        rmax_finish<<<(M + 255) / 256, 256, 0, s>>>(a.rmax_key, M);
        return otpu_launch_check("mm rmax");
    }
    return OTPU_OK;
}

extern "C" int otpu_mm_acc(const int8_t* q, int64_t ldq, const uint8_t* da, int64_t ldda, int M, int K,
                           const uint8_t* w, int64_t rs, const uint8_t* ws, int64_t srs, int N, int fmt,
                           int flags, int k0, int64_t* acc, otpu_stream_t stream) {
    int rc = check_mm("mm_acc", q, ldq, da, ldda, M, K, w, rs, ws, srs, N, fmt,
                      flags & ~(OTPU_ACC | OTPU_ASCALE | OTPU_RMAX), k0);
    if (rc) return rc;
    if (!acc) return otpu_fail(OTPU_EINVAL, "mm_acc: NULL acc");
    MMArgs a = make_args(q, ldq, nullptr, da, ldda, M, K, w, rs, ws, srs, N,
                         flags & ~(OTPU_ACC | OTPU_ASCALE | OTPU_RMAX), k0);
    a.acc_out = acc;
    return launch_gemv(a, fmt, 1, (hipStream_t)stream);
}

extern "C" int otpu_mm_batched(int B, const int8_t* q, int64_t ldq, int64_t q_bstride, const float* Sa,
                               int64_t sa_bstride, const uint8_t* da, int64_t ldda, int64_t da_bstride, int M,
                               int K, const uint8_t* w, int64_t rs, int64_t w_bstride, const uint8_t* ws,
                               int64_t srs, int64_t ws_bstride, int N, int fmt, int flags, int k0, float* out,
                               int64_t ors, int64_t out_bstride, otpu_stream_t stream) {
    if (B < 1 || B > 65535) return otpu_fail(OTPU_EINVAL, "mm_batched: B %d", B);
    if (flags & (OTPU_ACC | OTPU_ASCALE | OTPU_RMAX))
        return otpu_fail(OTPU_EINVAL, "mm_batched: no ACC, ASCALE or RMAX");
    int rc = check_mm("mm_batched", q, ldq, da, ldda, M, K, w, rs, ws, srs, N, fmt, flags, k0);
    if (rc) return rc;
    if (!Sa || !out || ors < N) return otpu_fail(OTPU_EINVAL, "mm_batched: Sa / out NULL or ors < N");
    if (q_bstride % 16 || w_bstride % 16 || (!(flags & OTPU_UNIT) && ws_bstride % 4))
        return otpu_fail(OTPU_EALIGN, "mm_batched: batch strides keep the operands aligned");
    MMArgs a = make_args(q, ldq, Sa, da, ldda, M, K, w, rs, ws, srs, N, flags, k0);
    a.out = out; a.ors = ors;
    a.q_bs = q_bstride; a.sa_bs = sa_bstride; a.da_bs = da_bstride;
    a.w_bs = w_bstride; a.ws_bs = ws_bstride; a.out_bs = out_bstride;
    return launch_gemv(a, fmt, B, (hipStream_t)stream);
}

extern "C" int otpu_mm_ranges(const int8_t* q, int64_t ldq, const float* Sa, const uint8_t* da, int64_t ldda,
                              int M, int K, int width, const uint8_t* w, int64_t rs, const uint8_t* ws, int64_t srs,
                              int N, int fmt, int flags, int k0, float* part, float* out, int64_t ors,
                              otpu_stream_t stream) {
    const int chunk = fmt == OTPU_INT8 ? OTPU_D : 2 * OTPU_D;
    if (width < chunk || width % chunk || K % width)
        return otpu_fail(OTPU_EINVAL, "mm_ranges: ranges of %d over K %d (multiples of %d for this format)", width,
                         K, chunk);
    if (flags & (OTPU_ASCALE | OTPU_RMAX)) return otpu_fail(OTPU_EINVAL, "mm_ranges: no ASCALE or RMAX");
    const int R = K / width;
    const bool plain = (flags & (OTPU_UNIT | OTPU_RSC)) != 0;
    int rc = check_mm("mm_ranges", q, ldq, da, ldda, M, width, w, rs, ws, srs, N, fmt, flags & ~OTPU_ACC,
                      plain ? k0 : k0 + (K - width) / OTPU_D);
    if (rc) return rc;
    if (ldq < K || ldda < K / 32 || rs < (fmt == OTPU_INT8 ? K : K / 2))
        return otpu_fail(OTPU_EINVAL, "mm_ranges: ldq %lld, ldda %lld, rs %lld short of K %d", (long long)ldq,
                         (long long)ldda, (long long)rs, K);
    if (!Sa || !part || !out || ors < N) return otpu_fail(OTPU_EINVAL, "mm_ranges: Sa / part / out NULL or ors < N");
    if (!al(part, 4)) return otpu_fail(OTPU_EALIGN, "mm_ranges: part");
    hipStream_t s = (hipStream_t)stream;
    MMArgs a = make_args(q, ldq, Sa, da, ldda, M, width, w, rs, ws, srs, N, flags & ~OTPU_ACC, k0);
    a.out = part; a.ors = N;
    a.q_bs = width; a.sa_bs = M; a.da_bs = width / 32;
    a.w_bs = fmt == OTPU_INT8 ? width : width / 2; a.ws_bs = 0; a.out_bs = (int64_t)M * N;
    a.k0_bs = plain ? 0 : width / OTPU_D;
    rc = launch_gemv(a, fmt, R, s);
    if (rc) return rc;
    const int64_t tot = (int64_t)M * N;
    sum_parts<<<(unsigned)((tot + 255) / 256), 256, 0, s>>>(part, (int64_t)M * N, R, M, N, (flags & OTPU_ACC) != 0,
                                                            out, ors);
    return otpu_launch_check("mm_ranges");
}

extern "C" int otpu_lm_head_argmax(const int8_t* q, const float* Sa, const uint8_t* da, int K, const uint8_t* w,
                                   int64_t rs, const uint8_t* ws, int64_t srs, int N, int fmt, int flags, int k0,
                                   int64_t base, float* logits, uint64_t* best, int32_t* token,
                                   otpu_stream_t stream) {
    if (flags & (OTPU_ACC | OTPU_ASCALE | OTPU_RMAX))
        return otpu_fail(OTPU_EINVAL, "lm_head_argmax: no ACC, ASCALE or RMAX");
    int rc = check_mm("lm_head_argmax", q, K, da, K / 32, 1, K, w, rs, ws, srs, N, fmt, flags, k0);
    if (rc) return rc;
    if (!Sa || !best || !token) return otpu_fail(OTPU_EINVAL, "lm_head_argmax: NULL Sa, best or token");
    if (base < 0 || base + (int64_t)N > 0xFFFFFFFFll) return otpu_fail(OTPU_EINVAL, "lm_head_argmax: base %lld", (long long)base);
    if (!al(best, 8)) return otpu_fail(OTPU_EALIGN, "lm_head_argmax: best 8-byte aligned");
    hipStream_t s = (hipStream_t)stream;
    MMArgs a = make_args(q, K, Sa, da, K / 32, 1, K, w, rs, ws, srs, N, flags, k0);
    a.out = logits; a.ors = N; a.best = best; a.base = base;
    fill_u32<<<1, 64, 0, s>>>(reinterpret_cast<uint32_t*>(best), 2, 0u);
    rc = launch_gemv(a, fmt, 1, s);
    if (rc) return rc;
    best_finish<<<1, 64, 0, s>>>(best, token);
    return otpu_launch_check("lm_head_argmax");
}

extern "C" int otpu_argmax(const float* x, int rows, int cols, int64_t ldx, int64_t base, float* pairs,
                           int64_t drs, otpu_stream_t stream) {
    if (rows < 1 || cols < 1 || ldx < cols || !x || !pairs || (rows > 1 && drs < 2))
        return otpu_fail(OTPU_EINVAL, "argmax: rows %d, cols %d, ldx %lld, drs %lld", rows, cols,
                         (long long)ldx, (long long)drs);
    argmax_rows<<<rows, 256, 0, (hipStream_t)stream>>>(x, cols, ldx, base, pairs, drs);
    return otpu_launch_check("argmax");
}
