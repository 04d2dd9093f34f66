// The decode GEMV kernel (MM for few activation rows, M <= 4 per launch), the LM head's variant
// with the greedy argmax fused into its epilogue, and the variant that quantizes its activation
// row in the prologue.  Semantics: opentpu/isasim.py:706-910 (MM), docs/isa.md:226-305.
//
// Layout of the work.  A weight row is cut into 16-byte pieces (int8: 16 elements, half a
// 32-group; 4-bit: 32 elements, one 32-group).  A team of T lanes (16, 32 or 64) owns a row, lane
// tl taking pieces tl, tl + T, .. (L a lane), so every load is a 16-byte global_load_dwordx4;
// a wave streams R rows per team per iteration (16 rows a wave for one activation row).  The
// activation pieces a lane needs are the same for every row: they are loaded once, into
// registers (4-bit: split into even / odd element bytes to meet the nibbles).  Per piece:
//   int8   c = 4 x v_dot4_i32_i8
//   int4   c = 8 x v_dot4 on (nibble << 4) bytes, then >> 4 (exact)
//   fp4    E2M1 codes through two v_perm_b32 tables and a sign select, then 8 x v_dot4
// then the term (m c) 2^(W - dw - da) (0 where the shift is negative) as an exact double.  A
// team reduce-scatters its rows' sums (v_permlane32/16_swap across lane bits 5 and 4, DPP
// below), and the lanes that end with a row's sum run the fp32 epilogue (cvt of the exact sum,
// then the FTZ products) and store.  Scale rows are read per lane piece (4 lanes share a word).
#pragma once
#include <cstdlib>

#include "gemv_args.h"

namespace otpu {

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

// ---- the persistent chain's hand-off entries (LL kernels) ----
#ifndef OTPU_LL_SLEEP
#define OTPU_LL_SLEEP 1                          // s_sleep between polls (64 clocks a unit)
#endif
// s_sleep between the polls of a hand-off row's last entry: ~1000 clocks, about one round trip.
// Fewer requests on that line measured faster than an earlier sight of it: c4 313.7-314.3 us a
// step at 1, 311.3-311.7 at 8, 309.3-311.5 at 12, 309.3-309.7 at 16, 308.9-311.0 at 24,
// 317.0-318.9 at 32 (interleaved, one box); 2-4 polls in flight at once measured 319-332.
#ifndef OTPU_LL_LAST_SLEEP
#define OTPU_LL_LAST_SLEEP 16
#endif
__device__ __forceinline__ uint64_t ll_load(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ll_store(uint64_t* p, uint32_t tag, float y) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | fbits(y), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// this thread's float4 chunks c = tid + 256 k (k < CPT, c < NC) of the entry row a.ll_in: once
// the row's last entry carries a.tag_in, every entry is loaded at once, then the entries that do
// not carry it yet are loaded again until they do.  A wait that runs out of polls sets *a.err and
// goes on with what it has (the step's output is then invalid; every wave still ends).
// (A workgroup of 256 threads: wave w's chunks of round k are the row's entries 1024 k + 256 w +
// [0, 256).)
template <int CPT>
__device__ __forceinline__ void ll_chunks(const MMArgs& a, int NC, float4 (&xv)[CPT]) {
    // (the mask tells the compiler that wave < 4, so that where NC is a constant the bounds
    // below resolve at compile time)
    const int tid = threadIdx.x & 255, lane = tid & 63, wave = tid >> 6;
    // First the row's last entry alone (every thread the same address: one request a wave),
    // which the highest-numbered producer writes, the one that tends to finish last.  Polling
    // the whole row from the start, 256 workgroups loaded up to 6 MB a round (the fold's
    // 24 KB input) while the producers still streamed their weights: c4 354.4-354.7 -> 326.7-
    // 329.3 us a step (first and last entry: 333 us; middle and last: 337.6).
    int n = 0;
    for (;; ++n) {
        if ((uint32_t)(ll_load(a.ll_in + 4 * NC - 1) >> 32) == a.tag_in) break;
        if (n >= a.spin) break;                      // (the wait below sets the error word)
        __builtin_amdgcn_s_sleep(OTPU_LL_LAST_SLEEP);
    }
    OTPU_STAMP(a, 7);
    OTPU_STAMP_COUNT(a, 8, n);                           // polls of the last entry that missed
    // Lane l loads the wave's entries 64 j + l (j < 4), so that each load instruction reads 512
    // contiguous bytes and each line of the row is requested once a wave; the chunks are then
    // regrouped through the wave's own LDS slot.  (Lane l loading its own chunk's 4 entries, 4
    // instructions each touched every line of the wave's 2 KB.)
    const int n_e = 4 * NC;
    // Entries past the row: a round wholly past it loads nothing and reads as carrying the tag
    // (a uniform test); in a round that ends inside the wave's part the lanes past the row load
    // the row's last entry instead of branching round their loads (a select on the loaded value
    // here would wait for each load before the next), and their values read as 0 at the regroup.
    uint64_t e[CPT][4];
#pragma unroll
    for (int k = 0; k < CPT; ++k)
#pragma unroll
        for (int j = 0; j < 4; ++j) e[k][j] = (uint64_t)a.tag_in << 32;
#pragma unroll
    for (int k = 0; k < CPT; ++k)
        if (1024 * k + 256 * wave < n_e)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int i = 1024 * k + 256 * wave + 64 * j + lane;
                e[k][j] = ll_load(a.ll_in + (i < n_e ? i : n_e - 1));
            }
    for (n = 0;; ++n) {
        bool done = true;
#pragma unroll
        for (int k = 0; k < CPT; ++k)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if ((uint32_t)(e[k][j] >> 32) != a.tag_in) {
                    done = false;
                    const int i = 1024 * k + 256 * wave + 64 * j + lane;
                    e[k][j] = ll_load(a.ll_in + (i < n_e ? i : n_e - 1));
                }
        if (done) break;
        if (n >= a.spin) {
            __hip_atomic_fetch_or(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
        if (OTPU_LL_SLEEP) __builtin_amdgcn_s_sleep(OTPU_LL_SLEEP);
    }
    OTPU_STAMP_COUNT(a, 9, n);                           // wave 0's rounds of re-polls
    // (no barrier: a wave's LDS accesses complete in order, and no other wave touches its slot)
    __shared__ __align__(16) float slot[4][256];
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            slot[wave][64 * j + lane] = 1024 * k + 256 * wave + 64 * j + lane < n_e ? bitsf((uint32_t)e[k][j]) : 0.0f;
        xv[k] = reinterpret_cast<const float4*>(slot[wave])[lane];
    }
}

// wait for entries [from, to) of the input row as well, values unused: a phase that reads part of
// its input row (o reads q of q, k, v) still waits for every producer of that row, so every
// workgroup that wrote into it has finished reading the row before (which the alternating
// entry rows rely on)
__device__ __forceinline__ void ll_drain(const MMArgs& a, int from, int to) {
    constexpr int NE = 8;                                // entries a thread at most (to - from <= 2048)
    const int tid = threadIdx.x;
    uint64_t e[NE];
#pragma unroll
    for (int j = 0; j < NE; ++j) {
        const int i = from + tid + 256 * j;
        e[j] = i < to ? ll_load(a.ll_in + i) : (uint64_t)a.tag_in << 32;
    }
    for (int n = 0;; ++n) {
        bool done = true;
#pragma unroll
        for (int j = 0; j < NE; ++j)
            if ((uint32_t)(e[j] >> 32) != a.tag_in) {
                done = false;
                e[j] = ll_load(a.ll_in + from + tid + 256 * j);
            }
        if (done) break;
        if (n >= a.spin) {
            __hip_atomic_fetch_or(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
        if (OTPU_LL_SLEEP) __builtin_amdgcn_s_sleep(OTPU_LL_SLEEP);
    }
}

// the prologue QACT's LDS: the quantized row, its group offsets, the waves' maxima (KM columns)
template <int KM>
struct QinLdsT {
    uint32_t qs[KM / 4];
    uint8_t ds[KM / 32];
    uint32_t red[4];
};
using QinLds = QinLdsT<QIN_KMAX>;

// the columns a QACT prologue of L pieces a lane and teams of T holds: one walk of the row, or
// (L = LMAX, a kernel of its own, not the chain's) rows up to QIN_KBIG walked in segments
template <int FMT, int L, int T, bool LL>
constexpr int qin_cols() {
    constexpr int one = L * T * (FMT == OTPU_INT8 ? 16 : 32);
    return LL ? QIN_KMAX : (L == LMAX ? QIN_KBIG : (one < QIN_KBIG ? one : QIN_KBIG));
}

// the activation pieces pbase + i T + tl (i < L) of lane tl from the quantized row in LDS, and
// their W - da (a piece past P gets a negative shift: its terms drop); 4-bit layouts split even
// / odd elements, as the loaded path permutes them
template <int FMT, int L, int T>
__device__ __forceinline__ void qin_act(const uint32_t* qs, const uint8_t* ds, int P, int pbase, int tl, int W,
                                        uint32_t (&act)[L][FMT == OTPU_INT8 ? 4 : 8], int (&shA)[L]) {
#pragma unroll
    for (int i = 0; i < L; ++i) {
        const int p = pbase + i * T + tl;
        const bool ok = p < P;
        if (FMT == OTPU_INT8) {
            const uint4 q4 = ok ? reinterpret_cast<const uint4*>(qs)[p] : make_uint4(0, 0, 0, 0);
            act[i][0] = q4.x; act[i][1] = q4.y; act[i][2] = q4.z; act[i][3] = q4.w;
            shA[i] = W - (ok ? (int)ds[p >> 1] : 0);
        } else {
            uint4 v0 = make_uint4(0, 0, 0, 0), v1 = v0;
            if (ok) {
                v0 = reinterpret_cast<const uint4*>(qs)[2 * p];
                v1 = reinterpret_cast<const uint4*>(qs)[2 * p + 1];
            }
            const uint32_t d[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                act[i][2 * t] = __builtin_amdgcn_perm(d[2 * t + 1], d[2 * t], 0x06040200u);
                act[i][2 * t + 1] = __builtin_amdgcn_perm(d[2 * t + 1], d[2 * t], 0x07050301u);
            }
            shA[i] = W - (ok ? (int)ds[p] : 0);
        }
    }
}

// QACT of the problem's fp32 row in the prologue (fp32.quantize_mx(x, 32) of one row, as
// qact_kernel computes it), once per workgroup: each thread takes float4 chunks of the row
// (folding nsum partial rows in order, times xmul when given, then QACT's RSCALE and CSCALE
// products when given), the workgroup finds the row
// maximum, each 32-group's 8 threads its group maximum (xor exchanges), and the quantized
// bytes and group offsets go to LDS; then every lane reads its own pieces (4-bit layouts:
// even / odd elements split, as the loaded path permutes them).
// issue_weights() issues the first rows' weight loads.  Loads complete in order, so with one
// input row (no fold) the row's loads go out first and the weights after them: the QACT then
// waits for the row only, while the weights stream in (c4: 724 -> 659 us a step).  With a fold
// (nsum > 1) the weights go first and the fold's loads after them (the other order measured
// the same).
// LL (the persistent chain): the LDS is the caller's (one block for all of the kernel's
// phases); LLIN: the row comes from the hand-off entries a.ll_in (the weights and scale factors
// go out first: they do not wait for the hand-off), else from the plain row (the step's first
// phase).
// qs_out / ds_out (optional): where the quantized row and its offsets stay in LDS (the rows of
// more than one walk read their later segments' pieces from there, qin_act)
template <int FMT, int L, int T, bool LL = false, bool LLIN = LL, int NRM = 0, typename IssueWeights>
__device__ __forceinline__ void qin_prologue(const MMArgs& a, int b, uint32_t (&act)[L][FMT == OTPU_INT8 ? 4 : 8],
                                             int (&shA)[L], float& sa2, IssueWeights&& issue_weights,
                                             QinLds* lds = nullptr, const uint32_t** qs_out = nullptr,
                                             const uint8_t** ds_out = nullptr) {
    constexpr int KM = qin_cols<FMT, L, T, LL>();
    uint32_t* qs;
    uint8_t* ds;
    uint32_t* red;
    if constexpr (LL) {
        qs = lds->qs;
        ds = lds->ds;
        red = lds->red;
    } else {
        __shared__ __align__(16) QinLdsT<KM> own;
        qs = own.qs;
        ds = own.ds;
        red = own.red;
    }
    if (qs_out) *qs_out = qs;
    if (ds_out) *ds_out = ds;
    // float4 chunks a thread holds at most: the row has at most KM elements (L T pieces of 16
    // (int8) or 32 (4-bit) elements in one walk), so for the small rows of a chain only the
    // chunks that can exist are compiled (the code runs once per launch, from a cold
    // instruction cache)
    constexpr int EPP = FMT == OTPU_INT8 ? 16 : 32;
    constexpr int CPT0 = (L * T * EPP / 4 + 255) / 256;
    constexpr int KC = (KM / 4 + 255) / 256;              // chunks a thread of the LDS's KM columns
    constexpr int CPT = (L == LMAX && !LL) || CPT0 > KC ? KC : CPT0;
    const int K = a.K, NC = K >> 2, W = window_of(FMT);
    // (workgroups of 256 threads: the mask tells the compiler so, and the chunk tests below then
    // resolve at compile time where K is a constant)
    const int tid = threadIdx.x & 255;
    const float* x = a.xin + b * a.xin_bs;
    const float* xm = a.xmul ? a.xmul + b * a.xin_bs : nullptr;
    // NRM: 0 the RSCALE / CSCALE factors when given, 1 none, 2 both (known at compile time)
    const bool has_r = NRM == 2 || (NRM == 0 && a.rscale != nullptr);
    const bool has_c = NRM == 2 || (NRM == 0 && a.cscale != nullptr);
    const float4* cs = has_c ? reinterpret_cast<const float4*>(a.cscale + b * a.xin_bs) : nullptr;
    float4 v[CPT], cv[CPT];
    float rf = 1.0f;
    uint32_t m = 0;
    // RSCALE / CSCALE factors, loaded with the row (QACT's pre-multiplies: (x * r) * c)
    auto load_scales = [&]() {
        if (has_r) rf = *a.rscale;
        if (has_c) {
#pragma unroll
            for (int k = 0; k < CPT; ++k) {
                const int c = tid + 256 * k;
                if (c < NC) cv[k] = cs[c];
            }
        }
    };
    auto finish = [&](float4 t, int k) {                 // VOP MUL done: pre-multiplies, flush, keep, row max
        if (has_r) { t.x = fmul(t.x, rf); t.y = fmul(t.y, rf); t.z = fmul(t.z, rf); t.w = fmul(t.w, rf); }
        if (has_c) { t.x = fmul(t.x, cv[k].x); t.y = fmul(t.y, cv[k].y); t.z = fmul(t.z, cv[k].z); t.w = fmul(t.w, cv[k].w); }
        // (hand-off entries are results of the FTZ arithmetic, flushed already, as are products)
        if constexpr (!LLIN) { t.x = ftz(t.x); t.y = ftz(t.y); t.z = ftz(t.z); t.w = ftz(t.w); }
        v[k] = t;
        m = max(m, max(max(fbits(t.x) & 0x7FFFFFFFu, fbits(t.y) & 0x7FFFFFFFu),
                       max(fbits(t.z) & 0x7FFFFFFFu, fbits(t.w) & 0x7FFFFFFFu)));
    };
    if (a.nsum == 1) {
        float4 xv[CPT], gv[CPT];
        if (LLIN) {                                      // (no VOP MUL in the chain's linears)
            load_scales();
            __builtin_amdgcn_sched_barrier(0);
            issue_weights();
            __builtin_amdgcn_sched_barrier(0);
            OTPU_STAMP(a, 1);
            ll_chunks<CPT>(a, NC, xv);
            if (a.ll_all > K) ll_drain(a, K, a.ll_all);
            OTPU_STAMP(a, 2);
        } else {
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
            const int c = tid + 256 * k;
            if (c < NC) {
                xv[k] = reinterpret_cast<const float4*>(x)[c];
                if (xm) gv[k] = reinterpret_cast<const float4*>(xm)[c];
            }
        }
        load_scales();
        __builtin_amdgcn_sched_barrier(0);
        issue_weights();
        __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
            const int c = tid + 256 * k;
            v[k] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (c < NC) {
                float4 t = xv[k];
                if (xm) {                                // VOP MUL
                    t.x = fmul(t.x, gv[k].x); t.y = fmul(t.y, gv[k].y); t.z = fmul(t.z, gv[k].z);
                    t.w = fmul(t.w, gv[k].w);
                }
                finish(t, k);
            }
        }
    } else {
    issue_weights();
    load_scales();
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
        const int c = tid + 256 * k;
        v[k] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (c < NC) {
            float4 u[QIN_NSUM_MAX];                      // every partial row's chunk in flight
#pragma unroll
            for (int s = 0; s < QIN_NSUM_MAX; ++s)
                if (s < a.nsum) u[s] = reinterpret_cast<const float4*>(x + s * a.sum_stride)[c];
            float4 t = u[0];
#pragma unroll
            for (int s = 1; s < QIN_NSUM_MAX; ++s)       // the ACC fold, in order
                if (s < a.nsum) {
                    t.x = fadd(t.x, u[s].x); t.y = fadd(t.y, u[s].y); t.z = fadd(t.z, u[s].z); t.w = fadd(t.w, u[s].w);
                }
            if (xm) {                                    // VOP MUL
                const float4 g = reinterpret_cast<const float4*>(xm)[c];
                t.x = fmul(t.x, g.x); t.y = fmul(t.y, g.y); t.z = fmul(t.z, g.z); t.w = fmul(t.w, g.w);
            }
            finish(t, k);
        }
    }
    }
    // (one chunk a thread: m is that chunk's maximum, and the row maximum's wave reduction
    // passes its 32-group's maximum on the way)
    uint32_t g0 = 0;
    if constexpr (CPT == 1) m = wave_max_dpp_64_8(m, g0);
    else m = wave_max_dpp(m, 64);
    if ((tid & 63) == 0) red[tid >> 6] = m;
    if constexpr (LL) OTPU_STAMP(a, 6);
    __syncthreads();
    if constexpr (LL) OTPU_STAMP(a, 5);
    const uint32_t amax = max(max(red[0], red[1]), max(red[2], red[3]));
    const float fa = bitsf(amax);
    // no test of amax (recip(0) is 0: a zero row quantizes to 0 with Sa 0) or of a group's
    // maximum (a zero group's offset selected as 0), and the LDS stores after the chunks'
    // math: without branches the chunks' chains interleave (one wave a SIMD)
    // fmul(127, recip(fa)) and fmul(inv, 2^dg) as plain products: recip gives +0 or a normal
    // number, so both are 0, normal or +inf (never a denormal or NaN to flush)
    const float inv = 127.0f * recip(fa);
    sa2 = fmul(fmul(fa, bitsf(0x3C010204u)), pow2f(-W));
    uint32_t qv[CPT];
    int dgv[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
        if (k * 256 >= NC) break;                        // uniform: the shuffles below converge
        uint32_t gm = g0;
        if constexpr (CPT > 1) {
            gm = max(max(fbits(v[k].x) & 0x7FFFFFFFu, fbits(v[k].y) & 0x7FFFFFFFu),
                     max(fbits(v[k].z) & 0x7FFFFFFFu, fbits(v[k].w) & 0x7FFFFFFFu));
            gm = wave_max_dpp(gm, 8);                     // the 8 chunks of this 32-group
        }
        int dg = (int)(amax >> 23) - (int)(gm >> 23) - ((gm & 0x7FFFFFu) > (amax & 0x7FFFFFu));
        dg = gm ? (dg < 0 ? 0 : (dg > 31 ? 31 : dg)) : 0;
        const float sc = inv * pow2f(dg);
        // v and sc are flushed: q8 of the IEEE product is q8 of fmul's (a denormal product
        // rounds to 0 either way, NaN gives 0)
        qv[k] = (uint32_t)(q8(v[k].x * sc) & 0xFF) | ((uint32_t)(q8(v[k].y * sc) & 0xFF) << 8)
              | ((uint32_t)(q8(v[k].z * sc) & 0xFF) << 16) | ((uint32_t)(q8(v[k].w * sc) & 0xFF) << 24);
        dgv[k] = dg;
    }
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
        const int c = tid + 256 * k;
        if (k * 256 >= NC) break;
        if (c < NC) {
            qs[c] = qv[k];
            if ((c & 7) == 0) ds[c >> 3] = (uint8_t)dgv[k];
        }
    }
    __syncthreads();
    qin_act<FMT, L, T>(qs, ds, a.P, 0, tid & (T - 1), W, act, shA);
}

// the kernel body for a team of T lanes (T a compile-time constant: the exchanges of the
// reduction are then straight-line code); QIN: the activation row is quantized in the prologue;
// LL: a phase of the persistent chain (hand-off entries in and out, the caller's LDS)
template <int FMT, int MR, int L, int T, bool PLAIN, bool QIN, int R, bool LL = false, bool LLIN = LL, int NRM = 0>
__device__ __forceinline__ void gemv_body(const MMArgs& a, QinLds* lds = nullptr) {
    constexpr int AW = FMT == OTPU_INT8 ? 4 : 8;          // activation dwords per piece
    constexpr int E = R * MR;                             // sums a lane carries per iteration
    constexpr bool SEGS = L == LMAX && !QIN && !LL;       // rows of more pieces than one walk holds
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
    float sa2[MR];
    static_assert(!QIN || MR == 1, "the prologue QACT quantizes one activation row");
    // (QIN: quantized by qin_prologue below, once the first rows' loads are in flight.)
    // Otherwise every activation load goes out at once (act_issue), then the first rows' weight
    // loads, then the pieces are unpacked (act_finish, whose waits, the loads completing in order,
    // do not cover the weights). A piece past P or a row past M reads piece 0 of row 0 and keeps
    // it: its shift is made negative, which drops its terms (piece_term), so no branch or select
    // sits between the loads (with a branch around each piece's loads, each offset byte's wait
    // came before the next piece's loads and before any weight load).
    constexpr int AQ = FMT == OTPU_INT8 ? 1 : 2;          // 16-byte loads a piece
    uint4 araw[MR][L][AQ];
    int draw[MR][L];
    auto act_issue = [&](int pbase) {
#pragma unroll
        for (int j = 0; j < MR; ++j) {
#pragma unroll
            for (int i = 0; i < L; ++i) {
                const int p = pbase + i * T + tl;
                const bool ok = p < P && j < a.M;
                const int8_t* qp = q + (ok ? j * a.ldq + 16 * AQ * p : 0);
#pragma unroll
                for (int h = 0; h < AQ; ++h) araw[j][i][h] = *reinterpret_cast<const uint4*>(qp + 16 * h);
                draw[j][i] = da[ok ? j * a.ldda + (FMT == OTPU_INT8 ? (p >> 1) : p) : 0];
            }
        }
    };
    auto act_finish = [&](int pbase) {
#pragma unroll
        for (int j = 0; j < MR; ++j) {
#pragma unroll
            for (int i = 0; i < L; ++i) {
                const uint4 v0 = araw[j][i][0];
                if (FMT == OTPU_INT8) {
                    act[j][i][0] = v0.x; act[j][i][1] = v0.y; act[j][i][2] = v0.z; act[j][i][3] = v0.w;
                } else {
                    const uint4 v1 = araw[j][i][AQ - 1];
                    const uint32_t d[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        act[j][i][2 * t] = __builtin_amdgcn_perm(d[2 * t + 1], d[2 * t], 0x06040200u);
                        act[j][i][2 * t + 1] = __builtin_amdgcn_perm(d[2 * t + 1], d[2 * t], 0x07050301u);
                    }
                }
                const bool ok = pbase + i * T + tl < P && j < a.M;
                shA[j][i] = ok ? W - draw[j][i] : -4096;
            }
        }
#pragma unroll
        for (int j = 0; j < MR; ++j) sa2[j] = (j < a.M && !a.acc_out) ? fmul(Sa[j], pow2f(-W)) : 0.0f;
    };

    // wave-uniform by construction; readfirstlane tells the compiler (scalar loop, no exec masks)
    const int wave = __builtin_amdgcn_readfirstlane((blockIdx.x * GEMV_THREADS + threadIdx.x) >> 6);
    const int nwaves = (gridDim.x * GEMV_THREADS) >> 6;
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
    // LL gate/up pairs (gu_pair = F; 4 rows a team, 2 teams a wave): the 8 slots of the wave's
    // group n0 are g rows n0/2 .. n0/2 + 3 and the u rows F after them, team t taking g and u of
    // rows n0/2 + 2t, + 1 (slot r: u for r >= 2, row + (r & 1)), so each g sits 16 lanes below
    // its u after the reduce-scatter
    constexpr bool PAIRS = LL && R == 4 && NT == 2;
    const int gp = PAIRS ? a.gu_pair : 0;
    auto slot_row = [&](int r) { return (r >= 2 ? gp : 0) + 2 * team + (r & 1); };
    auto load = [&](Stage& st, int n0, int pbase = 0) {
        const int base = gp ? n0 / 2 : n0;
        const uint8_t* wb = w + (int64_t)base * a.rs;
        const uint8_t* sb = ws + (int64_t)base * a.srs;
        const int last = a.N - 1 - n0;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int dn = gp ? slot_row(r) : min(r * NT + team, last);
            const uint32_t roff = (uint32_t)dn * (uint32_t)a.rs;
            const uint32_t soff = (uint32_t)dn * (uint32_t)a.srs;
#pragma unroll
            for (int i = 0; i < L; ++i) {
                const int p = pbase + i * T + tl;
                const int pc = p < P ? p : P - 1;
                st.wv[r][i] = ld16(wb + (roff + 16u * (uint32_t)pc));
                st.sc[r][i] = piece_scale<FMT>(sb, soff, k0, pc, plain);
            }
        }
        // (LL: flushed where it is used, so that issuing the loads waits for none of them and the
        // hand-off's polls go out at once)
        const int de = gp ? slot_row(er) : min(er * NT + team, last);
        const float swr = unit ? 1.0f : *reinterpret_cast<const float*>(sb + (uint32_t)de * (uint32_t)a.srs);
        st.sw = LL ? swr : ftz(swr);
    };
    // the exact sums of one segment's pieces (pbase on): v = them (first), else v += them
    auto dots = [&](const Stage& st, double (&v)[E], int pbase, bool first) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int j = 0; j < MR; ++j) {
                double acc = 0.0;
#pragma unroll
                for (int i = 0; i < L; ++i) {
                    int c0, c1;
                    piece_dot<FMT>(st.wv[r][i], act[j][i], c0, c1);
                    acc += piece_term<FMT, PLAIN>(c0, c1, st.sc[r][i], shA[j][i], pbase + i * T + tl);
                }
                v[r * MR + j] = first ? acc : v[r * MR + j] + acc;
            }
        }
    };
    auto epilogue = [&](double (&v)[E], float sw, int n0) {
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
        if constexpr (LL) {                           // (QIN, one activation row, no flags)
            // every lane forms its y (only the epilogue lanes' are kept): the pairs' exchange
            // below needs the whole wave
            const float y = fmul_f(fmul_f((float)tot, ftz(sw)), sa2[0]);
            if (gp) {
                const float yu = __uint_as_float(
                    __builtin_amdgcn_permlane16_swap(fbits(y), fbits(y), false, false)[1]);
                const int nl = n0 / 2 + slot_row(er);
                if (epilane) {
                    out[nl] = y;
                    if (er < 2) ll_store(a.ll_out + nl, a.tag_out, fmul(y, yu));   // VOP MUL g * u
                }
            } else {
                const int n = n0 + er * NT + team;
                if (epilane && n < a.N) {
                    out[n] = y;
                    ll_store(a.ll_out + n, a.tag_out, y);
                }
            }
            return;
        }
        const int n = n0 + er * NT + team;
        if (epilane && n < a.N && ej < a.M) {
            if (a.acc_out) {
                a.acc_out[(int64_t)ej * a.N + n] = (int64_t)tot;
            } else {
                // fmul(fmul(i2f(acc), Sw), Sa * 2^-W): the float of an integer, the flushed Sw
                // and the finished Sa * 2^-W need no operand flush
                float y = fmul_f(fmul_f((float)tot, sw), sa2[ej]);
                if constexpr (QIN) {                  // (no ACC / ASCALE / RMAX / LM head here)
                    out[(int64_t)ej * a.ors + n] = y;
                    return;
                }
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
    auto compute = [&](const Stage& st, int n0) {
        double v[E];
        dots(st, v, 0, true);
        epilogue(v, st.sw, n0);
    };

    // one stage per wave: the loads of an iteration go out together and the waves of the SIMD
    // (5-8 resident) overlap each other's memory latency; a second register stage per wave
    // costs occupancy and measured slower on MI355X
    if constexpr (QIN && L == LMAX && !LL) {
        // (the widest prologue: rows of more than one walk read each segment's pieces from LDS)
        Stage st;
        const int nfirst = wave * RW;
        const uint32_t* qs = nullptr;
        const uint8_t* ds = nullptr;
        qin_prologue<FMT, L, T, LL, LLIN, NRM>(a, b, act[0], shA[0], sa2[0], [&] {
            if (nfirst < a.N) load(st, nfirst);
        }, lds, &qs, &ds);
        if (a.nseg > 1) {
            const int PS = T * L;
            for (int n0 = nfirst; n0 < a.N; n0 += stride) {
                double v[E];
                float sw = 0.0f;
                for (int sg = 0; sg < a.nseg; ++sg) {
                    if (sg > 0 || n0 != nfirst) {
                        qin_act<FMT, L, T>(qs, ds, P, sg * PS, tl, W, act[0], shA[0]);
                        load(st, n0, sg * PS);
                    }
                    dots(st, v, sg * PS, sg == 0);
                    sw = st.sw;
                }
                epilogue(v, sw, n0);
            }
        } else {
            for (int n0 = nfirst; n0 < a.N; n0 += stride) {
                if (n0 != nfirst) load(st, n0);
                compute(st, n0);
            }
        }
    } else if constexpr (QIN) {
        // the first rows stream in while the workgroup quantizes the activation row
        Stage st;
        const int nfirst = wave * RW;
        qin_prologue<FMT, L, T, LL, LLIN, NRM>(a, b, act[0], shA[0], sa2[0], [&] {
            if (nfirst < a.N) load(st, nfirst);
        }, lds);
        if constexpr (LL) OTPU_STAMP(a, 3);
        for (int n0 = nfirst; n0 < a.N; n0 += stride) {
            if (n0 != nfirst) load(st, n0);
            compute(st, n0);
        }
    } else if (SEGS && a.nseg > 1) {
        // a row longer than the registers hold (T L pieces): each row group is walked in nseg
        // segments, the activation pieces of a segment loaded again for it (from the caches:
        // the row is small and every wave reads it), the exact double sums carried across
        const int PS = T * L;
        for (int n0 = wave * RW; n0 < a.N; n0 += stride) {
            double v[E];
            float sw = 0.0f;
            for (int sg = 0; sg < a.nseg; ++sg) {
                Stage st;
                act_issue(sg * PS);
                load(st, n0, sg * PS);
                act_finish(sg * PS);
                dots(st, v, sg * PS, sg == 0);
                sw = st.sw;
            }
            epilogue(v, sw, n0);
        }
    } else {
        // the first rows stream in while the activation row loads
        act_issue(0);
        const int nfirst = wave * RW;
        if (nfirst < a.N) {
            Stage st;
            load(st, nfirst);
            act_finish(0);
            compute(st, nfirst);
        }
        for (int n0 = nfirst + stride; n0 < a.N; n0 += stride) {
            Stage st;
            load(st, n0);
            compute(st, n0);
        }
    }
    if (a.best) {                               // one maximum a workgroup
        __shared__ uint64_t red[4];
        best = wave_max_u64(best);
        if (lane == 0) red[threadIdx.x >> 6] = best;
        __syncthreads();
        if (threadIdx.x == 0) {
            uint64_t m = red[0];
            for (int i = 1; i < GEMV_THREADS / 64; ++i) m = red[i] > m ? red[i] : m;
            // an atomic max without return on one of LM_WORDS words, each on a line of its own:
            // nothing waits for it (a test of the word first, or an atomic with return, would
            // hold the workgroup's CU slot for a device-scope round trip), and the words spread
            // the atomics, which serialize per line at the memory side
            if (m)
                __hip_atomic_fetch_max(reinterpret_cast<unsigned long long*>(a.best) + LM_STRIDE * (blockIdx.x % LM_WORDS),
                                       (unsigned long long)m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// R: rows a team takes per iteration
template <int FMT, int MR, int L, bool PLAIN, int R>
__global__ __launch_bounds__(256) void gemv_kernel(MMArgs a) {
    if (a.T == 64) gemv_body<FMT, MR, L, 64, PLAIN, false, R>(a);
    else if (a.T == 32) gemv_body<FMT, MR, L, 32, PLAIN, false, R>(a);
    else gemv_body<FMT, MR, L, 16, PLAIN, false, R>(a);
}

// MM with the QACT of its one activation row in the prologue
template <int FMT, int L, bool PLAIN, int R>
__global__ __launch_bounds__(256) void gemv_qin_kernel(MMArgs a) {
    if (a.T == 64) gemv_body<FMT, 1, L, 64, PLAIN, true, R>(a);
    else if (a.T == 32) gemv_body<FMT, 1, L, 32, PLAIN, true, R>(a);
    else gemv_body<FMT, 1, L, 16, PLAIN, true, R>(a);
}

// workgroups per CU the streaming grid aims for (measured on MI355X): for one piece a lane 64,
// where the 80-problem c2 and the 128-problem c1 give each wave one row group (c2: 7.01-7.03
// TB/s against 6.58-6.79 at 40, 6.74-6.83 at 32, 6.80-6.82 at 48 and 6.90 at 56, two runs on
// one box; c1: 6.86-6.92 against 6.59-6.62 at 32); 24 for four or more pieces (the LM head:
// 103.7-104.4 against 104.6-106.5 us at 16 over four paired runs, 106-108 at 8, 12 or 32),
// else 8; OTPU_GEMV_BLOCKS_PER_CU overrides
inline int gemv_blocks_per_cu(int L, int fmt) {
    (void)fmt;
    static const int v = [] {                   // read once (thread-safe static initialisation)
        const char* e = getenv("OTPU_GEMV_BLOCKS_PER_CU");
        const int x = e ? atoi(e) : 0;
        return (x > 0 && x <= 64) ? x : 0;
    }();
    return v ? v : (L == 1 ? 64 : (L >= 4 ? 24 : 8));
}

// rows a team takes per iteration (one activation row, one piece a lane) when the default
// would give fewer workgroups than CUs: a small single GEMV then still spreads over the chip
constexpr int R_SMALL = 4;

// the grid of a launch with R rows a team: about gemv_blocks_per_cu workgroups per CU over the
// whole batch, fewer when the rows run out (each wave then streams many row groups; its
// activation registers are loaded once)
inline int64_t gemv_blocks(const MMArgs& a, int fmt, int R, int L, int batch) {
    const int64_t waves = (a.N + (int64_t)R * (64 / a.T) - 1) / ((int64_t)R * (64 / a.T));
    int64_t blocks = (waves + 3) / 4;
    int64_t cap = (int64_t)otpu_cu_count() * gemv_blocks_per_cu(L, fmt) / batch;
    if (cap < 1) cap = 1;
    return blocks > cap ? cap : blocks;
}

template <int FMT, int MR, int L, int R>
void launch_grid(const MMArgs& a, int batch, hipStream_t s) {
    const int64_t blocks = gemv_blocks(a, FMT, R, L, batch);
    if (a.flags & (OTPU_UNIT | OTPU_RSC))
        gemv_kernel<FMT, MR, L, true, R><<<dim3((unsigned)blocks, batch), dim3(256), 0, s>>>(a);
    else
        gemv_kernel<FMT, MR, L, false, R><<<dim3((unsigned)blocks, batch), dim3(256), 0, s>>>(a);
}

template <int FMT, int MR, int L>
void launch_one(const MMArgs& a, int batch, hipStream_t s) {
    static_assert(fits<FMT, 1, L>(), "one activation row always fits");
    if constexpr (fits<FMT, MR, L>()) {
        constexpr int R = rows_per_team<L, MR>();
        if constexpr (MR == 1 && L == 1 && R > R_SMALL) {
            if (gemv_blocks(a, FMT, R, L, batch) * batch < otpu_cu_count()) {
                launch_grid<FMT, MR, L, R_SMALL>(a, batch, s);
                return;
            }
        }
        launch_grid<FMT, MR, L, R>(a, batch, s);
    }
}

template <int FMT, int MR>
void launch_L(const MMArgs& a, int L, int batch, hipStream_t s) {
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
void launch_fmt(const MMArgs& a, int mr, int L, int batch, hipStream_t s) {
    if (mr == 1) launch_L<FMT, 1>(a, L, batch, s);
    else if (mr == 2) launch_L<FMT, 2>(a, L, batch, s);
    else launch_L<FMT, 4>(a, L, batch, s);
}

template <int FMT, int L, int R>
void launch_qin_grid(const MMArgs& a, int batch, hipStream_t s) {
    const int64_t blocks = gemv_blocks(a, FMT, R, L, batch);
    if (a.flags & (OTPU_UNIT | OTPU_RSC))
        gemv_qin_kernel<FMT, L, true, R><<<dim3((unsigned)blocks, batch), dim3(256), 0, s>>>(a);
    else
        gemv_qin_kernel<FMT, L, false, R><<<dim3((unsigned)blocks, batch), dim3(256), 0, s>>>(a);
}

template <int FMT, int L>
void launch_qin(const MMArgs& a, int batch, hipStream_t s) {
    constexpr int R = rows_per_team<L, 1>();
    if constexpr (L == 1 && R > R_SMALL) {
        if (gemv_blocks(a, FMT, R, L, batch) * batch < otpu_cu_count()) {
            launch_qin_grid<FMT, L, R_SMALL>(a, batch, s);
            return;
        }
    }
    launch_qin_grid<FMT, L, R>(a, batch, s);
}

template <int FMT>
void launch_qin_fmt(const MMArgs& a, int L, int batch, hipStream_t s) {
    switch (L) {
        case 1: launch_qin<FMT, 1>(a, batch, s); break;
        case 2: launch_qin<FMT, 2>(a, batch, s); break;
        case 3: launch_qin<FMT, 3>(a, batch, s); break;
        case 4: launch_qin<FMT, 4>(a, batch, s); break;
        case 5: launch_qin<FMT, 5>(a, batch, s); break;
        case 6: launch_qin<FMT, 6>(a, batch, s); break;
        default: launch_qin<FMT, 8>(a, batch, s); break;
    }
}


}  // namespace otpu
