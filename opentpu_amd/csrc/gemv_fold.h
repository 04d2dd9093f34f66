// The down projection of a chained decode layer in one launch, its ranges folded in the kernel:
// the QACT of every F-chunk ("range", 256 elements) of the fp32 input row mul(x, xmul), one MM
// per range and weight row, and the ACC of the ranges' fp32 outputs in range order, so the layer
// leaves its output row folded (Builder.dot's per-range MMs + ACC, opentpu/compiler.py:2686-2720;
// swiglu_down's chunk loop, opentpu/kernels/mlp.py:87-120).  Bit for bit what otpu_mm_qin's
// ranges (one partial row each) followed by the fold of those rows compute.
//
// 4-bit weights with scale rows (int4x, fp4x6, nvfp4), whose down chunk is 256 elements (at
// F = 3072, opentpu/kernels/mlp.py:8-24): a range is 8 pieces of
// 16 bytes.  A team of T lanes owns a weight row, lane tl holding pieces i T + tl (i < L), whose
// range is (i T + tl) / 8: the 8 lanes tl >> 3 of slot i hold one range, so a range's integer
// sum is a reduction over 8 lanes.  Each range's epilogue runs in its lanes; the team's first
// lane gathers the ranges' outputs in order and adds them.
// The prologue needs no cross-wave reduction: with 256 threads taking float4 chunk tid + 256 k,
// wave w holds chunks 256 k + 64 w .. + 63, i.e. all of range 4 k + w.
#pragma once
#include "gemv_impl.h"

namespace otpu {

constexpr int FOLD_C = 256;                       // elements a range
constexpr int FOLD_PPR = FOLD_C / 32;             // 16-byte pieces a range
constexpr int FOLD_NRMAX = FOLD_KMAX / FOLD_C;    // ranges a row

// lane 8 g's x of each team of T lanes (g < T / 8), at the team's first lane: DPP row_ror:8
// moves lane 8 to lane 0 within a row of 16; v_permlane16_swap of (x, x) returns the other row
// of each row pair in its second half, v_permlane32_swap the other half-wave
__device__ __forceinline__ float ror8(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xF, 0xF, false));
}
__device__ __forceinline__ float row_swap16(float x) {
    return __uint_as_float(__builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false)[1]);
}
__device__ __forceinline__ float half_swap32(float x) {
    return __uint_as_float(__builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false)[1]);
}
template <int T>
__device__ __forceinline__ void gather8(float x, float (&v)[T / 8]) {
    v[0] = x;
    v[1] = ror8(x);
    if constexpr (T >= 32) {
        const float h = row_swap16(x);
        v[2] = h;
        v[3] = ror8(h);
    }
    if constexpr (T == 64) {
        const float q = half_swap32(x);
        v[4] = q;
        v[5] = ror8(q);
        const float qh = row_swap16(q);
        v[6] = qh;
        v[7] = ror8(qh);
    }
}

// the fold's LDS: the quantized row, its group offsets, each 256-column sub-range's Sa * 2^-W
// (its range's), the sub-ranges' maxima (ranges of more than one sub-range)
struct FoldLds {
    uint32_t qs[FOLD_KMAX / 4];
    uint8_t ds[FOLD_KMAX / 32];
    float sa2s[FOLD_NRMAX];
    uint32_t smaxs[FOLD_NRMAX];
};

// LL: a phase of the persistent chain: the input row mul(g, u) from hand-off entries (the gate/up
// phase publishes the products; the weights and scale factors go out first), the output row
// also as entries, the caller's LDS
template <int FMT, int L, int T, bool LL = false>
__device__ __forceinline__ void fold_body(const MMArgs& a, FoldLds* lds = nullptr) {
    static_assert(FMT != OTPU_INT8, "4-bit weights");
    static_assert(T % FOLD_PPR == 0, "a range's lanes inside one team");
    FoldLds* S;
    if constexpr (LL) {
        S = lds;
    } else {
        __shared__ __align__(16) FoldLds own;
        S = &own;
    }
    uint32_t* qs = S->qs;
    uint8_t* ds = S->ds;
    float* sa2s = S->sa2s;
    uint32_t* smaxs = S->smaxs;
    // float4 chunks a thread holds at most: K <= 32 L T (only the chunks that can exist are
    // compiled: the code runs once per launch, from a cold instruction cache)
    constexpr int CPT0 = (L * T * 8 + 255) / 256;
    constexpr int CPT = CPT0 < FOLD_KMAX / 4 / 256 ? CPT0 : FOLD_KMAX / 4 / 256;
    constexpr int NT = 64 / T;                    // teams a wave
    constexpr int GPT = T / FOLD_PPR;             // ranges a team slot holds
    // ranges of FC sub-ranges of 256 columns (the reference's down chunk is 256 up to F = 3840,
    // then wider: opentpu/kernels/mlp.py:8-30); NS sub-ranges, NR ranges
    const int FC = a.fold_c > 1 ? a.fold_c : 1;
    const int K = a.K, NC = K >> 2, W = window_of(FMT), P = a.P, NS = K / FOLD_C, NR = NS / FC;
    // (workgroups of 256 threads: the mask tells the compiler so, and the chunk tests below then
    // resolve at compile time where K is a constant)
    const int tid = threadIdx.x & 255, lane = tid & 63, tl = lane & (T - 1), team = lane / T;
    const int wave = __builtin_amdgcn_readfirstlane((blockIdx.x * GEMV_THREADS + tid) >> 6);
    const int nwaves = (gridDim.x * GEMV_THREADS) >> 6;
    const float* x = a.xin;
    const float* xm = a.xmul;

    struct Stage {
        uint4 wv[L];
        uint32_t sc[L];
        float sw;
    };
    // a team's row n: pieces past P read the last piece (they meet zero activations), rows
    // past N the last row (they reach no store)
    auto load = [&](Stage& st, int n) {
        const int nr = min(n, a.N - 1);
        const uint8_t* wr = a.w + (int64_t)nr * a.rs;
        const uint8_t* sr = a.ws + (int64_t)nr * a.srs;
#pragma unroll
        for (int i = 0; i < L; ++i) {
            const int p = i * T + tl, pc = p < P ? p : P - 1;
            st.wv[i] = ld16(wr + 16 * pc);
            st.sc[i] = piece_scale<FMT>(sr, 0u, a.k0, pc, false);
        }
        const float swr = *reinterpret_cast<const float*>(sr);
        st.sw = LL ? swr : ftz(swr);                    // (LL: flushed where used, as in gemv_body)
    };

    // 1. the input row's loads, then the first row's weights (loads complete in order); LL:
    // the weights first, then the hand-off's entries
    float4 xv[CPT], gv[CPT], cv[CPT];
    const float4* cs = reinterpret_cast<const float4*>(a.cscale);
    const float rf = a.rscale ? *a.rscale : 1.0f;
    Stage st;
    const int nfirst = wave * NT + team;
    if constexpr (LL) {
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
            const int c = tid + 256 * k;
            if (c < NC && cs) cv[k] = cs[c];
        }
        if (wave * NT < a.N) load(st, nfirst);
        __builtin_amdgcn_sched_barrier(0);
        OTPU_STAMP(a, 1);
        ll_chunks<CPT>(a, NC, xv);
        OTPU_STAMP(a, 2);
    } else {
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
        const int c = tid + 256 * k;
        if (c < NC) {
            xv[k] = reinterpret_cast<const float4*>(x)[c];
            if (xm) gv[k] = reinterpret_cast<const float4*>(xm)[c];
            if (cs) cv[k] = cs[c];
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    if (wave * NT < a.N) load(st, nfirst);
    __builtin_amdgcn_sched_barrier(0);
    }

    // 2. QACT of each range: the wave's 64 chunks at k are range 4 k + w (whole waves: K is a
    // multiple of 256, so NC of 64).  The chunks' products and maxima first, then their
    // reductions side by side (independent DPP chains).
    float4 tv[CPT];
    uint32_t cm[CPT], am[CPT], gm[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
        const int c = tid + 256 * k;
        float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
        if (LL || c < NC) t = xv[k];                     // (LL: entries past the row read as 0)
        if (c < NC) {
            if (!LL && xm) {                             // VOP MUL
                t.x = fmul(t.x, gv[k].x); t.y = fmul(t.y, gv[k].y); t.z = fmul(t.z, gv[k].z); t.w = fmul(t.w, gv[k].w);
            }
            if (a.rscale) { t.x = fmul(t.x, rf); t.y = fmul(t.y, rf); t.z = fmul(t.z, rf); t.w = fmul(t.w, rf); }
            if (cs) {                                    // RSCALE, then CSCALE: (x * r) * c
                t.x = fmul(t.x, cv[k].x); t.y = fmul(t.y, cv[k].y); t.z = fmul(t.z, cv[k].z); t.w = fmul(t.w, cv[k].w);
            }
            // (hand-off entries are results of the FTZ arithmetic, flushed already, as are products)
            if constexpr (!LL) { t.x = ftz(t.x); t.y = ftz(t.y); t.z = ftz(t.z); t.w = ftz(t.w); }
        }
        tv[k] = t;
        cm[k] = max(max(fbits(t.x) & 0x7FFFFFFFu, fbits(t.y) & 0x7FFFFFFFu),
                    max(fbits(t.z) & 0x7FFFFFFFu, fbits(t.w) & 0x7FFFFFFFu));
    }
#pragma unroll
    for (int k = 0; k < CPT; ++k)                          // the sub-range's maximum, and on the way
        am[k] = wave_max_dpp_64_8(cm[k], gm[k]);          // the 8 chunks' of this 32-group
    if (FC > 1) {                                          // (uniform) a range's maximum over its
#pragma unroll                                             // sub-ranges, which other waves hold
        for (int k = 0; k < CPT; ++k) {
            const int c = tid + 256 * k;
            if (c < NC && lane == 0) smaxs[c >> 6] = am[k];
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
            const int c = tid + 256 * k;
            if (c >= NC) continue;                           // whole waves: uniform
            const int r0 = c >> 6 < FC ? 0 : udiv_small(c >> 6, FC) * FC;
            uint32_t m = 0;
            for (int j = 0; j < FC; ++j) m = max(m, smaxs[r0 + j]);
            am[k] = m;
        }
    }
    // The chunks' quantization without branches (with one wave a SIMD a branch serializes what
    // follows it; branch-free, the chunks' chains interleave): no test of the range maximum
    // (recip(0) is 0, so a zero range quantizes to 0 and its Sa is 0) or of the group maximum
    // (a zero group's offset selected as 0).  The LDS stores follow, under the chunk tests.
    uint32_t qv[CPT];
    int dgv[CPT];
    float sav[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
        const uint32_t amax = am[k], g = gm[k];
        const float fa = bitsf(amax);
        // fmul(127, recip(fa)) and fmul(inv, 2^dg) as plain products: recip gives +0 or a normal
        // number, so both are 0, normal or +inf (never a denormal or NaN to flush)
        const float inv = 127.0f * recip(fa);
        sav[k] = fmul(fmul(fa, bitsf(0x3C010204u)), pow2f(-W));
        int dg = (int)(amax >> 23) - (int)(g >> 23) - ((g & 0x7FFFFFu) > (amax & 0x7FFFFFu));
        dg = g ? (dg < 0 ? 0 : (dg > 31 ? 31 : dg)) : 0;
        const float4 t = tv[k];
        const float sc = inv * pow2f(dg);
        // t and sc are flushed: q8 of the IEEE product is q8 of fmul's
        qv[k] = (uint32_t)(q8(t.x * sc) & 0xFF) | ((uint32_t)(q8(t.y * sc) & 0xFF) << 8)
              | ((uint32_t)(q8(t.z * sc) & 0xFF) << 16) | ((uint32_t)(q8(t.w * sc) & 0xFF) << 24);
        dgv[k] = dg;
    }
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
        const int c = tid + 256 * k;
        if (c >= NC) continue;                           // whole waves: uniform
        if (lane == 0) sa2s[c >> 6] = sav[k];
        qs[c] = qv[k];
        if ((c & 7) == 0) ds[c >> 3] = (uint8_t)dgv[k];
    }
    if constexpr (LL) OTPU_STAMP(a, 6);
    __syncthreads();
    if constexpr (LL) OTPU_STAMP(a, 5);

    // 3. this lane's activation pieces (even / odd element bytes) and the ranges' Sa * 2^-W
    uint32_t act[L][8];
    int shA[L];
    float sa2[L];
#pragma unroll
    for (int i = 0; i < L; ++i) {
        const int p = i * T + tl;
        const bool ok = p < P;
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
        sa2[i] = ok ? sa2s[p / FOLD_PPR] : 0.0f;
    }

    if constexpr (LL) OTPU_STAMP(a, 3);
    // 4. rows: per range the exact sum over its 8 lanes, its epilogue, the fold in range order
    for (int n0 = wave * NT; n0 < a.N; n0 += nwaves * NT) {
        const int n = n0 + team;
        if (n0 != wave * NT) load(st, n);
        double sr[L];
#pragma unroll
        for (int i = 0; i < L; ++i) {
            int c0, c1;
            piece_dot<FMT>(st.wv[i], act[i], c0, c1);
            double s = piece_term<FMT, false>(c0, c1, st.sc[i], shA[i], i * T + tl);
            s = xsum(s, 1);
            s = xsum(s, 2);
            sr[i] = xsum(s, 4);                          // the sub-range's exact sum
        }
        // fmul(fmul(i2f(acc), Sw), Sa * 2^-W): the float of an integer, the flushed Sw and the
        // finished Sa * 2^-W need no operand flush
        const float swf = LL ? ftz(st.sw) : st.sw;
        float y = 0.0f;
        if (FC == 1) {
            // every lane its range's epilogue; the team's first lane gathers the outputs (lanes
            // team T + 8 g of slot i hold range i GPT + g) and adds them in range order (fmul
            // results, flushed)
            float yr[L];
#pragma unroll
            for (int i = 0; i < L; ++i) yr[i] = fmul_f(fmul_f((float)sr[i], swf), sa2[i]);
#pragma unroll
            for (int i = 0; i < L; ++i) {
                float v[GPT];
                gather8<T>(yr[i], v);
#pragma unroll
                for (int g = 0; g < GPT; ++g) {
                    const int r = i * GPT + g;
                    if (r < NR) y = r ? fadd_f(y, v[g]) : v[g];
                }
            }
        } else {
            // the team's first lane gathers the sub-ranges' exact sums in order, adds each
            // range's FC of them (integers below 2^53: exact in double), then the range's
            // epilogue, and folds the ranges in order
            double acc = 0.0;
            int in_range = 0;                            // sub-ranges of the current range so far
#pragma unroll
            for (int i = 0; i < L; ++i) {
                float vh[GPT], vl[GPT], vs[GPT];
                gather8<T>(__int_as_float(__double2hiint(sr[i])), vh);
                gather8<T>(__int_as_float(__double2loint(sr[i])), vl);
                gather8<T>(sa2[i], vs);
#pragma unroll
                for (int g = 0; g < GPT; ++g) {
                    const int u = i * GPT + g;
                    if (u >= NS) continue;
                    acc += __hiloint2double(__float_as_int(vh[g]), __float_as_int(vl[g]));
                    if (++in_range == FC) {              // (a count, not (u + 1) % FC: no division)
                        in_range = 0;
                        const float yv = fmul_f(fmul_f((float)acc, swf), vs[g]);
                        y = u + 1 > FC ? fadd_f(y, yv) : yv;
                        acc = 0.0;
                    }
                }
            }
        }
        if (tl == 0 && n < a.N) {
            a.out[n] = y;
            if constexpr (LL) ll_store(a.ll_out + n, a.tag_out, y);
        }
    }
}

}  // namespace otpu
