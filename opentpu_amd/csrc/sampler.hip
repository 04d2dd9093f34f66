// The sampled decode's pick after the LM head, on the GPU, bit-exact with the reference's device
// sampler (opentpu/llm/generate.py:323-337 Sampler, :492-557 reference_pick at one slice) in the
// machine's fp32 arithmetic (every op RNE with flushed operands and results, canonical NaN).
//
// Two kernels on the caller's stream:
//   sample_blocks  16 lanes per block of 64 logits: l = ftz(logit), the soft cap
//                  2c recip(1 + exp2(l k1)) - c when asked, the repetition penalty
//                  fmin(l pa, l pb) when asked; the block's l to the work area, its maximum
//                  (total order) to bm, and each 16 blocks' maximum to sbm.
//   sample_pick    one workgroup of 256 threads:
//                  A. the n = min(k, nb) blocks with the largest maxima, as n rounds of
//                     "argmax (ties: the first), knock out to -inf" would take them;
//                  B. the same over the km x 64 candidates (those blocks' logits in pick order,
//                     -inf past them): the k values and ids;
//                  C. p = exp2((v - v0) itemp), cum by the 64-partial folding tree, top-p's
//                     kept prefix, and per uniform u the pick min(km - #{cum > u' zk}, #kept - 1).
// Selections.  The n largest by (key, then the lower position) of a list lie in the n largest
// of its groups (contiguous runs) ranked by their maxima the same way: a group outside those
// has n groups above it, each holding an entry above every entry of it.  So A selects 16-block
// groups (sbm) and then blocks among the chosen groups' blocks; B selects 16-candidate groups
// and then candidates among theirs.  The n chosen groups' maxima are n entries, so the second
// step drops every entry below the least of them before it ranks.  A selection of n among at
// most 1024 ranks each remaining entry by the number of remaining composites (key << 32 |
// ~position, all distinct) above its own: rank r < n is knock-out slot r.  Knock-out can take a position
// twice once everything left is -inf or below: the rounds past the m entries above -inf
// (m >= 1) all take the first position among the taken ones and the -inf ones, with value
// -inf; that is applied to the sorted list (only then is the first -inf position looked up).
#include <climits>
#include <mutex>

#include "otpu_common.h"

namespace otpu {

constexpr int SBLK = 64;                  // logits a block
constexpr int SKMAX = 64;                 // the largest top-k
constexpr int SNT = 256;                  // sample_pick's threads
constexpr int SRMAX = 4;                  // entries a thread in a selection (at most 1024)
constexpr int SGRP = 16;                  // a selection group: 16 blocks, or 16 candidates
constexpr int SRB = 16;                   // candidates a thread in B's direct selection (4096 / 256)
constexpr int NB_MAX = SRMAX * SNT * SGRP;   // blocks (16384: a vocabulary of 1M)
constexpr uint32_t KEY_NINF = 0x007FFFFFu;   // fkey(-inf)

// 2^f on [0, 1): the machine's degree-7 polynomial (fp32 coefficients, Horner from C7 down)
__device__ __forceinline__ float isa_exp2(float x) {
    const float C[8] = {__uint_as_float(0x3F800000u), __uint_as_float(0x3F317218u), __uint_as_float(0x3E75FDE9u),
                        __uint_as_float(0x3D63593Eu), __uint_as_float(0x3C1D8534u), __uint_as_float(0x3AAFE2F6u),
                        __uint_as_float(0x3916C07Cu), __uint_as_float(0x37B3C7D6u)};
    x = fin(ftz(x));
    const uint32_t kx = fkey_f(x);
    const bool lo = fkey_f(-126.0f) > kx;             // x < -126
    const bool hi = !(fkey_f(128.0f) > kx);           // x >= 128, or NaN
    const float xf = (!lo && !hi) ? x : 0.0f;
    const int i = (int)floorf(xf);
    const float f = fsub(xf, (float)i);
    float p = C[7];
#pragma unroll
    for (int c = 6; c >= 0; --c) p = fadd(fmul(p, f), C[c]);
    const float r = __uint_as_float((uint32_t)((int32_t)fbits(p) + i * (1 << 23)));
    return lo ? 0.0f : (hi ? __uint_as_float(0x7F800000u) : r);
}

// the machine's fmin / fmax: the total order of flushed values
__device__ __forceinline__ float tmin(float a, float b) {
    a = ftz(a);
    b = ftz(b);
    return fkey_f(b) > fkey_f(a) ? a : b;
}
__device__ __forceinline__ float tmax(float a, float b) {
    a = ftz(a);
    b = ftz(b);
    return fkey_f(a) > fkey_f(b) ? a : b;
}
__device__ __forceinline__ float step01(float x) { return tmin(tmax(fmul(x, 0x1p126f), 0.0f), 1.0f); }

struct SampleArgs {
    const float* logits;
    int V, nb;
    int vec4;                     // logits 16-byte aligned and V a multiple of 4: float4 loads
    const float* pa;              // penalty factors (NULL: none)
    const float* pb;
    int cap;                      // soft cap on
    float k1, k2, k3;             // -2 log2(e) / c, 2c, c
    int k, km;
    float itemp, top_p;
    const float* u;
    int nu;
    float* lg;                    // work: nb x 64 transformed logits
    float* bm;                    // work: nb block maxima
    float* sbm;                   // work: ceil(nb / 16) maxima of 16 blocks
    float* vs;                    // work: km candidate values
    int32_t* si;                  // work: km candidate ids
    int32_t* ids;                 // out: nu ids
    int32_t* status;              // out: 0, or 1 (top-p keeps no token)
};

__device__ __forceinline__ float sample_logit(const SampleArgs& a, int i, float l) {
    l = ftz(l);
    if (a.cap) l = fsub(fmul(recip(fadd(isa_exp2(fmul(l, a.k1)), 1.0f)), a.k2), a.k3);
    if (a.pa) l = tmin(fmul(l, a.pa[i]), fmul(l, a.pb[i]));
    return l;
}

// 16 lanes a block of 64 logits (4 each), 4 blocks a wave, 16 blocks a workgroup
__global__ __launch_bounds__(256) void sample_blocks(SampleArgs a) {
    const int lane = threadIdx.x & 63;
    const int blk = blockIdx.x * 16 + (threadIdx.x >> 4);
    const bool ok = blk < a.nb;
    const int i0 = blk * SBLK + 4 * (lane & 15);
    float l[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) l[j] = __uint_as_float(0xFF800000u);   // -inf past V
    if (ok && i0 + 3 < a.V && a.vec4) {          // (logits 16-byte aligned and V a multiple of 4)
        const float4 v = *reinterpret_cast<const float4*>(a.logits + i0);
        l[0] = v.x;
        l[1] = v.y;
        l[2] = v.z;
        l[3] = v.w;
#pragma unroll
        for (int j = 0; j < 4; ++j) l[j] = sample_logit(a, i0 + j, l[j]);
    } else if (ok) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (i0 + j < a.V) l[j] = sample_logit(a, i0 + j, a.logits[i0 + j]);
    }
    uint32_t kv = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) kv = max(kv, fkey_f(l[j]));
    if (ok) *reinterpret_cast<float4*>(a.lg + i0) = make_float4(l[0], l[1], l[2], l[3]);
    kv = wave_max_u32(kv, 16);
    if (ok && (lane & 15) == 0) a.bm[blk] = unkey(kv);
    // the workgroup's 16 blocks' maximum (blocks past nb hold key 0, below every real key)
    __shared__ uint32_t wmax[4];
    kv = ok ? kv : 0u;
    kv = max(kv, __shfl_xor(kv, 16, 64));
    kv = max(kv, __shfl_xor(kv, 32, 64));
    if (lane == 0) wmax[threadIdx.x >> 6] = kv;
    __syncthreads();
    if (threadIdx.x == 0) a.sbm[blockIdx.x] = unkey(max(max(wmax[0], wmax[1]), max(wmax[2], wmax[3])));
}

struct SelShared {
    uint64_t cand[SRMAX * SNT];       // a selection's entries at or above its bound: key << 32 | ~position
    int wtot[SNT / 64];
    int first_ninf;
    uint32_t skey[SKMAX];             // the n selected in knock-out order
    int spos[SKMAX];
};

// inclusive prefix sum over the wave: DPP row shifts 1, 2, 4, 8, then row 0's / 2's last lane
// into rows 1 / 3 and lane 31 into rows 2 and 3 (shifted-in lanes read 0)
__device__ __forceinline__ int wave_scan(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);
    return v;
}

// The n (1 <= n <= min(64, count)) largest of count (<= 256 RM) entries by (key, then the lower
// position), in that order, into S.skey / S.spos[0, n).  Thread t holds the keys of entries
// t R .. t R + R - 1 in kk (R = ceil(count / 256) <= RM); pos(p) is entry p's position
// (distinct).  lo is a key that at least n entries reach (0: no bound), so no entry below it is
// among the n.  The entries at or above lo are packed into S.cand; each one's rank is the number
// of packed composites above its own, and the composites are distinct, so the ranks below n are
// the n slots.  Returns false, having written nothing, when more than 1024 entries reach lo
// (never for count <= 1024).  Every thread calls it.
template <int RM, class PosFn>
__device__ bool select_top(int count, int n, const uint32_t (&kk)[RM], int R, uint32_t lo, PosFn pos,
                           SelShared& S) {
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    int mine = 0;
#pragma unroll
    for (int r = 0; r < RM; ++r) mine += (r < R && t * R + r < count && kk[r] >= lo) ? 1 : 0;
    const int incl = wave_scan(mine);
    if (lane == 63) S.wtot[w] = incl;
    if (t == 0) S.first_ninf = INT_MAX;
    __syncthreads();
    int off = incl - mine;
    for (int v = 0; v < w; ++v) off += S.wtot[v];
    const int c = S.wtot[0] + S.wtot[1] + S.wtot[2] + S.wtot[3];
    if (c > SRMAX * SNT) {                            // uniform; S.wtot is free again past the barrier
        __syncthreads();
        return false;
    }
#pragma unroll
    for (int r = 0; r < RM; ++r) {
        const int p = t * R + r;
        if (r < R && p < count && kk[r] >= lo) S.cand[off++] = ((uint64_t)kk[r] << 32) | (uint32_t)~(uint32_t)pos(p);
    }
    __syncthreads();
    for (int i = t; i < c; i += SNT) {
        const uint64_t me = S.cand[i];
        int rk = 0;
#pragma unroll 8
        for (int j = 0; j < c; ++j) rk += S.cand[j] > me ? 1 : 0;
        if (rk < n) {
            S.skey[rk] = (uint32_t)(me >> 32);
            S.spos[rk] = (int)~(uint32_t)me;
        }
    }
    __syncthreads();
    return true;
}

// The knock-out rule's corner on S.skey / S.spos[0, n) (knock-out order): the rounds past the
// m entries above -inf (m >= 1) take, with value -inf, the first position among the m taken
// ones and the -inf ones.  ninf(): a per-thread part of the first position holding -inf in the
// whole list (INT_MAX if none), asked only when m < n.  Every thread calls it.
template <class NinfFn>
__device__ void ninf_corner(int n, NinfFn ninf, SelShared& S) {
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    int m = __popcll(__ballot(lane < n && S.skey[lane] > KEY_NINF));   // the same in every wave
    m = m < 1 ? 1 : m;
    if (m < n) {                                      // uniform
        int fm = ninf();
        for (int o = 32; o > 0; o >>= 1) fm = min(fm, __shfl_xor(fm, o, 64));
        if (lane == 0 && fm != INT_MAX) atomicMin(&S.first_ninf, fm);
        __syncthreads();
        if (w == 0) {
            int rmin = lane < m ? S.spos[lane] : INT_MAX;
            for (int o = 32; o > 0; o >>= 1) rmin = min(rmin, __shfl_xor(rmin, o, 64));
            rmin = min(rmin, S.first_ninf);
            __builtin_amdgcn_wave_barrier();
            if (lane >= m && lane < n) {
                S.skey[lane] = KEY_NINF;
                S.spos[lane] = rmin;
            }
        }
        __syncthreads();
    }
}

// the 64-partial folding tree over x[0 .. 63] (partial c = +0 + x[c]): first half plus second
__device__ __forceinline__ float fold64(float (&x)[64]) {
#pragma unroll
    for (int h = 32; h > 0; h >>= 1)
#pragma unroll
        for (int c = 0; c < h; ++c) x[c] = fadd(x[c], x[c + h]);
    return x[0];
}

__global__ __launch_bounds__(SNT) void sample_pick(SampleArgs a) {
    __shared__ SelShared S;
    __shared__ int grp[SKMAX];
    __shared__ int qA[SKMAX];
    __shared__ float cum[SKMAX], sv[SKMAX];
    __shared__ int sid[SKMAX];
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const float u_first = a.nu > 0 ? a.u[0] : 0.0f;    // (its load overlaps the selections)
    const int nb = a.nb, nsb = (nb + SGRP - 1) / SGRP;
    const int nA = a.k < nb ? a.k : nb;
    uint32_t kk[SRMAX];
    // A1: the nA largest groups of 16 blocks (by sbm); loA: the least of their maxima when they
    // are nA groups (each holds a block at or above it), else 0
    const int gA = nA < nsb ? nA : nsb;
    uint32_t loA = 0u;
    {
        const int R = (nsb + SNT - 1) / SNT;
#pragma unroll
        for (int r = 0; r < SRMAX; ++r) {
            const int p = t * R + r;
            kk[r] = (r < R && p < nsb) ? fkey_f(a.sbm[p]) : 0u;
        }
        if (gA < nsb) {
            select_top(nsb, gA, kk, R, 0u, [](int p) { return p; }, S);
            if (t < gA) grp[t] = S.spos[t];
            loA = S.skey[gA - 1];
        } else if (t < gA) {
            grp[t] = t;
        }
        __syncthreads();
    }
    // A2: the nA largest blocks among the chosen groups' (positions: block ids), in order
    {
        const int cnt = gA * SGRP, R = (cnt + SNT - 1) / SNT;
#pragma unroll
        for (int r = 0; r < SRMAX; ++r) {
            const int p = t * R + r;
            const int b = (r < R && p < cnt) ? grp[p >> 4] * SGRP + (p & 15) : nb;
            kk[r] = b < nb ? fkey_f(a.bm[b]) : 0u;        // blocks past nb: below every key
        }
        select_top(cnt, nA, kk, R, loA, [](int p) { return grp[p >> 4] * SGRP + (p & 15); }, S);
        const float* bm = a.bm;
        ninf_corner(nA, [bm, nb, t]() {
            int f = INT_MAX;
            for (int b = t; b < nb; b += SNT)
                if (fkey_f(bm[b]) == KEY_NINF) f = min(f, b);
            return f;
        }, S);
        if (t < nA) qA[t] = S.spos[t];
        __syncthreads();
    }
    // B: the k largest of the km x 64 candidates (candidate c: block qA[c / 64]'s logit c % 64;
    // -inf past nA blocks).  B0, directly: when A took k blocks, their maxima are k candidates,
    // so none below the least of them is among the k.  When ties leave more than 1024 candidates
    // at or above it, B1 and B2 select groups of 16 candidates first.
    const float* lg = a.lg;
    const int nc = a.km * SBLK, ngc = nc / SGRP;
    bool done;
    {
        const uint32_t lo = nA == a.k ? S.skey[nA - 1] : 0u;
        const int R = nc / SNT;                       // 2 .. 16, even (km is a multiple of 8)
        uint32_t kb[SRB];
#pragma unroll
        for (int r = 0; r < SRB; r += 2) {
            // candidates c, c + 1 (c even) share a block; a thread's run may span two blocks
            const int c = t * R + r, j = c >> 6;
            uint32_t k0 = KEY_NINF, k1 = KEY_NINF;
            if (r < R && j < nA) {
                const float2 v = *reinterpret_cast<const float2*>(lg + qA[j] * SBLK + (c & 63));
                k0 = fkey_f(v.x);
                k1 = fkey_f(v.y);
            }
            kb[r] = k0;
            kb[r + 1] = k1;
        }
        done = select_top(nc, a.k, kb, R, lo, [](int p) { return p; }, S);
    }
    if (!done) {
        // B1: the k largest groups of 16 candidates by their maxima; loB: the least of those
        uint32_t loB;
        {
            // thread t: group t's maximum (ngc <= 256)
            uint32_t g = 0u;
            if (t < ngc) {
                const int j = t >> 2;
                g = KEY_NINF;
                if (j < nA) {
                    const float4* src = reinterpret_cast<const float4*>(lg + qA[j] * SBLK + 16 * (t & 3));
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float4 v = src[q];
                        g = max(g, max(max(fkey_f(v.x), fkey_f(v.y)), max(fkey_f(v.z), fkey_f(v.w))));
                    }
                }
            }
            kk[0] = g;
            select_top(ngc, a.k, kk, 1, 0u, [](int p) { return p; }, S);
            if (t < a.k) grp[t] = S.spos[t];
            loB = S.skey[a.k - 1];
            __syncthreads();
        }
        // B2: the k largest candidates among the chosen groups' (positions: candidate numbers)
        {
            const int cnt = a.k * SGRP, R = (cnt + SNT - 1) / SNT;
#pragma unroll
            for (int r = 0; r < SRMAX; ++r) {
                const int p = t * R + r;
                uint32_t key = 0u;
                if (r < R && p < cnt) {
                    const int c = grp[p >> 4] * SGRP + (p & 15), j = c >> 6;
                    key = j < nA ? fkey_f(lg[qA[j] * SBLK + (c & 63)]) : KEY_NINF;
                }
                kk[r] = key;
            }
            select_top(cnt, a.k, kk, R, loB, [](int p) { return grp[p >> 4] * SGRP + (p & 15); }, S);
        }
    }
    ninf_corner(a.k, [lg, nc, nA, t]() {
        int f = INT_MAX;
        for (int c = t; c < nc; c += SNT) {
            const int j = c >> 6;
            if (j >= nA || fkey_f(lg[qA[j] * SBLK + (c & 63)]) == KEY_NINF) f = min(f, c);
        }
        return f;
    }, S);
    if (w != 0) return;
    // C: one wave
    const int km = a.km;
    float v = __uint_as_float(0xFF800000u);
    int id = 0;
    if (lane < a.k) {
        v = unkey(S.skey[lane]);
        const int p = S.spos[lane], j = p >> 6;
        id = j < nA ? qA[j] * SBLK + (p & 63) : 0;
    }
    v = ftz(v);
    const float v0 = __shfl(v, 0, 64);
    const float p = isa_exp2(fmul(fsub(v, v0), a.itemp));
    sv[lane] = p;
    sid[lane] = id;
    // p is +0, a positive normal, or +inf / NaN (only when v0 is -inf or NaN).  Without the
    // last two every partial sum below is a non-negative normal or +0, so a plain IEEE add is
    // the machine's add (no denormal to flush, no NaN to canonicalize).
    const bool plain = __ballot(lane < km && !(p < __uint_as_float(0x7F800000u))) == 0;
    __builtin_amdgcn_wave_barrier();
    float c_i;                                        // cum[lane]
    if (plain) {
        float x[64];
#pragma unroll
        for (int c = 0; c < 64; ++c) x[c] = (c <= lane && c < km) ? sv[c] : 0.0f;
#pragma unroll
        for (int h = 32; h > 0; h >>= 1)
#pragma unroll
            for (int c = 0; c < h; ++c) x[c] = x[c] + x[c + h];
        c_i = x[0];
    } else {
        float x[64];
#pragma unroll
        for (int c = 0; c < 64; ++c) x[c] = c < km ? fadd(0.0f, fmul(c <= lane ? 1.0f : 0.0f, sv[c])) : 0.0f;
        c_i = fold64(x);
    }
    cum[lane] = c_i;
    __builtin_amdgcn_wave_barrier();
    const float total = cum[km - 1];
    const float prev = lane == 0 ? 0.0f : cum[lane - 1];
    const float kept = lane < km ? step01(fsub(fmul(total, a.top_p), prev)) : 0.0f;
    // zk: the largest kept cum (total order); the kept count's fold is an exact integer sum
    const float ck = lane < km ? fmul(c_i, kept) : 0.0f;
    uint32_t kz = lane < km ? fkey_f(ck) : 0u;
    kz = wave_max_u32(kz, 64);
    const float zk = unkey(kz);
    const int nkept = __popcll(__ballot(lane < km && kept == 1.0f));
    const float nk = (float)(nkept - 1);
    if (lane == 0) a.status[0] = kept == 0.0f ? 1 : 0;
    if (lane < km) {
        a.vs[lane] = v;
        a.si[lane] = id;
    }
    const float cap = 1.0f - 0x1p-24f;
    if (a.nu <= 16) {                                 // a uniform at a time: lane c tests cum[c]
        for (int j = 0; j < a.nu; ++j) {
            float uu = j == 0 ? u_first : a.u[j];
            uu = (uu != uu) ? uu : (uu < cap ? uu : cap);
            const float th = fmul(uu, zk);
            const float d = fsub(c_i, th);
            const int cnt = __popcll(__ballot(lane < km && (d >= 0x1p-126f || d != d)));
            const float le = fadd(fmul((float)cnt, -1.0f), (float)km);
            const int pk = (int)tmin(le, nk);
            if (lane == 0) a.ids[j] = sid[pk < 0 ? 0 : (pk > km - 1 ? km - 1 : pk)];
        }
        return;
    }
    for (int u0 = 0; u0 < a.nu; u0 += 64) {
        const int j = u0 + lane;
        float uu = a.u[j < a.nu ? j : a.nu - 1];
        uu = (uu != uu) ? uu : (uu < cap ? uu : cap);
        const float th = fmul(uu, zk);
        // #{c < km: step(cum[c] - th) = 1}: step is 1 for a difference of at least 2^-126 (the
        // flushed sub of a smaller one is 0) and for NaN; the sum of 0 / 1 terms is exact
        int cnt = 0;
        if (plain) {                                  // cum and th finite: the plain difference
#pragma unroll
            for (int c = 0; c < 64; ++c) cnt += (c < km && cum[c] - th >= 0x1p-126f) ? 1 : 0;
        } else {
#pragma unroll
            for (int c = 0; c < 64; ++c) {
                const float d = fsub(cum[c], th);
                cnt += (c < km && (d >= 0x1p-126f || d != d)) ? 1 : 0;
            }
        }
        const float le = fadd(fmul((float)cnt, -1.0f), (float)km);
        const int pk = (int)tmin(le, nk);
        if (j < a.nu) a.ids[j] = sid[pk < 0 ? 0 : (pk > km - 1 ? km - 1 : pk)];
    }
}

}  // namespace otpu

using namespace otpu;

// work area: vs [64] fp32, si [64] int32, lg [nb x 64], bm [nb], sbm [ceil(nb / 16)]
constexpr int64_t sample_work_bytes(int64_t V) {
    return 4 * (2 * SKMAX + (V + SBLK - 1) / SBLK * SBLK + (V + SBLK - 1) / SBLK
                + ((V + SBLK - 1) / SBLK + SGRP - 1) / SGRP);
}

extern "C" int64_t otpu_sample_work_bytes(int V) { return sample_work_bytes(V); }

// otpu_sample_static's work area: one per device, in the library's own device memory, for
// vocabularies of at most SAMPLE_STATIC_VMAX (1,066,496 bytes); every call overwrites all of
// the area it reads before reading it, so nothing is cleared between calls
constexpr int SAMPLE_STATIC_VMAX = 262144;
constexpr int SCRATCH_DEVICES = 64;
static __device__ __align__(256) uint8_t scratch[sample_work_bytes(SAMPLE_STATIC_VMAX)];
static void* scratch_ptr[SCRATCH_DEVICES];
static std::mutex scratch_mu;

// the current device's address of `scratch`: the array's name is a host-side stand-in, so its
// device address is looked up once per device (hipGetSymbolAddress with that device current)
static int scratch_of_current_device(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return otpu_fail(OTPU_ENODEV, "sample_static: hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= SCRATCH_DEVICES) return otpu_fail(OTPU_ENODEV, "sample_static: device %d", dev);
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (!scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return otpu_fail(OTPU_ELAUNCH, "sample_static: hipGetSymbolAddress: %s", hipGetErrorString(e));
        scratch_ptr[dev] = p;
    }
    *out = scratch_ptr[dev];
    return OTPU_OK;
}

static int sample_launch(const float* logits, int V, const float* pa, const float* pb, double softcap, int k,
                         float itemp, float top_p, const float* u, int nu, void* work, int32_t* ids,
                         int32_t* status, otpu_stream_t stream) {
    if (V < 1 || (int64_t)V > (int64_t)NB_MAX * SBLK)
        return otpu_fail(OTPU_EINVAL, "sample: vocabulary %d (1 .. %lld)", V, (long long)NB_MAX * SBLK);
    if (k < 1 || k > SKMAX) return otpu_fail(OTPU_EINVAL, "sample: top_k %d (1 .. %d)", k, SKMAX);
    if (!logits || !u || nu < 0 || !work || !ids || !status || ((pa == nullptr) != (pb == nullptr)))
        return otpu_fail(OTPU_EINVAL, "sample: missing operand (pa and pb go together)");
    if (((uintptr_t)work & 15) || ((uintptr_t)logits & 3))
        return otpu_fail(OTPU_EALIGN, "sample: work 16-byte, logits 4-byte aligned");
    SampleArgs a;
    a.logits = logits;
    a.V = V;
    a.vec4 = (V & 3) == 0 && ((uintptr_t)logits & 15) == 0;
    a.nb = (V + SBLK - 1) / SBLK;
    a.pa = pa;
    a.pb = pb;
    a.cap = softcap != 0.0;
    // the soft cap's constants, rounded to fp32 from double as the reference rounds them
    const double log2e = 1.0 / 0.69314718055994530942;
    a.k1 = a.cap ? (float)(-2.0 * log2e / softcap) : 0.0f;
    a.k2 = (float)(2.0 * softcap);
    a.k3 = (float)softcap;
    a.k = k;
    a.km = (k + 7) / 8 * 8;
    a.itemp = itemp;
    a.top_p = top_p;
    a.u = u;
    a.nu = nu;
    float* wf = (float*)work;
    a.vs = wf;
    a.si = (int32_t*)(wf + SKMAX);
    a.lg = wf + 2 * SKMAX;
    a.bm = a.lg + (int64_t)a.nb * SBLK;
    a.sbm = a.bm + a.nb;
    a.ids = ids;
    a.status = status;
    hipStream_t s = (hipStream_t)stream;
    sample_blocks<<<(a.nb + 15) / 16, 256, 0, s>>>(a);
    if (int rc = otpu_launch_check("sample_blocks")) return rc;
    sample_pick<<<1, SNT, 0, s>>>(a);
    return otpu_launch_check("sample_pick");
}

extern "C" int otpu_sample(const float* logits, int V, const float* pa, const float* pb, double softcap, int k,
                           float itemp, float top_p, const float* u, int nu, void* work, int32_t* ids,
                           int32_t* status, otpu_stream_t stream) {
    return sample_launch(logits, V, pa, pb, softcap, k, itemp, top_p, u, nu, work, ids, status, stream);
}

extern "C" int otpu_sample_static(const float* logits, int V, const float* pa, const float* pb, double softcap,
                                  int k, float itemp, float top_p, const float* u, int nu, int32_t* ids,
                                  int32_t* status, otpu_stream_t stream) {
    if (V > SAMPLE_STATIC_VMAX)
        return otpu_fail(OTPU_EINVAL, "sample_static: vocabulary %d above the static work area's %d (use otpu_sample)",
                         V, SAMPLE_STATIC_VMAX);
    void* work = nullptr;
    if (int rc = scratch_of_current_device(&work)) return rc;
    return sample_launch(logits, V, pa, pb, softcap, k, itemp, top_p, u, nu, work, ids, status, stream);
}
