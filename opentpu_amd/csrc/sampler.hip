// The sampled decode's pick after the LM head, on the GPU, bit-exact with the reference's device
// sampler (opentpu/llm/generate.py:323-337 Sampler, :492-557 reference_pick at one slice) in the
// machine's fp32 arithmetic (every op RNE with flushed operands and results, canonical NaN).
//
// Two kernels on the caller's stream:
//   sample_blocks  one wave per block of 64 logits: l = ftz(logit), the soft cap
//                  2c recip(1 + exp2(l k1)) - c when asked, the repetition penalty
//                  fmin(l pa, l pb) when asked; the block's l to the work area, its maximum
//                  (total order) to bm.
//   sample_pick    one workgroup of 1024 threads:
//                  A. the n = min(k, nb) blocks with the largest maxima, as n rounds of
//                     "argmax (ties: the first), knock out to -inf" would take them;
//                  B. the same over the km x 64 candidates (those blocks' logits in pick order,
//                     -inf past them): the k values and ids;
//                  C. p = exp2((v - v0) itemp), cum by the 64-partial folding tree, top-p's
//                     kept prefix, and per uniform u the pick min(km - #{cum > u' zk}, #kept - 1).
// The n largest are found without n rounds: a 4-pass radix select (8 bits a pass) finds the
// n-th largest key T; the keys above T and the first (by position) keys equal to T are the
// n; a rank sort by (key, -position) orders them.  Knock-out can take a position twice once
// everything left is -inf or below: the rounds past the m entries above -inf (m >= 1) all take
// the first position among the taken ones and the -inf ones, with value -inf; that is applied
// to the sorted list.
#include <climits>

#include "otpu_common.h"

namespace otpu {

constexpr int SBLK = 64;                  // logits a block
constexpr int SKMAX = 64;                 // the largest top-k
constexpr int SNT = 1024;                 // sample_pick's threads
constexpr int SRMAX = 16;                 // entries a thread in a selection (nb <= 16384)
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
    float* vs;                    // work: km candidate values
    int32_t* si;                  // work: km candidate ids
    int32_t* ids;                 // out: nu ids
    int32_t* status;              // out: 0, or 1 (top-p keeps no token)
};

__global__ __launch_bounds__(256) void sample_blocks(SampleArgs a) {
    const int lane = threadIdx.x & 63;
    const int blk = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (blk >= a.nb) return;                          // whole waves leave together
    const int i = blk * SBLK + lane;
    float l = __uint_as_float(0xFF800000u);           // -inf past V
    if (i < a.V) {
        l = ftz(a.logits[i]);
        if (a.cap) l = fsub(fmul(recip(fadd(isa_exp2(fmul(l, a.k1)), 1.0f)), a.k2), a.k3);
        if (a.pa) l = tmin(fmul(l, a.pa[i]), fmul(l, a.pb[i]));
    }
    a.lg[i] = l;
    uint32_t kv = fkey_f(l);
    const uint32_t best = wave_max_u32(kv, 64);
    if (lane == 0) a.bm[blk] = unkey(best);
}

struct SelShared {
    int hist[256];
    int wtot[SNT / 64];
    int digit, rem, cnt_gt, first_ninf;
    uint32_t key[SKMAX];
    int pos[SKMAX];
    uint32_t skey[SKMAX];
    int spos[SKMAX];
};

// The n (<= 64) entries that n knock-out rounds over keys kf(0 .. count-1) take, in order:
// S.skey / S.spos [0, n).  Every thread of the workgroup calls it.
template <class KeyFn>
__device__ void knock_select(int count, int n, KeyFn kf, SelShared& S) {
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int R = (count + SNT - 1) / SNT;
    uint32_t kk[SRMAX];
#pragma unroll
    for (int r = 0; r < SRMAX; ++r) {
        const int p = t * R + r;
        kk[r] = (r < R && p < count) ? kf(p) : 0u;
    }
    uint32_t prefix = 0, maskhi = 0;
    int remaining = n;
    for (int pass = 0; pass < 4; ++pass) {
        const int shift = 24 - 8 * pass;
        if (t < 256) S.hist[t] = 0;
        if (t == 0) {
            S.cnt_gt = 0;
            S.first_ninf = INT_MAX;
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < SRMAX; ++r) {
            const int p = t * R + r;
            if (r < R && p < count && (kk[r] & maskhi) == prefix) atomicAdd(&S.hist[(kk[r] >> shift) & 255], 1);
        }
        __syncthreads();
        if (w == 0) {                                 // lane l: bins 255-4l .. 252-4l
            int h[4], c = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                h[j] = S.hist[255 - 4 * lane - j];
                c += h[j];
            }
            int incl = c;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int y = __shfl_up(incl, o, 64);
                if (lane >= o) incl += y;
            }
            int acc = incl - c;                        // entries in higher bins
            if (acc < remaining && remaining <= incl) {
                for (int j = 0; j < 4; ++j) {
                    if (acc + h[j] >= remaining) {
                        S.digit = 255 - 4 * lane - j;
                        S.rem = remaining - acc;
                        break;
                    }
                    acc += h[j];
                }
            }
        }
        __syncthreads();
        prefix |= (uint32_t)S.digit << shift;
        maskhi |= 0xFFu << shift;
        remaining = S.rem;
    }
    const uint32_t T = prefix;
    const int c_gt = n - remaining;
    // the keys equal to T, by position: an exclusive scan of the per-thread counts
    int eqc = 0;
#pragma unroll
    for (int r = 0; r < SRMAX; ++r) {
        const int p = t * R + r;
        eqc += (r < R && p < count && kk[r] == T) ? 1 : 0;
    }
    int incl = eqc;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o, 64);
        if (lane >= o) incl += y;
    }
    if (lane == 63) S.wtot[w] = incl;
    __syncthreads();
    int rank = incl - eqc;
    for (int v = 0; v < w; ++v) rank += S.wtot[v];
#pragma unroll
    for (int r = 0; r < SRMAX; ++r) {
        const int p = t * R + r;
        if (!(r < R && p < count)) continue;
        if (kk[r] > T) {
            const int s = atomicAdd(&S.cnt_gt, 1);
            S.key[s] = kk[r];
            S.pos[s] = p;
        } else if (kk[r] == T) {
            if (rank < remaining) {
                S.key[c_gt + rank] = T;
                S.pos[c_gt + rank] = p;
            }
            ++rank;
        }
        if (kk[r] == KEY_NINF) atomicMin(&S.first_ninf, p);
    }
    __syncthreads();
    if (w == 0) {
        // rank sort by (key descending, position ascending)
        uint32_t mk = 0;
        int mp = 0, rk = 0;
        if (lane < n) {
            mk = S.key[lane];
            mp = S.pos[lane];
            const uint64_t me = ((uint64_t)mk << 32) | (uint32_t)~(uint32_t)mp;
            for (int j = 0; j < n; ++j) {
                const uint64_t o = ((uint64_t)S.key[j] << 32) | (uint32_t)~(uint32_t)S.pos[j];
                rk += o > me ? 1 : 0;
            }
        }
        // every lane has read S.key / S.pos before any lane writes the sorted list
        __builtin_amdgcn_wave_barrier();
        if (lane < n) {
            S.skey[rk] = mk;
            S.spos[rk] = mp;
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        // knock-out: past the m entries above -inf, the first of the taken and the -inf ones
        const uint32_t sk = lane < n ? S.skey[lane] : 0u;
        const int sp = lane < n ? S.spos[lane] : INT_MAX;
        const uint64_t above = __ballot(lane < n && sk > KEY_NINF);
        int m = __popcll(above);
        m = m < 1 ? 1 : m;
        if (m < n) {
            int rmin = lane < m ? sp : INT_MAX;
            for (int o = 32; o > 0; o >>= 1) rmin = min(rmin, __shfl_xor(rmin, o, 64));
            rmin = min(rmin, S.first_ninf);
            if (lane >= m && lane < n) {
                S.skey[lane] = KEY_NINF;
                S.spos[lane] = rmin;
            }
        }
    }
    __syncthreads();
}

// the 64-partial folding tree over x[0 .. 63] (partial c = +0 + x[c]): first half plus second
__device__ __forceinline__ float fold64(float* x) {
    for (int h = 32; h > 0; h >>= 1)
        for (int c = 0; c < h; ++c) x[c] = fadd(x[c], x[c + h]);
    return x[0];
}

__global__ __launch_bounds__(SNT) void sample_pick(SampleArgs a) {
    __shared__ SelShared S;
    __shared__ int qA[SKMAX];
    __shared__ float cum[SKMAX], sv[SKMAX];
    __shared__ int sid[SKMAX];
    __shared__ float sNk;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int nA = a.k < a.nb ? a.k : a.nb;
    const float* bm = a.bm;
    knock_select(a.nb, nA, [bm](int p) { return fkey_f(bm[p]); }, S);
    if (t < nA) qA[t] = S.spos[t];
    __syncthreads();
    const float* lg = a.lg;
    const int nc = a.km * SBLK;
    knock_select(nc, a.k, [lg, nA](int p) {
        const int j = p >> 6;
        return j < nA ? fkey_f(lg[qA[j] * SBLK + (p & 63)]) : KEY_NINF;
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
    __builtin_amdgcn_wave_barrier();
    float x[64];
    float c_i = 0.0f;
    if (lane < km) {
        for (int c = 0; c < 64; ++c) x[c] = c < km ? fadd(0.0f, fmul(c <= lane ? 1.0f : 0.0f, sv[c])) : 0.0f;
        c_i = fold64(x);
        cum[lane] = c_i;
    }
    __builtin_amdgcn_wave_barrier();
    const float total = cum[km - 1];
    const float prev = lane == 0 ? 0.0f : (lane < km ? cum[lane - 1] : 0.0f);
    const float kept = lane < km ? step01(fsub(fmul(total, a.top_p), prev)) : 0.0f;
    // zk: the largest kept cum (total order); #kept - 1
    const float ck = lane < km ? fmul(c_i, kept) : 0.0f;
    uint32_t kz = lane < km ? fkey_f(ck) : 0u;
    kz = wave_max_u32(kz, 64);
    const float zk = unkey(kz);
    sv[lane] = kept;
    __builtin_amdgcn_wave_barrier();
    if (lane == 0) {
        for (int c = 0; c < 64; ++c) x[c] = c < km ? fadd(0.0f, sv[c]) : 0.0f;
        sNk = fsub(fold64(x), 1.0f);
        a.status[0] = sv[0] == 0.0f ? 1 : 0;
    }
    if (lane < km) {
        a.vs[lane] = v;
        a.si[lane] = id;
    }
    __builtin_amdgcn_wave_barrier();
    const float nk = sNk;
    for (int u0 = 0; u0 < a.nu; u0 += 64) {
        const int j = u0 + lane;
        if (j >= a.nu) break;
        float uu = a.u[j];
        const float cap = 1.0f - 0x1p-24f;
        uu = (uu != uu) ? uu : (uu < cap ? uu : cap);
        const float th = fmul(uu, zk);
        for (int c = 0; c < 64; ++c) x[c] = c < km ? fadd(0.0f, step01(fsub(cum[c], th))) : 0.0f;
        const float le = fadd(fmul(fold64(x), -1.0f), (float)km);
        const int pk = (int)tmin(le, nk);
        a.ids[j] = sid[pk < 0 ? 0 : (pk > km - 1 ? km - 1 : pk)];
    }
}

}  // namespace otpu

using namespace otpu;

extern "C" int64_t otpu_sample_work_bytes(int V) {
    const int64_t nb = ((int64_t)V + SBLK - 1) / SBLK;
    return 4 * (nb * SBLK + nb + 2 * SKMAX);
}

extern "C" int otpu_sample(const float* logits, int V, const float* pa, const float* pb, double softcap, int k,
                           float itemp, float top_p, const float* u, int nu, void* work, int32_t* ids,
                           int32_t* status, otpu_stream_t stream) {
    if (V < 1 || V > SRMAX * SNT * SBLK)
        return otpu_fail(OTPU_EINVAL, "sample: vocabulary %d (1 .. %d)", V, SRMAX * SNT * SBLK);
    if (k < 1 || k > SKMAX) return otpu_fail(OTPU_EINVAL, "sample: top_k %d (1 .. %d)", k, SKMAX);
    if (!logits || !u || nu < 0 || !work || !ids || !status || ((pa == nullptr) != (pb == nullptr)))
        return otpu_fail(OTPU_EINVAL, "sample: missing operand (pa and pb go together)");
    if (((uintptr_t)work & 3) || ((uintptr_t)logits & 3))
        return otpu_fail(OTPU_EALIGN, "sample: 4-byte aligned operands");
    SampleArgs a;
    a.logits = logits;
    a.V = V;
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
    a.lg = wf;
    a.bm = wf + (int64_t)a.nb * SBLK;
    a.vs = a.bm + a.nb;
    a.si = (int32_t*)(a.vs + SKMAX);
    a.ids = ids;
    a.status = status;
    hipStream_t s = (hipStream_t)stream;
    sample_blocks<<<(a.nb + 3) / 4, 256, 0, s>>>(a);
    if (int rc = otpu_launch_check("sample_blocks")) return rc;
    sample_pick<<<1, SNT, 0, s>>>(a);
    return otpu_launch_check("sample_pick");
}
