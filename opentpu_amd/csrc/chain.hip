// The chained decode step of a stack of 4-bit quantized linears in one persistent launch: per
// layer MM qkv, MM o (on q), MM gate/up and the folded down projection on mul(g, u), each with
// the QACT of its input row in the prologue (the fused chain's four kernels a layer,
// `opentpu/kernels/mlp.py`, `Builder.dot` `opentpu/compiler.py:2686-2720`), bit for bit what
// otpu_mm_qin / otpu_mm_qin_fold compute one launch at a time.
//
// Why one launch.  In a chain of 112 dependent launches each costs ~5 us for 1-3 MB of weights:
// the dispatch gap, the input row's first read, and the code fetched cold each time.  Here one
// workgroup a CU runs every phase of the step; a phase hands its output row to the next as
// 8-byte entries (tag << 32 | fp32 bits) written with device-scope stores and read with
// device-scope loads (they bypass the XCDs' non-coherent L2s) until every entry carries the
// phase's tag: no fences, no counters, no grid barrier (one with agent-scope release / acquire
// costs ~30 us on MI355X, a hand-off ~2-3 us).  A phase issues its first weight rows before it
// waits, so the weights stream in during the hand-off.  Three entry rows rotate: phase i + 3
// writes the row phase i used.  Its writers have read all of phase i + 2, whose producers read
// all of phase i + 1 (o reads only q, but every workgroup with q/k/v rows also has o rows, which
// it writes after reading its q/k/v input; where a shape breaks that, o waits for k and v too),
// whose producers wrote their entries after reading phase i.  A workgroup without rows in a
// phase reads nothing in it.
//
// Tags.  Phase i of a call carries tag E * 4 L + i + 1, E the call's number: every workgroup
// keeps its own call counter (read at the start, advanced at the end), so graph replays of the
// same launch get fresh tags with no host involvement.  Every wait is bounded: one that runs out
// of polls sets the plan's error word and the step goes on (its output is then invalid).
//
// Phases' teams (compile-time): qkv and gate/up 32 lanes a row (K <= 1024), o 64 lanes
// (K <= 2048), the down projection 64 lanes with 2 pieces each (F <= 4096, F-chunks of 256).
#include <algorithm>
#include <cstddef>
#include <cstdlib>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "gemv_fold.h"

namespace otpu {

int qin_args(MMArgs* ap, int* Lp, const float* x, const float* xmul, const float* rscale, const float* cscale,
             int nsum, int64_t sum_stride, int K, int width, const uint8_t* w, int64_t rs, const uint8_t* ws,
             int64_t srs, int N, int fmt, int flags, int k0, float* out, int64_t ors, int64_t part_stride);
int fold_args(MMArgs* ap, int* Lp, const float* x, const float* xmul, const float* rscale, const float* cscale,
              int K, int width, const uint8_t* w, int64_t rs, const uint8_t* ws, int64_t srs, int N, int fmt, int flags,
              int k0, float* out);

constexpr int CHAIN_SLOTS = 4096;               // workgroups' call counters a plan holds
constexpr int CHAIN_SPIN = 1 << 16;             // polls a wait allows (~1 us each; OTPU_CHAIN_SPIN at plan time)
constexpr int CHAIN_PAD_LDS = 96 * 1024;        // dynamic LDS that keeps one workgroup a CU

// the phases' teams: T lanes a row, R rows a team (the prologue QACT holds K <= 32 T elements)
// q/k/v: 2 rows a team, so that 4096 rows (Qwen3-0.6B's and 1.7B's q, k and v) take the 256
// workgroups of one a CU with one row group each (4 rows a team: 128 workgroups of 32 rows, the
// other half of the chip idle in the phase, its rows 0.60 us; c4 297.3-298.4 -> 289.4-290.5 us a
// step, the Qwen3-1.7B shape 540-545 -> 523-526, interleaved on one box)
#ifndef OTPU_CHAIN_R
#define OTPU_CHAIN_R 2
#endif
constexpr int QKV_T = 32, QKV_R = OTPU_CHAIN_R;
#ifndef OTPU_CHAIN_OR
#define OTPU_CHAIN_OR 1
#endif
constexpr int O_T = 64, O_R = OTPU_CHAIN_OR;
constexpr int GU_T = 32, GU_R = 4;              // 4 rows a team, 2 teams a wave: the g / u pairs
// the fold: 64 lanes a row (1024 rows on 256 workgroups; 32 lanes with 128 workgroups measured
// 526 against 519 us a step)
#ifndef OTPU_CHAIN_DNT
#define OTPU_CHAIN_DNT 64
#endif
constexpr int DN_T = OTPU_CHAIN_DNT, DN_L = 128 / DN_T;  // F <= 4096: 128 pieces a row

struct ChainLayer {                              // the pointers of one layer (qkv, o, gu, down)
    const uint8_t* w[4];
    const uint8_t* ws[4];
    const float* cs[2];                          // CSCALE of the qkv and the gate/up QACTs (or NULL)
    float* out[4];                               // the phases' plain output rows
};

struct ChainPlan {                               // device memory: the header, then the layers
    MMArgs kind[4];                              // per phase: shape, strides and team (pointers per layer)
    const float* x0;                             // the step's input row
    const float* rnorm;                          // RSCALE factors [layers, 2] or NULL
    const ChainLayer* layer;
    uint64_t* ll[3];                             // the rotating entry rows
    uint32_t* calls;                             // call counter per workgroup
    uint32_t* err;
    int layers, fmt;
    int kv_wait;                                 // o waits for the k and v entries as well
    int norms;                                   // 0 no RSCALE / CSCALE factors, 1 some, 2 both in every layer
    int spin;                                    // polls a wait allows
    int combo;                                   // the phases' pieces a lane: 0 (LQ, LO, LF) = (1, 1, 2), 1 (2, 1, 4)
    int generic;                                 // never a shape's own copy (OTPU_GENERIC_COPIES at plan time)
    uint64_t* stamps;                            // [4 layers][grid][16] clock stamps (stamped build)
};

// rows of phase kind k the first iteration of workgroup b covers start at b * rows_per_wg(k)
__host__ __device__ constexpr int rows_per_wg(int k) {
    return k == 0 ? 4 * (64 / QKV_T) * QKV_R : k == 1 ? 4 * (64 / O_T) * O_R : k == 2 ? 4 * (64 / GU_T) * GU_R : 4 * (64 / DN_T);
}

union ChainLds {
    QinLds q;
    FoldLds f;
};

// FIXED: the default poll limit as a constant (folded into the waits: a limit read from the plan
// measured 16 us a step slower); the other copy serves plans with an OTPU_CHAIN_SPIN override.
// SH: a copy for one layer shape, its phases' K, pieces, rows and strides as constants (0: the
// generic copy, which reads them from the plan; OTPU_CHAIN_SHAPES=0 picks no shape copies)
#ifndef OTPU_CHAIN_SHAPES
#define OTPU_CHAIN_SHAPES 1
#endif
struct ChainShape {
    int K[4], P[4], N[4], rs[4], srs[4];         // per phase: qkv, o, gu, down
    int gu_pair, fold_c;                         // gate/up's pairs (F); the fold's sub-ranges a range
    int combo;                                   // the teams it runs (ChainPlan::combo)
};
// 4-bit rows of K / 2 bytes (K / 32 pieces), scale rows of 8 + 8 ceil(K / 256) bytes
constexpr ChainShape CHAIN_SHAPES[3] = {
    {},                                          // 0: the generic copy
    // 1: Qwen3-0.6B (hidden 1024, q_dim 2048, kv_dim 1024, F 3072: down chunks of 256)
    {{1024, 2048, 1024, 3072}, {32, 64, 32, 96}, {4096, 1024, 6144, 1024}, {512, 1024, 512, 1536},
     {40, 72, 40, 104}, 3072, 1, 0},
    // 2: Qwen3-1.7B (hidden 2048, q_dim 2048, kv_dim 1024, F 6144: down chunks of 768)
    {{2048, 2048, 2048, 6144}, {64, 64, 64, 192}, {4096, 2048, 12288, 2048}, {1024, 1024, 1024, 3072},
     {72, 72, 72, 200}, 6144, 3, 1},
};

// a field of the plan or of its layer table, read through the constant address space: the
// plan does not change while a step runs (only what its pointers point to), and the compiler,
// told so, reads it with scalar loads. Read as global memory after the step's first stores,
// which it cannot prove do not alias the plan, every phase re-read its fields with vector
// loads and waited for them before issuing its weights.
template <typename T>
__device__ __forceinline__ T cload(const T& r) {
#ifdef __HIP_DEVICE_COMPILE__
    return *(const __attribute__((address_space(4))) T*)&r;
#else
    return r;                                    // (the host pass of this device code)
#endif
}

// a phase's argument block, field by field through cload: a copy of the whole struct through
// the constant address space is lowered to vector loads, whose waits (vmcnt counts stores as
// well) also held each phase until the previous phase's output stores were acknowledged,
// before any of its weight loads issued.  Only the fields a phase uses are loaded.
__device__ __forceinline__ MMArgs cload_args(const MMArgs& r) {
    static_assert(sizeof(MMArgs) == 336, "every field of MMArgs copied below");
    MMArgs a;
    a.q = cload(r.q); a.ldq = cload(r.ldq); a.Sa = cload(r.Sa); a.da = cload(r.da); a.ldda = cload(r.ldda);
    a.M = cload(r.M); a.K = cload(r.K); a.w = cload(r.w); a.rs = cload(r.rs); a.ws = cload(r.ws);
    a.srs = cload(r.srs); a.N = cload(r.N); a.flags = cload(r.flags); a.k0 = cload(r.k0);
    a.alpha = cload(r.alpha); a.out = cload(r.out); a.ors = cload(r.ors); a.rmax_key = cload(r.rmax_key);
    a.acc_out = cload(r.acc_out); a.best = cload(r.best); a.base = cload(r.base); a.P = cload(r.P);
    a.T = cload(r.T); a.nseg = cload(r.nseg); a.q_bs = cload(r.q_bs); a.sa_bs = cload(r.sa_bs);
    a.da_bs = cload(r.da_bs); a.w_bs = cload(r.w_bs); a.ws_bs = cload(r.ws_bs); a.out_bs = cload(r.out_bs);
    a.k0_bs = cload(r.k0_bs); a.xin = cload(r.xin); a.xmul = cload(r.xmul); a.rscale = cload(r.rscale);
    a.cscale = cload(r.cscale); a.nsum = cload(r.nsum); a.sum_stride = cload(r.sum_stride);
    a.xin_bs = cload(r.xin_bs); a.ll_in = cload(r.ll_in); a.ll_out = cload(r.ll_out);
    a.tag_in = cload(r.tag_in); a.tag_out = cload(r.tag_out); a.err = cload(r.err); a.spin = cload(r.spin);
    a.ll_all = cload(r.ll_all); a.gu_pair = cload(r.gu_pair); a.fold_c = cload(r.fold_c);
    a.stamp = cload(r.stamp);
    return a;
}

// NORMS: 0 no RSCALE / CSCALE factors (constant NULLs), 1 some, 2 both in every layer (the
// prologues' tests of the factors drop out).  LQ, LO, LF: the 16-byte pieces a lane holds in
// the q/k/v and gate/up phases (32 lanes a row: hidden <= 1024 LQ), in o (64 lanes: q_dim <=
// 2048 LO) and in the fold (64 lanes: F <= 2048 LF)
template <int FMT, bool FIXED, int SH, int NORMS, int LQ = 1, int LO = 1, int LF = DN_L>
__device__ __forceinline__ void chain_run(const ChainPlan& P, ChainLds& lds) {
    constexpr int NRM = NORMS == 0 ? 1 : NORMS == 2 ? 2 : 0;    // the prologues' factor flag
    constexpr ChainShape S = CHAIN_SHAPES[SH];
    const int b = blockIdx.x;
    const uint32_t E = __hip_atomic_load(P.calls + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int NL = cload(P.layers);
    const uint32_t t0 = E * (uint32_t)(4 * NL);
    const ChainLayer* LY = cload(P.layer);
    for (int l = 0; l < NL; ++l) {
        const ChainLayer& ly = LY[l];
#pragma unroll 1
        for (int k = 0; k < 4; ++k) {
            const int i = 4 * l + k;
            MMArgs a = cload_args(P.kind[k]);
            // stamps: 0 phase start, 1 weights issued (the wait starts), 7 the input row's last
            // entry in, 2 the whole row in, 3 QACT done, 4 rows stored (6, 5: the QACT's barrier);
            // counts: 8 the last entry's polls that missed, 9 the rounds of re-polls after it
            uint64_t* const st = cload(P.stamps);
            a.stamp = st ? st + ((int64_t)i * gridDim.x + b) * 16 : nullptr;
            OTPU_STAMP(a, 0);
            // (a select on k, not S.N[k]: indexed by the loop's k, the table read became a switch, and
            // the compiler then copied the rest of the phase's code for each k)
            static_assert(S.N[1] == S.N[3], "o and the down projection both write the hidden row");
            if (SH) a.N = k == 0 ? S.N[0] : k == 2 ? S.N[2] : S.N[1];
            if (b * rows_per_wg(k) >= a.N) continue;     // no rows here: nothing to wait for
            a.w = cload(ly.w[k]);
            a.ws = cload(ly.ws[k]);
            a.out = cload(ly.out[k]);
            // what every chain phase shares, as constants (their branches drop out of the code):
            // weights with scale rows from block 0, one input row, no VOP MUL, no batch
            a.flags = 0;
            a.k0 = 0;
            a.M = 1;
            a.nsum = 1;
            a.xmul = nullptr;
            a.acc_out = nullptr;
            a.best = nullptr;
            a.rmax_key = nullptr;
            a.q_bs = a.sa_bs = a.da_bs = a.w_bs = a.ws_bs = a.out_bs = a.xin_bs = 0;
            a.k0_bs = 0;
            a.ll_in = i ? cload(P.ll[(i - 1) % 3]) : nullptr;
            a.xin = cload(P.x0);
            a.ll_out = cload(P.ll[i % 3]);
            a.tag_in = t0 + (uint32_t)i;
            a.tag_out = t0 + (uint32_t)i + 1;
            a.err = cload(P.err);
            a.spin = FIXED ? CHAIN_SPIN : cload(P.spin);
            a.ll_all = 0;
            a.rscale = nullptr;                          // (o and the fold have none)
            a.cscale = nullptr;
            if (NORMS != 0 && (k == 0 || k == 2)) {
                const float* const rn = cload(P.rnorm);
                a.rscale = rn ? rn + 2 * l + (k >> 1) : nullptr;
                a.cscale = cload(ly.cs[k >> 1]);
            }
            if (k == 1) {
                if (cload(P.kv_wait)) a.ll_all = cload(P.kind[0].N);   // o waits for k and v too
                if constexpr (SH != 0) { a.K = S.K[1]; a.P = S.P[1]; a.N = S.N[1]; a.ll_all = 0; a.rs = S.rs[1]; a.srs = S.srs[1]; }
                gemv_body<FMT, 1, LO, O_T, false, true, O_R, true, true, 1>(a, &lds.q);
            } else if (k == 3) {
                if constexpr (SH != 0) { a.K = S.K[3]; a.P = S.P[3]; a.N = S.N[3]; a.rs = S.rs[3]; a.srs = S.srs[3]; a.fold_c = S.fold_c; }
                // the next layer's table line read into the scalar cache during the fold, so that
                // its first phase finds its weight pointers there (the empty asm keeps the load;
                // its wait falls after the fold's own waits): ~1.5 us a step
                const uint8_t* const next = cload(LY[l + 1 < NL ? l + 1 : l].w[0]);
                fold_body<FMT, LF, DN_T, true>(a, &lds.f);
                asm volatile("" ::"s"(next));
            } else if (SH != 0 && (k == 0 || k == 2)) { // q/k/v and gate/up: their shape constants (one body when their teams match)
                if constexpr (SH != 0) {
                    static_assert(S.K[0] == S.K[2] && S.P[0] == S.P[2] && S.rs[0] == S.rs[2] && S.srs[0] == S.srs[2],
                                  "q/k/v and gate/up share their K");
                    a.K = S.K[0]; a.P = S.P[0]; a.rs = S.rs[0]; a.srs = S.srs[0];
                    a.N = k == 0 ? S.N[0] : S.N[2];
                    a.gu_pair = k == 0 ? 0 : S.gu_pair;
                }
                if (i == 0) gemv_body<FMT, 1, LQ, QKV_T, false, true, QKV_R, true, false, NRM>(a, &lds.q);   // plain x0
                else if (QKV_R != GU_R && k == 0) gemv_body<FMT, 1, LQ, QKV_T, false, true, QKV_R, true, true, NRM>(a, &lds.q);
                else gemv_body<FMT, 1, LQ, GU_T, false, true, GU_R, true, true, NRM>(a, &lds.q);
            } else if (k == 2) {
                gemv_body<FMT, 1, LQ, GU_T, false, true, GU_R, true, true, NRM>(a, &lds.q);
            } else if (i == 0) {                         // the step's first phase reads the plain x0
                gemv_body<FMT, 1, LQ, QKV_T, false, true, QKV_R, true, false, NRM>(a, &lds.q);
            } else {
                gemv_body<FMT, 1, LQ, QKV_T, false, true, QKV_R, true, true, NRM>(a, &lds.q);
            }
            OTPU_STAMP(a, 4);
            __syncthreads();                             // the next phase reuses the LDS
        }
    }
    if (threadIdx.x == 0) __hip_atomic_store(P.calls + b, E + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One kernel per compiled copy of the step, each its own function: as copies of one kernel, the
// code of each moved whenever another was added (the Qwen3-0.6B copy measured 358 -> 363 us a
// step with an unused copy compiled in beside it).  otpu_chain_plan picks the kernel
// (chain_pick) and otpu_chain_step launches it.
template <int FMT, bool FIXED, int SH, int NORMS, int LQ, int LO, int LF>
__global__ __launch_bounds__(256) void chain_kernel(const ChainPlan* plan) {
    __shared__ __align__(16) ChainLds lds;
    chain_run<FMT, FIXED, SH, NORMS, LQ, LO, LF>(*plan, lds);
}

// the plan's phases are shape sh's (dense 4-bit rows and scale rows, o waiting for q alone)
static bool is_shape(const ChainPlan& P, int sh) {
    const ChainShape& S = CHAIN_SHAPES[sh];
    if (P.combo != S.combo || P.kv_wait || P.kind[2].gu_pair != S.gu_pair || P.kind[3].fold_c != S.fold_c) return false;
    for (int k = 0; k < 4; ++k)
        if (P.kind[k].K != S.K[k] || P.kind[k].P != S.P[k] || P.kind[k].N != S.N[k] || P.kind[k].rs != S.rs[k] ||
            P.kind[k].srs != S.srs[k])
            return false;
    return true;
}

// the kernel for a plan: the format; the poll limit a constant (FIXED) or the plan's; a shape's
// own copy (Qwen3-0.6B's or Qwen3-1.7B's, unless OTPU_GENERIC_COPIES was set); the norm factors
// none / some / both in every layer; the phases' pieces a lane (combo)
template <int FMT, int SH, int LQ, int LF>
static const void* chain_pick_norms(int norms) {
    return norms == 0 ? (const void*)chain_kernel<FMT, true, SH, 0, LQ, 1, LF>
         : norms == 2 ? (const void*)chain_kernel<FMT, true, SH, 2, LQ, 1, LF>
                      : (const void*)chain_kernel<FMT, true, SH, 1, LQ, 1, LF>;
}
template <int FMT>
static const void* chain_pick_fmt(const ChainPlan& P) {
    const bool fixed = P.spin == CHAIN_SPIN;
    if (!fixed)
        return P.combo == 1 ? (const void*)chain_kernel<FMT, false, 0, 1, 2, 1, 4>
                            : (const void*)chain_kernel<FMT, false, 0, 1, 1, 1, DN_L>;
    if constexpr (FMT != OTPU_NVFP4) {          // (nvfp4's scale rows fit no shape of the table)
        const bool own = OTPU_CHAIN_SHAPES && !P.generic;
        if (own && is_shape(P, 2)) return chain_pick_norms<FMT, 2, 2, 4>(P.norms);
        if (own && is_shape(P, 1)) return chain_pick_norms<FMT, 1, 1, DN_L>(P.norms);
    }
    return P.combo == 1 ? chain_pick_norms<FMT, 0, 2, 4>(P.norms) : chain_pick_norms<FMT, 0, 1, DN_L>(P.norms);
}
static const void* chain_pick(const ChainPlan& P) {
    return P.fmt == OTPU_INT4 ? chain_pick_fmt<OTPU_INT4>(P)
         : P.fmt == OTPU_FP4  ? chain_pick_fmt<OTPU_FP4>(P)
                              : chain_pick_fmt<OTPU_NVFP4>(P);
}

static int64_t rnd256(int64_t x) { return (x + 255) / 256 * 256; }

struct ChainLayout {
    int64_t layer, calls, ll, rowb, total;
};
static ChainLayout chain_layout(int layers, int maxn) {
    ChainLayout c;
    c.layer = rnd256(sizeof(ChainPlan));
    c.calls = c.layer + rnd256((int64_t)layers * sizeof(ChainLayer));
    c.ll = c.calls + rnd256((int64_t)(CHAIN_SLOTS + 1) * 4);       // the call counters, then the error word
    c.rowb = rnd256((int64_t)maxn * 8);
    c.total = c.ll + 3 * c.rowb;
    return c;
}

}  // namespace otpu

using namespace otpu;

// The kernel each plan was built for, by the plan's device address (set by otpu_chain_plan; a
// plan rebuilt at the same address replaces its entry), with the dynamic LDS it launches with.
struct ChainPick {
    const void* fn;
    int pad;
};
static std::mutex chain_mu;
static std::unordered_map<uintptr_t, ChainPick> chain_picks;

// The step's dynamic LDS: one workgroup a CU (the padding leaves room for no second; without it
// the workgroups are resident all the same, some sharing a CU).
static int chain_pad(const void* fn) {
    return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, CHAIN_PAD_LDS) == hipSuccess
               ? CHAIN_PAD_LDS : 0;
}

// The step's workgroups wait on each other's rows, so all of them must be resident at once: the
// occupancy the compiled kernel allows with its LDS, times the CUs, must cover the grid of one
// workgroup a CU.  Checked when a plan is built (a plan serves the device current then); a device
// where it does not hold refuses the plan instead of running into the waits' time-out.
static int chain_resident_check(const char* what, const void* fn, int pad) {
    int per_cu = 0;
    const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 256, pad);
    if (e != hipSuccess) return otpu_fail(OTPU_ELAUNCH, "%s: occupancy query: %s", what, hipGetErrorString(e));
    // (one workgroup a CU: the grid is the CU count)
    if (per_cu < 1)
        return otpu_fail(OTPU_ELAUNCH,
                         "%s: the persistent step's %d workgroups cannot all be resident at once on this "
                         "device (%d a CU); use the launch-per-linear path", what, otpu_cu_count(), per_cu);
    return OTPU_OK;
}

extern "C" int64_t otpu_chain_plan_bytes(int layers, int hidden, int q_dim, int kv_dim, int F) {
    if (layers < 1 || hidden < 1 || q_dim < 1 || kv_dim < 0 || F < 1) return -1;
    const int maxn = std::max(std::max(q_dim + 2 * kv_dim, hidden), 2 * F);
    return chain_layout(layers, maxn).total;
}

extern "C" int otpu_chain_plan(int layers, int hidden, int q_dim, int kv_dim, int F, int down_width, int fmt,
                               const uint8_t* const* w, const int64_t* rs, const uint8_t* const* ws,
                               const int64_t* srs, const float* rnorm, const float* const* cscale, const float* x,
                               float* const* outs, void* plan, int64_t plan_bytes) {
    if (fmt != OTPU_INT4 && fmt != OTPU_FP4 && fmt != OTPU_NVFP4)
        return otpu_fail(OTPU_EINVAL, "chain_plan: int4x, fp4x6 or nvfp4 weights");
    if (layers < 1 || !w || !rs || !ws || !srs || !x || !outs || !plan)
        return otpu_fail(OTPU_EINVAL, "chain_plan: layers %d, NULL arrays", layers);
    // the compiled teams: combo 0 (pieces a lane 1, 1, 2) or 1 (2, 1, 4)
    const int combo = hidden <= 32 * QKV_T && q_dim <= 32 * O_T && F <= 32 * DN_T * DN_L ? 0
                      : hidden <= 2 * 32 * QKV_T && q_dim <= 32 * O_T && F <= 4 * 32 * DN_T ? 1 : -1;
    if (combo < 0 || F % 256 || q_dim % 32 || hidden % 32 || kv_dim < 0)
        return otpu_fail(OTPU_EINVAL, "chain_plan: hidden %d (<= %d), q_dim %d (<= %d), F %d (a multiple of 256, <= %d)",
                         hidden, 2 * 32 * QKV_T, q_dim, 32 * O_T, F, 4 * 32 * DN_T);
    if ((uintptr_t)plan % 256) return otpu_fail(OTPU_EALIGN, "chain_plan: plan 256-byte aligned");
    const int nq = q_dim + 2 * kv_dim;
    const int maxn = std::max(std::max(nq, hidden), 2 * F);
    const ChainLayout lay = chain_layout(layers, maxn);
    if (plan_bytes < lay.total)
        return otpu_fail(OTPU_EINVAL, "chain_plan: %lld bytes, the plan needs %lld", (long long)plan_bytes,
                         (long long)lay.total);
    if (otpu_cu_count() > CHAIN_SLOTS) return otpu_fail(OTPU_EINVAL, "chain_plan: more than %d CUs", CHAIN_SLOTS);
    // each phase kind checked and built as its one-launch entry point would (layer 0's
    // pointers); then every layer's pointers checked the same way
    const int Ns[4] = {nq, hidden, 2 * F, hidden}, Ks[4] = {hidden, q_dim, hidden, F};
    std::vector<ChainLayer> ly(layers);
    ChainPlan hp = {};
    for (int l = 0; l < layers; ++l) {
        for (int k = 0; k < 4; ++k) {
            const int j = 4 * l + k;
            if (!outs[j]) return otpu_fail(OTPU_EINVAL, "chain_plan: layer %d phase %d output NULL", l, k);
            if ((uintptr_t)outs[j] % 16) return otpu_fail(OTPU_EALIGN, "chain_plan: outputs 16-byte aligned");
            MMArgs a;
            int L = 1, rc;
            const float* cs = (k == 0 || k == 2) && cscale ? cscale[2 * l + (k >> 1)] : nullptr;
            const float* rsc = (k == 0 || k == 2) && rnorm ? rnorm + 2 * l + (k >> 1) : nullptr;
            if (k < 3)
                rc = qin_args(&a, &L, x, nullptr, rsc, cs, 1, 0, Ks[k], Ks[k], w[j], rs[j], ws[j], srs[j], Ns[k], fmt, 0,
                              0, outs[j], Ns[k], 0);
            else
                rc = fold_args(&a, &L, x, x, nullptr, nullptr, F, down_width, w[j], rs[j], ws[j], srs[j], hidden, fmt,
                               0, 0, outs[j]);
            if (rc) return rc;
            if (l > 0 && (rs[j] != rs[k] || srs[j] != srs[k]))
                return otpu_fail(OTPU_EINVAL, "chain_plan: layer %d phase %d row strides differ from layer 0's", l, k);
            if (l == 0) {
                a.T = k == 0 ? QKV_T : k == 1 ? O_T : k == 2 ? GU_T : DN_T;
                if (k == 2) a.gu_pair = F;                 // the fold reads g * u, F entries
                hp.kind[k] = a;
            }
            ly[l].w[k] = w[j];
            ly[l].ws[k] = ws[j];
            ly[l].out[k] = outs[j];
            if (k == 0 || k == 2) ly[l].cs[k >> 1] = cs;
        }
    }
    uint8_t* base = static_cast<uint8_t*>(plan);
    hp.x0 = x;
    hp.rnorm = rnorm;
    hp.layer = reinterpret_cast<const ChainLayer*>(base + lay.layer);
    hp.calls = reinterpret_cast<uint32_t*>(base + lay.calls);
    hp.err = hp.calls + CHAIN_SLOTS;
    hp.ll[0] = reinterpret_cast<uint64_t*>(base + lay.ll);
    hp.ll[1] = reinterpret_cast<uint64_t*>(base + lay.ll + lay.rowb);
    hp.ll[2] = reinterpret_cast<uint64_t*>(base + lay.ll + 2 * lay.rowb);
    // the rotation needs every workgroup with q/k/v rows to have o rows (see the top)
    {
        const int G = otpu_cu_count();
        const int wq = std::min(G, (nq + rows_per_wg(0) - 1) / rows_per_wg(0));
        const int wo = std::min(G, (hidden + rows_per_wg(1) - 1) / rows_per_wg(1));
        hp.kv_wait = wq > wo;
        if (hp.kv_wait && 2 * kv_dim > 2048)             // (ll_drain's entries: 8 a thread)
            return otpu_fail(OTPU_EINVAL, "chain_plan: o waits for k and v here, so 2 kv_dim must be <= 2048 (kv_dim %d)",
                             kv_dim);
    }
    hp.layers = layers;
    hp.fmt = fmt;
    hp.combo = combo;
    {
        bool any = rnorm != nullptr, all = rnorm != nullptr && cscale != nullptr;
        for (int j = 0; cscale && j < 2 * layers; ++j) {
            any = any || cscale[j] != nullptr;
            all = all && cscale[j] != nullptr;
        }
        hp.norms = all ? 2 : any ? 1 : 0;
    }
    // the waits' poll limit: OTPU_CHAIN_SPIN (0 .. 2^20) overrides it, e.g. to drive the timeout
    // path from the host in a test (every wait then gives up at once and sets the error word)
    hp.generic = getenv("OTPU_GENERIC_COPIES") != nullptr;
    hp.spin = CHAIN_SPIN;
    if (const char* e = getenv("OTPU_CHAIN_SPIN")) {
        const long v = strtol(e, nullptr, 10);
        if (v >= 0 && v <= (1 << 20)) hp.spin = (int)v;
    }
    // the kernel compiled for this plan, and whether its workgroups fit the device at once
    const ChainPick pick = {chain_pick(hp), 0};
    const ChainPick pk = {pick.fn, chain_pad(pick.fn)};
    if (int rc = chain_resident_check("chain_plan", pk.fn, pk.pad)) return rc;
    // synchronous copies: a plan is built once, outside any capture
    hipError_t e = hipMemset(base, 0, (size_t)lay.total);
    if (e == hipSuccess) e = hipMemcpy(base, &hp, sizeof(hp), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(base + lay.layer, ly.data(), sizeof(ChainLayer) * layers, hipMemcpyHostToDevice);
    if (e != hipSuccess) return otpu_fail(OTPU_ELAUNCH, "chain_plan: %s", hipGetErrorString(e));
    {
        std::lock_guard<std::mutex> g(chain_mu);
        chain_picks[(uintptr_t)plan] = pk;
    }
    return OTPU_OK;
}

extern "C" int otpu_chain_step(const void* plan, otpu_stream_t stream) {
    if (!plan || (uintptr_t)plan % 256) return otpu_fail(OTPU_EINVAL, "chain_step: plan NULL or misaligned");
    ChainPick pk = {nullptr, 0};
    {
        std::lock_guard<std::mutex> g(chain_mu);
        const auto it = chain_picks.find((uintptr_t)plan);
        if (it != chain_picks.end()) pk = it->second;
    }
    if (!pk.fn) return otpu_fail(OTPU_EINVAL, "chain_step: no plan built at %p by otpu_chain_plan in this process", plan);
    const ChainPlan* P = static_cast<const ChainPlan*>(plan);
    void* args[] = {&P};
    const hipError_t e = hipLaunchKernel(pk.fn, dim3((unsigned)otpu_cu_count()), dim3(256), args, (size_t)pk.pad,
                                         (hipStream_t)stream);
    if (e != hipSuccess) return otpu_fail(OTPU_ELAUNCH, "chain_step: %s", hipGetErrorString(e));
    return otpu_launch_check("chain_step");
}

extern "C" int otpu_chain_stamps(void* plan, uint64_t* stamps) {
#ifdef OTPU_PHASE_STAMPS
    if (!plan) return otpu_fail(OTPU_EINVAL, "chain_stamps: plan NULL");
    hipError_t e = hipMemcpy(static_cast<uint8_t*>(plan) + offsetof(ChainPlan, stamps), &stamps, sizeof(stamps),
                             hipMemcpyHostToDevice);
    if (e != hipSuccess) return otpu_fail(OTPU_ELAUNCH, "chain_stamps: %s", hipGetErrorString(e));
    return OTPU_OK;
#else
    (void)plan;
    (void)stamps;
    return otpu_fail(OTPU_EINVAL, "chain_stamps: a build without phase stamps (python -m opentpu_amd.build --stamps)");
#endif
}

extern "C" int otpu_chain_error(const void* plan, uint32_t* err) {
    if (!plan || !err) return otpu_fail(OTPU_EINVAL, "chain_error: NULL");
    ChainPlan hp;
    hipError_t e = hipMemcpy(&hp, plan, sizeof(hp), hipMemcpyDeviceToHost);
    if (e == hipSuccess) e = hipMemcpy(err, hp.err, 4, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return otpu_fail(OTPU_ELAUNCH, "chain_error: %s", hipGetErrorString(e));
    return OTPU_OK;
}
