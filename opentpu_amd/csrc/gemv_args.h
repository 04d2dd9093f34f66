// Shared by the decode GEMV sources: the argument block of one MM launch, the register-
// tiling constants (also used on the host to pick a launch shape) and the per-format launchers,
// each instantiated in its own translation unit (gemv_int8.hip, gemv_int4.hip, gemv_fp4.hip,
// gemv_nvfp4.hip) so the four compile in parallel.
#pragma once
#include "otpu_common.h"

namespace otpu {

// threads of every kernel over the GEMV bodies (their __launch_bounds__ and launches): a
// constant, since blockDim.x is read from the dispatch packet with a load and a wait
constexpr int GEMV_THREADS = 256;
constexpr int LM_WORDS = 64;      // the LM head's running maxima (one line each)
constexpr int LM_STRIDE = 32;     // u64 words from one to the next (256 bytes)
constexpr int LMAX = 8;            // pieces per lane held in registers at once (a segment of a row)
constexpr int KMAX_MM = 32640;     // K an MM takes: blocks of 128 below 256 (isa.py's 8-bit KB field)

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
    uint64_t* best;                // LM head: the maxima of (key << 32 | ~index), LM_WORDS words
                                   // LM_STRIDE apart (workgroup b raises word b % LM_WORDS)
    int64_t base;                  // LM head: index of row 0
    int P, T;                      // 16-byte pieces per row, lanes per row (team)
    int nseg;                      // segments a row is walked in: T * L pieces each (0 or 1: one)
    // batch strides (elements of each pointer's type; bytes for w / ws; blocks for k0)
    int64_t q_bs, sa_bs, da_bs, w_bs, ws_bs, out_bs;
    int k0_bs;
    // QACT in the prologue (one activation row): the fp32 row xin (problem b at + b * xin_bs),
    // the fold of nsum rows sum_stride apart, times xmul when given, then times rscale[0]
    // (RSCALE) and cscale[column] (CSCALE) when given
    const float* xin;
    const float* xmul;
    const float* rscale;
    const float* cscale;
    int nsum;
    int64_t sum_stride, xin_bs;
    // the persistent chain's hand-off rows (LL kernels only): 8-byte entries tag << 32 | fp32
    // bits, written with device-scope stores and polled with device-scope loads until every
    // entry a workgroup needs carries the phase's tag (no fences, no counters)
    const uint64_t* ll_in;         // input entries (NULL: the plain row xin)
    uint64_t* ll_out;              // output entries, besides the plain row out
    uint32_t tag_in, tag_out;
    uint32_t* err;                 // set when a wait runs out of polls
    int spin;                      // polls a wait allows (~1 us each)
    int ll_all;                    // entries of the input row to wait for when more than K (see ll_drain)
    int gu_pair;                   // F: gate/up rows taken in g / u pairs, the entries g * u (see gemv_body)
    int fold_c;                    // the folded down projection: 256-column sub-ranges a QACT range (0: 1)
    uint64_t* stamp;               // the phase's clock stamps (builds with OTPU_PHASE_STAMPS only)
};

// a clock stamp (100 MHz wall clock) of the persistent chain's phase breakdown, by the first
// thread, compiled only into the stamped build (python -m opentpu_amd.build --stamps)
#ifdef OTPU_PHASE_STAMPS
#define OTPU_STAMP(a, j)                                                                           \
    do {                                                                                           \
        if ((a).stamp && threadIdx.x == 0) (a).stamp[j] = __builtin_amdgcn_s_memrealtime();        \
    } while (0)
#define OTPU_STAMP_COUNT(a, j, n)                                                                  \
    do {                                                                                           \
        if ((a).stamp && threadIdx.x == 0) (a).stamp[j] = (uint64_t)(n);                           \
    } while (0)
#else
#define OTPU_STAMP(a, j) \
    do {                 \
    } while (0)
#define OTPU_STAMP_COUNT(a, j, n) \
    do {                          \
    } while (0)
#endif

constexpr int QIN_KMAX = 4096;     // columns the persistent chain's and the fold's prologue QACT hold in LDS
constexpr int QIN_KBIG = 16384;    // columns otpu_mm_qin's prologue QACT holds in LDS (its widest kernels)
constexpr int FOLD_KMAX = 8192;    // columns (F) the folded down projection's prologue QACT holds in LDS
constexpr int QIN_NSUM_MAX = 16;   // partial rows the prologue folds

// rows a team takes per iteration: 8 rows' loads in flight per wave for one activation row
// with one piece a lane (measured on MI355X: 16 the same for the 80-problem launches, 8 faster
// for small grids), 4 when that still leaves CUs idle (R_SMALL); 4 a team with four or more
// pieces a lane (the LM head: 105.4 against 106.0 us at 8 over three paired runs, 4% over 2);
// fewer as activation rows add sums to carry
#ifndef OTPU_GEMV_R1
#define OTPU_GEMV_R1 8
#endif
#ifndef OTPU_GEMV_NT
#define OTPU_GEMV_NT 1
#endif
#ifndef OTPU_GEMV_R2
#define OTPU_GEMV_R2 2
#endif
#ifndef OTPU_GEMV_R4
#define OTPU_GEMV_R4 4
#endif
constexpr int rows_per_team_rt(int L, int mr) {
    return L >= 4 ? (OTPU_GEMV_R4 / mr > 0 ? OTPU_GEMV_R4 / mr : 1) : (L == 1 ? OTPU_GEMV_R1 / mr : OTPU_GEMV_R2);
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

// launch the streaming GEMV for MR <= 4 activation rows, L pieces a lane (team size a.T)
template <int FMT>
void launch_fmt(const MMArgs& a, int mr, int L, int batch, hipStream_t s);
// launch the GEMV with the QACT of its activation row in the prologue
template <int FMT>
void launch_qin_fmt(const MMArgs& a, int L, int batch, hipStream_t s);

}  // namespace otpu
