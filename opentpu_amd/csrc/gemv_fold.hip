// The folded down projection's kernels and launcher (the body is in gemv_fold.h, shared with
// the persistent chain).
#include "gemv_fold.h"

namespace otpu {

template <int FMT, int L>
__global__ __launch_bounds__(256) void gemv_fold_kernel(MMArgs a) {
    if (a.T == 64) fold_body<FMT, L, 64>(a);
    else if (a.T == 32) fold_body<FMT, L, 32>(a);
    else fold_body<FMT, L, 16>(a);
}

template <int FMT>
static void launch_fold_fmt(const MMArgs& a, int L, int64_t blocks, hipStream_t s) {
    switch (L) {
        case 1: gemv_fold_kernel<FMT, 1><<<(unsigned)blocks, 256, 0, s>>>(a); break;
        case 2: gemv_fold_kernel<FMT, 2><<<(unsigned)blocks, 256, 0, s>>>(a); break;
        case 3: gemv_fold_kernel<FMT, 3><<<(unsigned)blocks, 256, 0, s>>>(a); break;
        default: gemv_fold_kernel<FMT, 4><<<(unsigned)blocks, 256, 0, s>>>(a); break;
    }
}

// the grid: a team a row, 4 waves a workgroup, as many workgroups as rows allow up to 32 a CU
void launch_fold(const MMArgs& a, int fmt, int L, hipStream_t s) {
    const int64_t rows_per_wave = 64 / a.T;
    const int64_t waves = (a.N + rows_per_wave - 1) / rows_per_wave;
    int64_t blocks = (waves + 3) / 4;
    const int64_t cap = (int64_t)otpu_cu_count() * 32;
    if (blocks > cap) blocks = cap;
    if (fmt == OTPU_INT4) launch_fold_fmt<OTPU_INT4>(a, L, blocks, s);
    else if (fmt == OTPU_FP4) launch_fold_fmt<OTPU_FP4>(a, L, blocks, s);
    else launch_fold_fmt<OTPU_NVFP4>(a, L, blocks, s);
}

}  // namespace otpu
