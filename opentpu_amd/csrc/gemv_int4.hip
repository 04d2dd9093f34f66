// The decode GEMV kernels of the int4 weight format (the kernel source is gemv_impl.h).
#include "gemv_impl.h"

namespace otpu {
template void launch_fmt<OTPU_INT4>(const MMArgs& a, int mr, int L, int batch, hipStream_t s);
template void launch_qin_fmt<OTPU_INT4>(const MMArgs& a, int L, int batch, hipStream_t s);
}  // namespace otpu
