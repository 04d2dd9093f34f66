// VOP MUL (opentpu/isasim.py:1181, V_MUL -> fp32.mul, opentpu/fp32.py:100): one IEEE RNE
// product with flush-to-zero on operands and result.  The chained decode's glue between the
// gate / up MM and the down MM's QACT ranges (opentpu/kernels/mlp.py:101-104).
#include "otpu_common.h"

namespace otpu {

__global__ __launch_bounds__(256) void vmul_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                   float* __restrict__ out, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = fmul(a[i], b[i]);
}

}  // namespace otpu

using namespace otpu;

extern "C" int otpu_vmul(const float* a, const float* b, float* out, int64_t n, otpu_stream_t stream) {
    if (n < 1 || !a || !b || !out) return otpu_fail(OTPU_EINVAL, "vmul: n %lld", (long long)n);
    const int64_t blocks = (n + 255) / 256;
    if (blocks > 0x7FFFFFFF) return otpu_fail(OTPU_EINVAL, "vmul: n %lld too large", (long long)n);
    vmul_kernel<<<(unsigned)blocks, 256, 0, (hipStream_t)stream>>>(a, b, out, n);
    return otpu_launch_check("vmul");
}
