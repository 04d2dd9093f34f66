// MM for many activation rows on the int8 MFMA units (prefill GEMM).  Placeholder until the
// MFMA kernel lands: returns 1 ("not this path") so that otpu_mm runs the row-streaming kernel.
#include "otpu_common.h"

int otpu_gemm_try(const int8_t*, int64_t, const float*, const uint8_t*, int64_t, int, int,
                  const uint8_t*, int64_t, const uint8_t*, int64_t, int, int, int, float*, int64_t,
                  hipStream_t) {
    return 1;
}
