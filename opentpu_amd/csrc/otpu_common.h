// Device helpers shared by the HIP kernels: the machine's fp32 arithmetic (IEEE RNE with
// flush-to-zero on operands and results, canonical NaN), the exact int64 -> fp32 conversion,
// recip, q8 and the total-order key.  Semantics: opentpu/fp32.py:45-121, :162-172, :242-261
// and docs/isa.md:88-135 of the reference.  Every file that includes this is compiled with
// -ffp-contract=off and fp32 denormals enabled, so each `a * b` below is one rounded v_mul_f32
// on the subnormal grid and the flushes are explicit.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/otpu.h"

#define OTPU_D 128          // K-block (MXU depth)

namespace otpu {

__device__ __forceinline__ uint32_t fbits(float x) { return __float_as_uint(x); }
__device__ __forceinline__ float bitsf(uint32_t u) { return __uint_as_float(u); }

// A denormal becomes the zero of its sign; everything else (NaN too) keeps its bits.  The
// comparison runs on the subnormal grid (denormals are enabled in these builds), so |x| < 2^-126
// holds exactly for the denormals and the zeros; three instructions (compare with the |.|
// modifier, sign mask, select).  These kernels run their code once per launch from a cold
// instruction cache, so the helpers' length is their latency.
__device__ __forceinline__ float ftz(float x) {
    return __builtin_fabsf(x) < 0x1p-126f ? bitsf(fbits(x) & 0x80000000u) : x;
}
// an arithmetic result: flush a denormal, canonical NaN
__device__ __forceinline__ float fin(float r) {
    r = ftz(r);
    return (r != r) ? bitsf(0x7FC00000u) : r;
}
__device__ __forceinline__ float fmul(float a, float b) { return fin(ftz(a) * ftz(b)); }
// fmul for operands already flushed (a fin() result, a flushed load, an integer's float)
__device__ __forceinline__ float fmul_f(float a, float b) { return fin(a * b); }
__device__ __forceinline__ float fadd(float a, float b) { return fin(ftz(a) + ftz(b)); }
// fadd for operands already flushed
__device__ __forceinline__ float fadd_f(float a, float b) { return fin(a + b); }
__device__ __forceinline__ float fsub(float a, float b) { return fin(ftz(a) - ftz(b)); }
__device__ __forceinline__ float pow2f(int d) { return bitsf((uint32_t)(d + 127) << 23); }

// total-order key of flushed bits: the unsigned order of keys is -NaN < -inf < .. < -0 < +0
// < .. < inf < NaN
__device__ __forceinline__ uint32_t fkey(float x) {
    uint32_t u = fbits(ftz(x));
    return (u >> 31) ? ~u : (u | 0x80000000u);
}
// fkey of a value already flushed
__device__ __forceinline__ uint32_t fkey_f(float x) {
    uint32_t u = fbits(x);
    return (u >> 31) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float unkey(uint32_t k) {
    return bitsf((k >> 31) ? (k & 0x7FFFFFFFu) : ~k);
}

// signed int64 -> fp32, round to nearest even, exact for every input (MM's |acc| < 2^47)
__device__ __forceinline__ float i2f(int64_t v) {
    uint64_t u = v < 0 ? (uint64_t)0 - (uint64_t)v : (uint64_t)v;
    float s;
    if (u < (1ull << 24)) {
        s = (float)(uint32_t)u;
    } else {
        int sh = 40 - __clzll((long long)u);          // bits below the 24-bit significand
        uint64_t mant = u >> sh;
        uint64_t rem = u & ((1ull << sh) - 1);
        uint64_t half = 1ull << (sh - 1);
        mant += (rem > half || (rem == half && (mant & 1))) ? 1 : 0;
        s = ldexpf((float)(uint32_t)mant, sh);         // mant <= 2^24: exact
    }
    return v < 0 ? -s : s;
}

// recip: seed 0x7EF311C3 - bits(a) on the significand a in [1, 2), two Newton steps, the
// correction step y*e + y, then 127 - exponent field added back; zero -> +0, |x| >= 2^126
// (and inf / NaN bits) -> a zero with x's sign.
__device__ __forceinline__ float recip(float x) {
    x = ftz(x);
    const uint32_t xb = fbits(x), mag = xb & 0x7FFFFFFFu, sign = xb & 0x80000000u;
    // Every value of the iteration is a normal float or zero (a in [1, 2), y in (0.47, 1], the
    // residue 1 - a y a multiple of 2^-24 of at most 2^-22), so the FTZ operations of the
    // definition are plain IEEE operations here: the same bits with no flush steps.  The
    // iteration runs for every input (a is in [1, 2) whatever the exponent) and the two special
    // cases select their results at the end: no branches, so the callers' independent recips
    // interleave (with one wave a SIMD, a branch serializes what follows it).
    const float a = bitsf(0x3F800000u | (mag & 0x7FFFFFu));
    float y = bitsf(0x7EF311C3u - fbits(a));
    y = y * (2.0f - a * y);
    y = y * (2.0f - a * y);
    y = y * (1.0f - a * y) + y;
    const int32_t k = 127 - (int32_t)(mag >> 23);       // (|sum| < 2^31 for every exponent)
    const float r = bitsf((uint32_t)((int32_t)fbits(y) + k * (1 << 23)) | sign);
    return mag == 0 ? 0.0f : (mag >= 0x7E800000u ? bitsf(sign) : r);
}

// q8: round half to even, saturate to +-127, NaN -> 0.  v_rndne_f32, then v_cvt_i32_f32 (which
// converts NaN to 0 and saturates out-of-range values and infinities), then a clamp; a
// denormal rounds to zero with or without its flush.
__device__ __forceinline__ int q8(float x) {
    int r;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(__builtin_rintf(x)));
    return min(max(r, -127), 127);
}

// floor(x / d) for 0 <= x < 2^16 and 1 <= d < 2^16, without the integer division's long
// sequence: the float quotient from the reciprocal (within 1 ulp) is off by at most one, which
// the two corrections remove
__device__ __forceinline__ int udiv_small(int x, int d) {
    int q = (int)((float)x * __builtin_amdgcn_rcpf((float)d));
    if ((q + 1) * d <= x) ++q;
    if (q * d > x) --q;
    return q;
}

__device__ __forceinline__ int window_of(int fmt) {
    return fmt == OTPU_INT8 ? 16 : (fmt == OTPU_NVFP4 ? 13 : 11);
}

// wave-wide reductions (wave64)
__device__ __forceinline__ int64_t wave_sum_i64(int64_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        uint64_t w = __shfl_xor(v, o, 64);
        v = w > v ? w : v;
    }
    return v;
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v, int width) {
    for (int o = width >> 1; o > 0; o >>= 1) {
        uint32_t w = __shfl_xor(v, o, 64);
        v = w > v ? w : v;
    }
    return v;
}

// max of v over aligned groups of `width` lanes (2, 4, .., 64), every lane receiving it; every
// lane of the wave must be active.  DPP quad_perm swaps cross lane bits 0 and 1, then
// row_half_mirror (lane i <-> 7 - i within 8) and row_mirror (i <-> 15 - i within 16) -- each
// pairs lanes of two halves already reduced -- then v_permlane16_swap / v_permlane32_swap cross
// bits 4 and 5.  A __shfl_xor step (wave_max_u32) is an LDS permute, ~10x the latency.
__device__ __forceinline__ uint32_t wave_max_dpp(uint32_t v, int width) {
    if (width >= 2) v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));
    if (width >= 4) v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
    if (width >= 8) v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));
    if (width >= 16) v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));
    if (width >= 32) {
        const auto p16 = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        v = max((uint32_t)p16[0], (uint32_t)p16[1]);
    }
    if (width >= 64) {
        const auto p32 = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        v = max((uint32_t)p32[0], (uint32_t)p32[1]);
    }
    return v;
}

// wave_max_dpp(v, 64), with wave_max_dpp(v, 8) -- the first three steps of the same reduction
// -- returned in g8
__device__ __forceinline__ uint32_t wave_max_dpp_64_8(uint32_t v, uint32_t& g8) {
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));
    g8 = v;
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));
    const auto p16 = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = max((uint32_t)p16[0], (uint32_t)p16[1]);
    const auto p32 = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return max((uint32_t)p32[0], (uint32_t)p32[1]);
}

}  // namespace otpu

// host-side error reporting shared by the entry points (abi.hip)
int otpu_fail(int code, const char* fmt, ...);
int otpu_launch_check(const char* what);
int otpu_cu_count();
