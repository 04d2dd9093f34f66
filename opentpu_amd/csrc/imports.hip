// Checkpoint imports on the GPU: OCP MXFP4 and NVFP4 weights into the MXU's fp4 / nvfp4 rows,
// exactly (opentpu/quant.py:1070-1182, import_mxfp4 / import_nvfp4).  One wave per weight row.
// The kernels write the asked format's rows and a per-row status word of the reasons the
// reference would refuse the matrix in that format (NotExact); the host reduces the status
// words, raises, or (MXFP4 that fp4 does not hold) asks again for nvfp4.
//
// MXFP4 (codes one per byte, an E8M0 exponent per 32):
//   live sub-block: a code with magnitude bits (c & 7) set;
//   fp4:   per block lo / hi = the smallest / largest live e; top = the largest block lo (129
//          for a row without live blocks); dw = top - lo; m_b = 2^(e_b - lo) (1 if dead);
//          Sw = 2^(top - 128);
//   nvfp4: top = the row's largest live e (131 if none); span = top - e; byte = (15 - span) << 3,
//          4, 2, 1 for spans 15, 16, 17 (0 if dead), twice per sub-block; Sw = 2^(top - 131).
// NVFP4 (codes, an E4M3 scale per 16, a tensor scale ts):
//   m 2^p (m = 8 + M normal, M subnormal; p = max(E, 1) - 10) -> m' = m << sh in 8..15,
//   p' = p - sh; top = the row's largest live p' (1 if none); dw = top - p'; byte
//   ((15 - dw) << 3) | (m' - 8) for dw <= 14, else the MXU subnormal m' >> (dw - 14);
//   Sw = f32(ts) 2^(top - 1).
#include "otpu_common.h"

namespace otpu {

enum : int32_t {
    MX_NAN = 1,          // an E8M0 NaN (0xFF)
    MX_SPAN5 = 2,        // a K-block's live exponents span more than 5 (no fp4)
    MX_DW = 4,           // fp4: a block more than 255 octaves below the row's top
    MX_SW4 = 8,          // fp4: Sw outside fp32's normal range
    MX_SPAN17 = 16,      // a row's live exponents span more than 17 (no nvfp4)
    MX_SWNV = 32,        // nvfp4: Sw outside fp32's normal range
    NV_NEG = 1,          // a negative E4M3 scale
    NV_NAN = 2,          // an E4M3 NaN (0x7F)
    NV_FAR = 4,          // a scale too far below the row's largest to hold exactly
    NV_SW = 8,           // Sw outside fp32's normal range
};

__device__ __forceinline__ int wave_max_i(int v) {
    for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ int wave_min_i(int v) {
    for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ int32_t wave_or(int32_t v) {
    for (int o = 32; o > 0; o >>= 1) v |= __shfl_xor(v, o, 64);
    return v;
}

// 32 codes (one a byte) -> 16 packed bytes (element 2i low nibble); live = any magnitude bit
__device__ __forceinline__ uint4 pack_codes32(const uint8_t* c, bool& live) {
    const uint4 a = *reinterpret_cast<const uint4*>(c);
    const uint4 b = *reinterpret_cast<const uint4*>(c + 16);
    const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint32_t o[4];
    uint32_t any = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {               // input words 2q, 2q+1 -> output word q
        uint32_t v = 0;
#pragma unroll
        for (int t = 0; t < 4; ++t) {           // output byte t: codes 8q + 2t, 8q + 2t + 1
            const uint32_t lo = (w[2 * q + (t >> 1)] >> (16 * (t & 1))) & 0xFF;
            const uint32_t hi = (w[2 * q + (t >> 1)] >> (16 * (t & 1) + 8)) & 0xFF;
            v |= ((lo | (hi << 4)) & 0xFF) << (8 * t);
        }
        o[q] = v;
        any |= w[2 * q] | w[2 * q + 1];
    }
    live = (any & 0x07070707u) != 0;
    return make_uint4(o[0], o[1], o[2], o[3]);
}

constexpr int BIG = 1 << 20;

template <bool NV>
__global__ __launch_bounds__(64) void import_mx_kernel(const uint8_t* __restrict__ codes, int64_t ldc,
                                                       const uint8_t* __restrict__ ex, int64_t lde, int K,
                                                       uint8_t* __restrict__ rows, int64_t rs,
                                                       uint8_t* __restrict__ srows, int64_t srs,
                                                       int32_t* __restrict__ status) {
    const int row = blockIdx.x, lane = threadIdx.x;
    const int NS = K / 32, KB = K / 128;
    const uint8_t* c = codes + (int64_t)row * ldc;
    const uint8_t* e = ex + (int64_t)row * lde;
    uint8_t* erow = rows + (int64_t)row * rs;
    uint8_t* srow = srows + (int64_t)row * srs;
    int32_t st = 0;
    int top = -BIG, rmin = BIG;                 // fp4: max block lo; nvfp4: max / min live e
    // pass 1: the row's top and the refusal reasons; the packed codes
    for (int s0 = 0; s0 < NS; s0 += 64) {       // uniform: every lane shuffles
        const int s = s0 + lane;
        const bool ok = s < NS;
        bool live = false;
        if (ok) *reinterpret_cast<uint4*>(erow + 16 * s) = pack_codes32(c + 32 * s, live);
        const int ev = ok ? (int)e[s] : 0;
        if (ok && ev == 0xFF) st |= MX_NAN;
        int lo = live ? ev : BIG, hi = live ? ev : -BIG;
        lo = min(lo, __shfl_xor(lo, 1, 64));
        lo = min(lo, __shfl_xor(lo, 2, 64));
        hi = max(hi, __shfl_xor(hi, 1, 64));
        hi = max(hi, __shfl_xor(hi, 2, 64));
        const bool blive = lo != BIG;
        if (ok && blive && hi - lo > 5) st |= MX_SPAN5;
        if (!NV && ok && blive) top = max(top, lo);
        if (NV && ok && live) {
            rmin = min(rmin, ev);
            top = max(top, ev);
        }
    }
    top = wave_max_i(top);
    rmin = wave_min_i(rmin);
    st = wave_or(st);
    if (NV && top != -BIG && top - rmin > 17) st |= MX_SPAN17;
    const bool none = top == -BIG;
    if (NV) {
        top = none ? 131 : top;
        if (top - 131 < -126 || top - 131 > 127) st |= MX_SWNV;
    } else {
        top = none ? 129 : top;
        if (top - 128 < -126 || top - 128 > 127) st |= MX_SW4;
    }
    // pass 2: the scale row
    for (int s0 = 0; s0 < NS; s0 += 64) {
        const int s = s0 + lane;
        const bool ok = s < NS;
        bool live = false;
        if (ok) {
            const uint4 a = *reinterpret_cast<const uint4*>(c + 32 * s);
            const uint4 b = *reinterpret_cast<const uint4*>(c + 32 * s + 16);
            live = ((a.x | a.y | a.z | a.w | b.x | b.y | b.z | b.w) & 0x07070707u) != 0;
        }
        const int ev = ok ? (int)e[s] : 0;
        int lo = live ? ev : BIG;
        lo = min(lo, __shfl_xor(lo, 1, 64));
        lo = min(lo, __shfl_xor(lo, 2, 64));
        const bool blive = lo != BIG;
        if (NV) {
            const int span = live ? top - ev : 0;
            const int E = 15 - span;
            const uint32_t byte = !live ? 0u : (E >= 1 ? (uint32_t)(E << 3) & 0xFF : (E == 0 ? 4u : (E == -1 ? 2u : 1u)));
            const uint32_t pair = byte | (byte << 8);
            const uint32_t p1 = __shfl_xor(pair, 1, 64), p2 = __shfl_xor(pair, 2, 64), p3 = __shfl_xor(pair, 3, 64);
            if (ok && (s & 3) == 0)
                *reinterpret_cast<uint2*>(srow + 16 + 2 * s) = make_uint2(pair | (p1 << 16), p2 | (p3 << 16));
        } else {
            const int dw = blive ? top - lo : 0;
            if (ok && dw > 255) st |= MX_DW;
            int sh = live ? ev - lo : 0;
            sh = sh < 0 ? 0 : (sh > 7 ? 7 : sh);
            const uint32_t mb = (1u << sh) & 0xFF;
            const uint32_t m1 = __shfl_xor(mb, 1, 64), m2 = __shfl_xor(mb, 2, 64), m3 = __shfl_xor(mb, 3, 64);
            if (ok && (s & 3) == 0) {
                const uint32_t wd = ((uint32_t)dw & 0xFF) | (mb << 8) | (m1 << 14) | (m2 << 20) | (m3 << 26);
                *reinterpret_cast<uint32_t*>(srow + 8 + 4 * (s >> 2)) = wd;
            }
        }
    }
    st = wave_or(st);
    if (lane == 0) {
        const int sh = NV ? top - 131 : top - 128;
        const float Sw = (sh < -126 || sh > 127) ? 0.0f : __builtin_ldexpf(1.0f, sh);
        *reinterpret_cast<float*>(srow) = Sw;
        *reinterpret_cast<uint32_t*>(srow + 4) = 0u;
        if (NV) *reinterpret_cast<uint2*>(srow + 8) = make_uint2(0u, 0u);
        const int hdr = NV ? 16 : 8, per = NV ? 8 : 4;
        if (KB & 1) {                               // the scale row's pad to a whole pair
            if (NV) *reinterpret_cast<uint2*>(srow + hdr + per * KB) = make_uint2(0u, 0u);
            else *reinterpret_cast<uint32_t*>(srow + hdr + per * KB) = 0u;
        }
        status[row] = st;
    }
    const int64_t rb = (int64_t)((K + 255) / 256) * 128;
    for (int64_t t = K / 2 + 16 * lane; t < rb; t += 1024)
        *reinterpret_cast<uint4*>(erow + t) = make_uint4(0, 0, 0, 0);
}

__global__ __launch_bounds__(64) void import_nv_kernel(const uint8_t* __restrict__ codes, int64_t ldc,
                                                       const uint8_t* __restrict__ sc, int64_t lds, float ts,
                                                       int K, uint8_t* __restrict__ rows, int64_t rs,
                                                       uint8_t* __restrict__ srows, int64_t srs,
                                                       int32_t* __restrict__ status) {
    const int row = blockIdx.x, lane = threadIdx.x;
    const int NG = K / 16, KB = K / 128;
    const uint8_t* c = codes + (int64_t)row * ldc;
    const uint8_t* sv = sc + (int64_t)row * lds;
    uint8_t* erow = rows + (int64_t)row * rs;
    uint8_t* srow = srows + (int64_t)row * srs;
    int32_t st = 0;
    int top = -BIG;
    for (int g = lane; g < NG; g += 64) {
        const int b = sv[g];
        if (b & 0x80) st |= NV_NEG;
        if (b == 0x7F) st |= NV_NAN;
        const int E = (b >> 3) & 15, M = b & 7;
        const int m = E > 0 ? 8 + M : M;
        if (m > 0) {
            const int sh = 3 - (31 - __builtin_clz((unsigned)m));
            top = max(top, (E > 0 ? E : 1) - 10 - sh);
        }
        // the group's 16 codes -> 8 packed bytes
        const uint4 a = *reinterpret_cast<const uint4*>(c + 16 * g);
        const uint32_t w[4] = {a.x, a.y, a.z, a.w};
        uint32_t o[2] = {0, 0};
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const uint32_t lo = (w[t >> 1] >> (16 * (t & 1))) & 0xFF;
            const uint32_t hi = (w[t >> 1] >> (16 * (t & 1) + 8)) & 0xFF;
            o[t >> 2] |= ((lo | (hi << 4)) & 0xFF) << (8 * (t & 3));
        }
        *reinterpret_cast<uint2*>(erow + 8 * g) = make_uint2(o[0], o[1]);
    }
    top = wave_max_i(top);
    top = top == -BIG ? 1 : top;
    for (int g0 = 0; g0 < NG; g0 += 64) {                 // uniform: every lane shuffles
        const int g = g0 + lane;
        const bool ok = g < NG;
        const int b = ok ? sv[g] : 0;
        const int E = (b >> 3) & 15, M = b & 7;
        const int m = E > 0 ? 8 + M : M;
        uint32_t byte = 0;
        if (ok && m > 0) {
            const int sh = 3 - (31 - __builtin_clz((unsigned)m));
            const int mn = m << sh, pn = (E > 0 ? E : 1) - 10 - sh;
            const int dw = top - pn;
            if (dw > 17) st |= NV_FAR;
            if (dw <= 14) {
                byte = (uint32_t)((((15 - dw) << 3) | (mn - 8)) & 0xFF);
            } else {
                const int drop = dw - 14 > 3 ? 3 : dw - 14;
                const int ms = mn >> drop;
                if ((ms << drop) != mn) st |= NV_FAR;
                byte = (uint32_t)ms;
            }
        }
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t v = (uint32_t)__shfl(byte, (lane & ~7) + j, 64);
            if (j < 4) lo |= v << (8 * j);
            else hi |= v << (8 * (j - 4));
        }
        if (ok && (g & 7) == 0) *reinterpret_cast<uint2*>(srow + 16 + g) = make_uint2(lo, hi);
    }
    st = wave_or(st);
    if (lane == 0) {
        const double sw = (double)ts * __builtin_ldexp(1.0, top - 1);
        const double a = fabs(sw);
        if (sw != 0.0 && (a < 0x1p-126 || a >= 0x1p128)) st |= NV_SW;
        *reinterpret_cast<float*>(srow) = (float)sw;
        *reinterpret_cast<uint32_t*>(srow + 4) = 0u;
        *reinterpret_cast<uint2*>(srow + 8) = make_uint2(0u, 0u);
        if (KB & 1) *reinterpret_cast<uint2*>(srow + 16 + 8 * KB) = make_uint2(0u, 0u);
        status[row] = st;
    }
    const int64_t rb = (int64_t)((K + 255) / 256) * 128;
    for (int64_t t = K / 2 + 16 * lane; t < rb; t += 1024)
        *reinterpret_cast<uint4*>(erow + t) = make_uint4(0, 0, 0, 0);
}

}  // namespace otpu

using namespace otpu;

static int check_import(const char* what, const uint8_t* codes, int64_t ldc, int N, int K, uint8_t* rows, int64_t rs,
                        uint8_t* srows, int64_t srs, int64_t sneed, const int32_t* status) {
    if (N < 1 || K < OTPU_D || K % OTPU_D || ldc < K)
        return otpu_fail(OTPU_EINVAL, "%s: N %d, K %d (whole blocks of %d), ldc %lld", what, N, K, OTPU_D, (long long)ldc);
    const int64_t rb = (int64_t)((K + 255) / 256) * 128;
    if (!codes || !rows || !srows || !status || rs < rb || srs < sneed || rs % 16 || srs % 8 || ldc % 16)
        return otpu_fail(OTPU_EINVAL, "%s: rows of %lld bytes (need %lld), scale rows of %lld (need %lld), ldc %lld "
                         "(multiples of 16, 8, 16)", what, (long long)rs, (long long)rb, (long long)srs,
                         (long long)sneed, (long long)ldc);
    if (((uintptr_t)codes & 15) || ((uintptr_t)rows & 15) || ((uintptr_t)srows & 7) || ((uintptr_t)status & 3))
        return otpu_fail(OTPU_EALIGN, "%s: codes and rows 16-byte, scale rows 8-byte aligned", what);
    return 0;
}

extern "C" int otpu_import_mxfp4(const uint8_t* codes, int64_t ldc, const uint8_t* e8m0, int64_t lde, int N, int K,
                                 int fmt, uint8_t* rows, int64_t rs, uint8_t* srows, int64_t srs, int32_t* status,
                                 otpu_stream_t stream) {
    if (fmt != OTPU_FP4 && fmt != OTPU_NVFP4) return otpu_fail(OTPU_EFORMAT, "import_mxfp4: into format %d (fp4 or nvfp4)", fmt);
    const int KB = K / OTPU_D;
    const int64_t sneed = fmt == OTPU_NVFP4 ? 16 + 16 * ((KB + 1) / 2) : 8 + 8 * ((KB + 1) / 2);
    if (int rc = check_import("import_mxfp4", codes, ldc, N, K, rows, rs, srows, srs, sneed, status)) return rc;
    if (!e8m0 || lde < K / 32) return otpu_fail(OTPU_EINVAL, "import_mxfp4: exponent rows of %lld (need %d)", (long long)lde, K / 32);
    hipStream_t s = (hipStream_t)stream;
    if (fmt == OTPU_NVFP4) import_mx_kernel<true><<<N, 64, 0, s>>>(codes, ldc, e8m0, lde, K, rows, rs, srows, srs, status);
    else import_mx_kernel<false><<<N, 64, 0, s>>>(codes, ldc, e8m0, lde, K, rows, rs, srows, srs, status);
    return otpu_launch_check("import_mxfp4");
}

extern "C" int otpu_import_nvfp4(const uint8_t* codes, int64_t ldc, const uint8_t* scales, int64_t lds, float ts,
                                 int N, int K, uint8_t* rows, int64_t rs, uint8_t* srows, int64_t srs, int32_t* status,
                                 otpu_stream_t stream) {
    const int KB = K / OTPU_D;
    if (int rc = check_import("import_nvfp4", codes, ldc, N, K, rows, rs, srows, srs, 16 + 16 * ((KB + 1) / 2), status))
        return rc;
    if (!scales || lds < K / 16) return otpu_fail(OTPU_EINVAL, "import_nvfp4: scale rows of %lld (need %d)", (long long)lds, K / 16);
    import_nv_kernel<<<N, 64, 0, (hipStream_t)stream>>>(codes, ldc, scales, lds, ts, K, rows, rs, srows, srs, status);
    return otpu_launch_check("import_nvfp4");
}
