// The int4x / fp4x6 and nvfp4 weight packers on the GPU, bit-exact with opentpu/quant.py:325-367
// (_x4), :368-400 (_nv) and :403-425 (pack_scales), which the reference runs on the host in numpy
// float64.
//
// One wave per weight row; lane s takes the 32-element sub-blocks s, s+64, ...  All arithmetic
// is IEEE float64 with FMA contraction off, in the reference's order:
//   sb = max|x| / qmax (qmax 7 int4, 6 E2M1)          top = max sb over the row
//   Sw = f32(top / 63) (1 for an all-zero row)        bmax = max sb over the block
//   d  = clip(floor(log2(63 Sw / bmax)), 0, 255)      unit = Sw * 2^-d
//   for f in linspace(0.64, 1.12, 13): m = clip(rint(sb / unit * f), 1, 63), s = unit * m,
//     err = sum((grid(x / s) * s - x)^2) in numpy's pairwise order (8 running partials,
//     ((p0+p1)+(p2+p3))+((p4+p5)+(p6+p7))); the first strictly smaller err wins.
// floor(log2(v)) is taken exactly from v's exponent. numpy's rounded log2 agrees for every
// float32 input: 63 qmax Sw has at most 33 significant bits and bmax = rnd(a / qmax) for a
// float32 a, so v is a power of two or at least ~2^-34 (relative) away from every one.
#include <cmath>

#include "otpu_common.h"

namespace otpu {

struct Search { double f[13]; };

__device__ __forceinline__ double grid_value(double v, bool e2m1) {
    if (!e2m1) {
        double r = __builtin_rint(v);
        return r < -7.0 ? -7.0 : (r > 7.0 ? 7.0 : r);          // NaN passes through, as np.clip
    }
    const double a = fabs(v);
    const int code = (a > 0.25) + (a >= 0.75) + (a > 1.25) + (a >= 1.75) + (a > 2.5) + (a >= 3.5) + (a > 5.0);
    const double mag[8] = {0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0};
    const double sg = v > 0.0 ? 1.0 : (v < 0.0 ? -1.0 : (v == 0.0 ? 0.0 : v));   // np.sign
    return sg * mag[code];
}

__device__ __forceinline__ int e2m1_code(double v) {
    const double a = fabs(v);
    return (a > 0.25) + (a >= 0.75) + (a > 1.25) + (a >= 1.75) + (a > 2.5) + (a >= 3.5) + (a > 5.0);
}

template <bool E2M1>
__global__ __launch_bounds__(64) void pack_x4_kernel(const float* __restrict__ W, int K, int64_t ldw,
                                                     uint8_t* __restrict__ rows, int64_t rs,
                                                     uint8_t* __restrict__ srows, int64_t srs, Search sr) {
    const int row = blockIdx.x, lane = threadIdx.x;
    const float* x = W + (int64_t)row * ldw;
    const int NS = K / 32, KB = K / 128;
    const double qmax = E2M1 ? 6.0 : 7.0;

    double top = 0.0;
    for (int s = lane; s < NS; s += 64) {
        double m = 0.0;
        for (int i = 0; i < 32; ++i) m = fmax(m, fabs((double)x[32 * s + i]));
        top = fmax(top, m / qmax);
    }
    for (int o = 32; o > 0; o >>= 1) top = fmax(top, __shfl_xor(top, o, 64));
    const double Sw = top == 0.0 ? 1.0 : (double)(float)(top / 63.0);
    uint8_t* srow = srows + (int64_t)row * srs;
    uint8_t* erow = rows + (int64_t)row * rs;

    for (int s0 = 0; s0 < NS; s0 += 64) {               // uniform: every lane shuffles
        const int s = s0 + lane;
        const bool ok = s < NS;
        double xv[32];
        double amax = 0.0;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            xv[i] = ok ? (double)x[32 * s + i] : 0.0;
            amax = fmax(amax, fabs(xv[i]));
        }
        const double sb = amax / qmax;
        double bmax = fmax(sb, __shfl_xor(sb, 1, 64));
        bmax = fmax(bmax, __shfl_xor(bmax, 2, 64));
        double d = 0.0;
        if (bmax > 0.0) {
            const double v = 63.0 * Sw / bmax;
            if (isinf(v)) d = 255.0;
            else if (v > 0.0) {
                int e;
                frexp(v, &e);                            // v in [2^(e-1), 2^e)
                d = (double)(e - 1);
                d = d < 0.0 ? 0.0 : (d > 255.0 ? 255.0 : d);
            }
        }
        const double unit = Sw * exp2(-d);
        const double m0 = sb / unit;
        double best_m = 0.0, best_e = 0.0;
        for (int c = 0; c < 13; ++c) {
            double m = __builtin_rint(m0 * sr.f[c]);
            m = m < 1.0 ? 1.0 : (m > 63.0 ? 63.0 : m);
            const double sc = unit * m;
            double p[8];
#pragma unroll
            for (int i = 0; i < 32; ++i) {
                const double q = grid_value(xv[i] / sc, E2M1) * sc;
                const double e = (q - xv[i]) * (q - xv[i]);
                if (i < 8) p[i] = e;
                else p[i & 7] = p[i & 7] + e;
            }
            const double err = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
            if (c == 0 || err < best_e) { best_e = err; best_m = m; }
        }
        // element codes of the winner: g = (grid(x/s) * s) / (unit * m)
        const double sc = unit * best_m;
        uint32_t word[4] = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            const double g = (grid_value(xv[i] / sc, E2M1) * sc) / sc;
            uint32_t code;
            if (!E2M1) {
                code = (uint32_t)((long long)__builtin_rint(g) & 15);
            } else {
                const int mag = e2m1_code(g);
                code = (uint32_t)(mag | ((signbit(g) && mag != 0) ? 8 : 0));
            }
            word[i >> 3] |= code << (4 * (i & 7));
        }
        if (ok) *reinterpret_cast<uint4*>(erow + 16 * s) = make_uint4(word[0], word[1], word[2], word[3]);
        // the block's scale word: dw | m_b << (8 + 6 b), assembled by the block's first lane
        const uint32_t mb = (uint32_t)best_m;
        const uint32_t m1 = __shfl_xor(mb, 1, 64), m2 = __shfl_xor(mb, 2, 64), m3 = __shfl_xor(mb, 3, 64);
        if (ok && (s & 3) == 0) {
            const uint32_t wd = (uint32_t)d | (mb << 8) | (m1 << 14) | (m2 << 20) | (m3 << 26);
            *reinterpret_cast<uint32_t*>(srow + 8 + 4 * (s >> 2)) = wd;
        }
    }
    if (lane == 0) {
        const float swf = E2M1 ? (float)(Sw * 0.5) : (float)Sw;
        *reinterpret_cast<float*>(srow) = swf;
        *reinterpret_cast<uint32_t*>(srow + 4) = 0u;
    }
    // padding: scale-row words past the last block, element bytes past K/2
    for (int t = 8 + 4 * KB + 4 * lane; t + 4 <= srs && t < 8 + 8 * ((KB + 1) / 2); t += 256)
        *reinterpret_cast<uint32_t*>(srow + t) = 0u;
    const int64_t rb = (int64_t)((K + 255) / 256) * 128;
    for (int64_t t = K / 2 + 16 * lane; t < rb; t += 1024)
        *reinterpret_cast<uint4*>(erow + t) = make_uint4(0, 0, 0, 0);
}

// E4M3 (bias 7, subnormals at E = 0, no infinities): round a non-negative float64 to nearest,
// ties to the even mantissa, saturating at 448 (code 126).  From the binade: a = f 2^e with f in
// [1, 2) -> code ((e + 7) << 3) + rint((f - 1) 8) (a mantissa carry moves into the exponent);
// below 2^-6 the subnormal step 2^-9.  Every operation is exact but the final rint.
__device__ __forceinline__ int e4m3_rne(double a) {
    if (!(a > 0.0)) return 0;
    int ex;
    frexp(a, &ex);                                               // a in [2^(ex-1), 2^ex)
    const int e = ex - 1;
    int code;
    if (e < -6) code = (int)__builtin_rint(a * 512.0);
    else code = ((e + 7) << 3) + (int)__builtin_rint((ldexp(a, -e) - 1.0) * 8.0);
    return code > 126 ? 126 : code;
}

__device__ __forceinline__ double e4m3_val(int c) {
    const int E = c >> 3, m = c & 7;
    return E == 0 ? (double)m * 0x1p-9 : (double)(8 + m) * ldexp(1.0, E - 10);
}

// nvfp4 with a per-row scale (opentpu/quant.py:368-400, _nv): one wave per row, lane t takes the
// 16-element groups t, t + 64, ...  ts = f32(row amax / 2688) (1 for a zero row); per group the
// E4M3 scale s = e4m3(amax_g / ts * f / 6) over the 13 candidates f, s = 1 where the group or s
// is 0, err = sum((sign(xb) E2M1(|xb| / s) s - xb)^2) in numpy's order for 16 terms (8 running
// partials then ((p0+p1)+(p2+p3))+((p4+p5)+(p6+p7))), the first strictly smaller err wins;
// element codes of q / s; Sw = f32(16 ts).
__global__ __launch_bounds__(64) void pack_nv_kernel(const float* __restrict__ W, int K, int64_t ldw,
                                                     uint8_t* __restrict__ rows, int64_t rs,
                                                     uint8_t* __restrict__ srows, int64_t srs, Search sr) {
    const int row = blockIdx.x, lane = threadIdx.x;
    const float* x = W + (int64_t)row * ldw;
    const int NG = K / 16, KB = K / 128;
    const double mag[8] = {0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0};

    float am = 0.0f;
    for (int i = lane; i < K; i += 64) am = fmaxf(am, fabsf(x[i]));
    for (int o = 32; o > 0; o >>= 1) am = fmaxf(am, __shfl_xor(am, o, 64));
    double ts = (double)am / 2688.0;
    ts = (double)(float)(ts == 0.0 ? 1.0 : ts);
    uint8_t* srow = srows + (int64_t)row * srs;
    uint8_t* erow = rows + (int64_t)row * rs;

    for (int g0 = 0; g0 < NG; g0 += 64) {                // uniform: every lane shuffles
        const int g = g0 + lane;
        const bool ok = g < NG;
        double xv[16];
        double amax = 0.0;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            xv[i] = ok ? (double)x[16 * g + i] / ts : 0.0;
            amax = fmax(amax, fabs(xv[i]));
        }
        double best_s = 1.0, best_e = 0.0;
        for (int c = 0; c < 13; ++c) {
            double s = e4m3_val(e4m3_rne(amax * sr.f[c] / 6.0));
            if (amax == 0.0 || s == 0.0) s = 1.0;
            double p[8];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const double v = xv[i];
                const double sg = v > 0.0 ? 1.0 : (v < 0.0 ? -1.0 : 0.0);
                const double q = sg * mag[e2m1_code(v / s)] * s;
                const double e = (q - v) * (q - v);
                if (i < 8) p[i] = e;
                else p[i & 7] = p[i & 7] + e;
            }
            const double err = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
            if (c == 0 || err < best_e) { best_e = err; best_s = s; }
        }
        uint32_t word[2] = {0, 0};
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const double v = xv[i];
            const double sg = v > 0.0 ? 1.0 : (v < 0.0 ? -1.0 : 0.0);
            const double gq = (sg * mag[e2m1_code(v / best_s)] * best_s) / best_s;
            const int mg = e2m1_code(gq);
            const uint32_t code = (uint32_t)(mg | ((signbit(gq) && mg != 0) ? 8 : 0));
            word[i >> 3] |= code << (4 * (i & 7));
        }
        if (ok) *reinterpret_cast<uint2*>(erow + 8 * g) = make_uint2(word[0], word[1]);
        // the block's eight E4M3 bytes, assembled by its first lane
        const uint32_t b = (uint32_t)e4m3_rne(best_s);
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t v = (uint32_t)__shfl(b, (lane & ~7) + j, 64);
            if (j < 4) lo |= v << (8 * j);
            else hi |= v << (8 * (j - 4));
        }
        if (ok && (g & 7) == 0) *reinterpret_cast<uint2*>(srow + 16 + g) = make_uint2(lo, hi);
    }
    if (lane == 0) {
        *reinterpret_cast<float*>(srow) = (float)(16.0 * ts);
        *reinterpret_cast<uint32_t*>(srow + 4) = 0u;
        *reinterpret_cast<uint2*>(srow + 8) = make_uint2(0u, 0u);
        if (KB & 1) *reinterpret_cast<uint2*>(srow + 16 + 8 * KB) = make_uint2(0u, 0u);
    }
    const int64_t rb = (int64_t)((K + 255) / 256) * 128;
    for (int64_t t = K / 2 + 16 * lane; t < rb; t += 1024)
        *reinterpret_cast<uint4*>(erow + t) = make_uint4(0, 0, 0, 0);
}

}  // namespace otpu

using namespace otpu;

extern "C" int otpu_pack_x4(const float* W, int N, int K, int64_t ldw, int fmt, uint8_t* rows, int64_t rs,
                            uint8_t* srows, int64_t srs, otpu_stream_t stream) {
    if (fmt != OTPU_INT4 && fmt != OTPU_FP4 && fmt != OTPU_NVFP4)
        return otpu_fail(OTPU_EFORMAT, "pack_x4: format %d (int4, fp4 or nvfp4)", fmt);
    if (N < 1 || K < OTPU_D || K % OTPU_D || ldw < K)
        return otpu_fail(OTPU_EINVAL, "pack_x4: N %d, K %d, ldw %lld", N, K, (long long)ldw);
    const int KB = K / OTPU_D;
    const int64_t rb = (int64_t)((K + 255) / 256) * 128;
    const int64_t sb = fmt == OTPU_NVFP4 ? 16 + 16 * ((KB + 1) / 2) : 8 + 8 * ((KB + 1) / 2);
    if (rs < rb || srs < sb || rs % 16 || srs % 8)
        return otpu_fail(OTPU_EINVAL, "pack_x4: rows of %lld bytes (need %lld, a multiple of 16), scale rows of %lld (need %lld, a multiple of 8)",
                         (long long)rs, (long long)rb, (long long)srs, (long long)sb);
    if (((uintptr_t)rows & 15) || ((uintptr_t)srows & 7) || ((uintptr_t)W & 3))
        return otpu_fail(OTPU_EALIGN, "pack_x4: rows 16-byte, scale rows 8-byte aligned");
    Search sr;
    const double start = 0.64, stop = 1.12, step = (stop - start) / 12.0;   // numpy.linspace(0.64, 1.12, 13)
    for (int i = 0; i < 12; ++i) {
        volatile double t = (double)i * step;                                // no contraction
        sr.f[i] = t + start;
    }
    sr.f[12] = stop;
    hipStream_t s = (hipStream_t)stream;
    if (fmt == OTPU_NVFP4) pack_nv_kernel<<<N, 64, 0, s>>>(W, K, ldw, rows, rs, srows, srs, sr);
    else if (fmt == OTPU_FP4) pack_x4_kernel<true><<<N, 64, 0, s>>>(W, K, ldw, rows, rs, srows, srs, sr);
    else pack_x4_kernel<false><<<N, 64, 0, s>>>(W, K, ldw, rows, rs, srows, srs, sr);
    return otpu_launch_check("pack_x4");
}
