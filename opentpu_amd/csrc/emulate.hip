// The reference's float64 emulation of the operator (opentpu/quant.py:895-1067: fake_act,
// fake_w's dequantization and group offsets, mx_matmul), on the GPU.  These are the values the
// reference's model code checks the machine against: QACT's values as float64 multiples of the
// range's scale, the weights' exact float64 values, and the float64 product that leaves out the
// 16-element groups MM's window drops.
//
//   fake_act:  per range of n columns, s = amax / 127 (1 for a zero range), per group of g
//              d = the largest (<= 31) with the group's amax 2^d <= amax (0 in row mode),
//              unit = s 2^-d, q = rint(x / unit) -- where x / unit lies within 2^-31 of a tie,
//              the device quantizer's q (fp32.quantize_mx) -- and value clip(q, +-127) unit;
//              da: d for each 16-element group.
//   dequant:   w m 2^-dw Sw in float64 (exact), a denormal Sw 0; dw for each 16-element group.
//   mx_matmul: y[j, n] = sum over 16-element groups kept of sum_k h[j, k] w[n, k], a group
//              kept when da[j, g] + dw[n, g] <= W (no da: every group).
#include <math.h>

#include "otpu_common.h"

namespace otpu {

constexpr int EG = 16;            // a drop group: D / 8 elements

// |x| of a float64 as an ordered key (the unsigned order of the magnitude's bits), and back
__device__ __forceinline__ uint64_t mag64(double x) { return (uint64_t)__double_as_longlong(x) & 0x7FFFFFFFFFFFFFFFull; }

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v, int width) {
    for (int o = width >> 1; o > 0; o >>= 1) {
        const uint64_t w = __shfl_xor(v, o, 64);
        v = w > v ? w : v;
    }
    return v;
}

// four consecutive elements of a row: e the float64 values the emulation quantizes (the input as
// given), f their float32 values (the input the device quantizer's tie rule reads: fp32 as given,
// or float64 rounded to nearest as numpy's astype(float32) rounds it)
__device__ __forceinline__ void load4(const float* r, int c, double e[4], float f[4]) {
    const float4 t = reinterpret_cast<const float4*>(r)[c];
    f[0] = t.x; f[1] = t.y; f[2] = t.z; f[3] = t.w;
#pragma unroll
    for (int i = 0; i < 4; ++i) e[i] = (double)f[i];
}
__device__ __forceinline__ void load4(const double* r, int c, double e[4], float f[4]) {
    const double2 t0 = reinterpret_cast<const double2*>(r)[2 * c], t1 = reinterpret_cast<const double2*>(r)[2 * c + 1];
    e[0] = t0.x; e[1] = t0.y; e[2] = t1.x; e[3] = t1.y;
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = (float)e[i];
}

// one workgroup per (row, range) of width n (a multiple of g and of 4); lane t takes elements
// 4t .. 4t + 3 (T: float or double, the input's type)
template <int GL, typename T>     // lanes a group (g / 4); 0: row mode
__global__ __launch_bounds__(256) void fake_act_kernel(const T* __restrict__ x, int64_t ldx, int n, int nr,
                                                       double* __restrict__ v, int64_t ldv,
                                                       uint8_t* __restrict__ da, int64_t ldda) {
    __shared__ uint64_t red[4];
    __shared__ uint32_t redf[4];
    const int row = blockIdx.x / nr, rg = blockIdx.x % nr;
    const int lane = threadIdx.x;
    const T* xr = x + (int64_t)row * ldx + (int64_t)rg * n;
    double* vr = v + (int64_t)row * ldv + (int64_t)rg * n;
    uint8_t* dr = da + (int64_t)row * ldda + (int64_t)rg * (n / EG);
    const int nc = n >> 2;
    // the range's amax: of |x| as given (float64), and of the flushed fp32 |x| (the device
    // quantizer's)
    uint64_t m = 0;
    uint32_t mf = 0;
    for (int c = lane; c < nc; c += 256) {
        double e[4];
        float f[4];
        load4(xr, c, e, f);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            m = max(m, mag64(e[i]));
            mf = max(mf, fbits(ftz(f[i])) & 0x7FFFFFFFu);
        }
    }
    m = wave_max_u64(m, 64);
    mf = wave_max_u32(mf, 64);
    if ((lane & 63) == 0) {
        red[lane >> 6] = m;
        redf[lane >> 6] = mf;
    }
    __syncthreads();
    const uint64_t am = max(max(red[0], red[1]), max(red[2], red[3]));
    const uint32_t amf = max(max(redf[0], redf[1]), max(redf[2], redf[3]));
    const double amax = __longlong_as_double((long long)am);
    const double s = am == 0 ? 1.0 : amax / 127.0;
    int ea = 0;
    const double fam = am ? frexp(amax, &ea) : 0.0;
    const float inv = amf ? fmul(127.0f, recip(bitsf(amf))) : 0.0f;          // the device's
    for (int base = 0; base < nc; base += 256) {          // uniform trip count: shuffles converge
        const int c = base + lane;
        const bool ok = c < nc;
        double e[4] = {0.0, 0.0, 0.0, 0.0};
        float f[4] = {0.f, 0.f, 0.f, 0.f};
        if (ok) load4(xr, c, e, f);
        int d = 0, dd = 0;                                 // float64 offset; the device's
        if (GL > 0) {
            uint64_t g = 0;
            uint32_t gf = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                g = max(g, mag64(e[i]));
                gf = max(gf, fbits(ftz(f[i])) & 0x7FFFFFFFu);
            }
            g = wave_max_u64(g, GL);
            gf = wave_max_u32(gf, GL);
            if (g) {
                int eg = 0;
                const double fg = frexp(__longlong_as_double((long long)g), &eg);
                d = ea - eg - (fg > fam ? 1 : 0);
                d = d < 0 ? 0 : (d > 31 ? 31 : d);
            }
            if (gf) {
                dd = (int)(amf >> 23) - (int)(gf >> 23) - ((gf & 0x7FFFFFu) > (amf & 0x7FFFFFu));
                dd = dd < 0 ? 0 : (dd > 31 ? 31 : dd);
            }
        }
        if (!ok) continue;
        const double unit = __builtin_ldexp(s, -d);
        const float sc = fmul(inv, pow2f(dd));
        double o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const double r = e[i] / unit;
            double q = __builtin_rint(r);
            if (fabs(r - q) > 0.5 - 0x1p-31) q = (double)q8(fmul(f[i], sc));   // a tie: the device's
            q = q < -127.0 ? -127.0 : (q > 127.0 ? 127.0 : q);
            o[i] = q * unit;
        }
        *reinterpret_cast<double2*>(vr + 4 * c) = make_double2(o[0], o[1]);
        *reinterpret_cast<double2*>(vr + 4 * c + 2) = make_double2(o[2], o[3]);
        if ((c & 3) == 0) dr[c >> 2] = (uint8_t)d;
    }
}

// element k's block offset dw and multiplier m from its row's scale row sr (NULL: UNIT, dw 0 and
// m 1; rsc: Sw alone, dw 0 and m 1)
__device__ __forceinline__ int group_dw(const uint8_t* sr, int fmt, int rsc, int k) {
    if (!sr || rsc) return 0;
    const int kb = k / OTPU_D;
    if (fmt == OTPU_INT8) return sr[4 + kb];
    if (fmt == OTPU_NVFP4) {
        const int E = (sr[16 + 8 * kb + ((k % OTPU_D) >> 4)] >> 3) & 15;
        return 15 - (E > 1 ? E : 1);
    }
    return (int)(*reinterpret_cast<const uint32_t*>(sr + 8 + 4 * kb) & 0xFF);
}
__device__ __forceinline__ int group_m(const uint8_t* sr, int fmt, int rsc, int k) {
    if (!sr || rsc || fmt == OTPU_INT8) return 1;
    const int kb = k / OTPU_D;
    if (fmt == OTPU_NVFP4) {
        const int e4 = sr[16 + 8 * kb + ((k % OTPU_D) >> 4)], E = (e4 >> 3) & 15, M = e4 & 7;
        return E ? 8 + M : M;
    }
    return (int)((*reinterpret_cast<const uint32_t*>(sr + 8 + 4 * kb) >> (8 + 6 * ((k % OTPU_D) >> 5))) & 63);
}

// one thread per weight element: value and (for the group's first element) its offset
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ rows, int64_t rs,
                                                      const uint8_t* __restrict__ srows, int64_t srs, int N, int K,
                                                      int fmt, int rsc, double* __restrict__ out, int64_t ldo,
                                                      uint8_t* __restrict__ dwo, int64_t lddw) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)N * K) return;
    const int n = (int)(idx / K), k = (int)(idx % K);
    const uint8_t* sr = srows ? srows + (int64_t)n * srs : nullptr;
    if (!out) {                                            // the offsets alone
        if ((k & (EG - 1)) == 0) dwo[(int64_t)n * lddw + k / EG] = (uint8_t)group_dw(sr, fmt, rsc, k);
        return;
    }
    const uint8_t* wr = rows + (int64_t)n * rs;
    int w;
    if (fmt == OTPU_INT8) {
        w = (int)(int8_t)wr[k];
    } else {
        const int code = (wr[k >> 1] >> (4 * (k & 1))) & 15;
        if (fmt == OTPU_INT4) w = code & 8 ? code - 16 : code;
        else {
            const int mag[8] = {0, 1, 2, 3, 4, 6, 8, 12};     // E2M1 x 2
            w = code & 8 ? -mag[code & 7] : mag[code & 7];
        }
    }
    if (!sr) {                                             // UNIT: the elements themselves
        out[(int64_t)n * ldo + k] = (double)w;
        if (dwo && (k & (EG - 1)) == 0) dwo[(int64_t)n * lddw + k / EG] = 0;
        return;
    }
    const int dw = group_dw(sr, fmt, rsc, k), mm = group_m(sr, fmt, rsc, k);
    float Sw = *reinterpret_cast<const float*>(sr);
    if (fabsf(Sw) < 0x1p-126f) Sw = 0.0f;                  // a denormal Sw (or -0) is +0
    const double scv = (double)mm * __builtin_ldexp(1.0, -dw);
    out[(int64_t)n * ldo + k] = ((double)w * scv) * (double)Sw;
    if (dwo && (k & (EG - 1)) == 0) dwo[(int64_t)n * lddw + k / EG] = (uint8_t)dw;
}

// 16 x 16 outputs a workgroup; a drop group of 16 columns a step, staged in LDS
__global__ __launch_bounds__(256) void mx_matmul_kernel(const double* __restrict__ h, int64_t ldh,
                                                        const uint8_t* __restrict__ da, int64_t ldda,
                                                        const double* __restrict__ w, int64_t ldw,
                                                        const uint8_t* __restrict__ dw, int64_t lddw, int dw_rows,
                                                        int W, int M, int N, int K, double* __restrict__ y,
                                                        int64_t ldy) {
    __shared__ double hs[16][EG + 1], ws[16][EG + 1];
    __shared__ int das[16], dws[16];
    const int t = threadIdx.x, tj = t >> 4, tn = t & 15;
    const int j0 = blockIdx.y * 16, n0 = blockIdx.x * 16;
    const int j = j0 + tj, n = n0 + tn;
    double acc = 0.0;
    for (int g = 0; g < K / EG; ++g) {
        const int jr = min(j0 + tj, M - 1), nr = min(n0 + tj, N - 1);
        hs[tj][tn] = h[(int64_t)jr * ldh + g * EG + tn];
        ws[tj][tn] = w[(int64_t)nr * ldw + g * EG + tn];
        if (t < 16) das[t] = da ? (int)da[(int64_t)min(j0 + t, M - 1) * ldda + g] : 0;
        else if (t < 32) dws[t - 16] = dw ? (int)dw[(int64_t)(dw_rows == 1 ? 0 : min(n0 + t - 16, N - 1)) * lddw + g] : 0;
        __syncthreads();
        if (!da || das[tj] + dws[tn] <= W) {
            double sgrp = 0.0;
#pragma unroll
            for (int i = 0; i < EG; ++i) sgrp += hs[tj][i] * ws[tn][i];
            acc += sgrp;
        }
        __syncthreads();
    }
    if (j < M && n < N) y[(int64_t)j * ldy + n] = acc;
}

}  // namespace otpu

using namespace otpu;

template <typename T>
static int fake_act_launch(const T* x, int M, int K, int64_t ldx, int n, int g, int row_mode, double* v, int64_t ldv,
                           uint8_t* da, int64_t ldda, otpu_stream_t stream) {
    constexpr int V4 = 16 / sizeof(T);                     // elements of a 16-byte load
    if (M < 1 || K < 1 || n < 1 || K % n || ldx < K || ldv < K || ldda < K / EG)
        return otpu_fail(OTPU_EINVAL, "fake_act: M %d, K %d, ranges of %d, ldx %lld", M, K, n, (long long)ldx);
    if (g != 16 && g != 32 && g != 64 && g != 128)
        return otpu_fail(OTPU_EINVAL, "fake_act: groups of %d (16, 32, 64 or 128: whole 16-element groups)", g);
    if (n % g || n % EG || n % 4)
        return otpu_fail(OTPU_EINVAL, "fake_act: ranges of %d are not whole groups of %d and of %d", n, g, EG);
    if (!x || !v || !da || ((uintptr_t)x & 15) || ((uintptr_t)v & 15) || (ldx % V4) || (ldv % 2))
        return otpu_fail(OTPU_EALIGN, "fake_act: x and v 16-byte aligned, row strides of whole 16-byte chunks");
    const dim3 grid(M * (K / n)), block(256);
    hipStream_t s = (hipStream_t)stream;
    const int nr = K / n;
    if (row_mode) {
        fake_act_kernel<0, T><<<grid, block, 0, s>>>(x, ldx, n, nr, v, ldv, da, ldda);
    } else {
        switch (g) {
            case 16: fake_act_kernel<4, T><<<grid, block, 0, s>>>(x, ldx, n, nr, v, ldv, da, ldda); break;
            case 32: fake_act_kernel<8, T><<<grid, block, 0, s>>>(x, ldx, n, nr, v, ldv, da, ldda); break;
            case 64: fake_act_kernel<16, T><<<grid, block, 0, s>>>(x, ldx, n, nr, v, ldv, da, ldda); break;
            default: fake_act_kernel<32, T><<<grid, block, 0, s>>>(x, ldx, n, nr, v, ldv, da, ldda); break;
        }
    }
    return otpu_launch_check("fake_act");
}

extern "C" int otpu_fake_act(const float* x, int M, int K, int64_t ldx, int n, int g, int row_mode, double* v,
                             int64_t ldv, uint8_t* da, int64_t ldda, otpu_stream_t stream) {
    return fake_act_launch(x, M, K, ldx, n, g, row_mode, v, ldv, da, ldda, stream);
}

extern "C" int otpu_fake_act_f64(const double* x, int M, int K, int64_t ldx, int n, int g, int row_mode, double* v,
                                 int64_t ldv, uint8_t* da, int64_t ldda, otpu_stream_t stream) {
    return fake_act_launch(x, M, K, ldx, n, g, row_mode, v, ldv, da, ldda, stream);
}

extern "C" int otpu_dequant(const uint8_t* rows, int64_t rs, const uint8_t* srows, int64_t srs, int N, int K, int fmt,
                            int rsc, double* out, int64_t ldo, uint8_t* dw, int64_t lddw, otpu_stream_t stream) {
    if (fmt < OTPU_INT8 || fmt > OTPU_NVFP4) return otpu_fail(OTPU_EFORMAT, "dequant: format %d", fmt);
    if (rsc && fmt == OTPU_NVFP4) return otpu_fail(OTPU_EFORMAT, "dequant: RSC does not take NVFP4");
    if (N < 1 || K < OTPU_D || K % OTPU_D || (out && (ldo < K || !rows)) || (dw && lddw < K / EG) || (!out && !dw) ||
        (!out && !srows))
        return otpu_fail(OTPU_EINVAL, "dequant: N %d, K %d (whole blocks of %d), values or offsets", N, K, OTPU_D);
    if (srows && (((uintptr_t)srows & 3) || (srs % 4)))
        return otpu_fail(OTPU_EALIGN, "dequant: scale rows 4-byte aligned");
    const int64_t tot = (int64_t)N * K;
    dequant_kernel<<<(unsigned)((tot + 255) / 256), 256, 0, (hipStream_t)stream>>>(rows, rs, srows, srs, N, K, fmt, rsc,
                                                                                  out, ldo, dw, lddw);
    return otpu_launch_check("dequant");
}

extern "C" int otpu_mx_matmul(const double* h, int64_t ldh, const uint8_t* da, int64_t ldda, const double* w,
                              int64_t ldw, const uint8_t* dw, int64_t lddw, int dw_rows, int W, int M, int N, int K,
                              double* y, int64_t ldy, otpu_stream_t stream) {
    if (M < 1 || N < 1 || K < EG || K % EG || ldh < K || ldw < K || ldy < N || !h || !w || !y)
        return otpu_fail(OTPU_EINVAL, "mx_matmul: M %d, N %d, K %d (whole groups of %d)", M, N, K, EG);
    if (dw && dw_rows != 1 && dw_rows != N) return otpu_fail(OTPU_EINVAL, "mx_matmul: dw has %d rows (1 or N)", dw_rows);
    if ((da && ldda < K / EG) || (dw && lddw < K / EG)) return otpu_fail(OTPU_EINVAL, "mx_matmul: offset rows too short");
    const dim3 grid((N + 15) / 16, (M + 15) / 16), block(256);
    mx_matmul_kernel<<<grid, block, 0, (hipStream_t)stream>>>(h, ldh, da, ldda, w, ldw, dw, lddw, dw_rows, W, M, N, K, y,
                                                             ldy);
    return otpu_launch_check("mx_matmul");
}
