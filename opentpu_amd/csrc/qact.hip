// QACT: the row / MX quantizer (fp32.quantize_mx, opentpu/fp32.py:321-343; docs/isa.md:163-178)
// and the int8x / RSC weight packers built on it (opentpu/quant.py:316-322, runtime.py:66-76).
//
// One workgroup of 256 lanes quantizes one row.  A lane owns float4 chunks, so a group of g
// elements is g/4 adjacent lanes and its maximum is a few xor-shuffles; the row maximum is a
// wave reduction plus one LDS exchange.  The row is read twice (max, then quantize), the
// second time from L2; q is written as packed 32-bit words.
#include "otpu_common.h"

namespace otpu {

// one workgroup per (row, range): K columns starting at range r's first, its S at
// S[r * sr + row * lds] (nr ranges a row; one range: the whole row)
template <int GL>   // lanes per group (g / 4); 0: row mode (every offset 0)
__global__ __launch_bounds__(256) void qact_kernel(const float* __restrict__ x, int K, int64_t ldx,
                                                   int8_t* __restrict__ q, int64_t ldq,
                                                   float* __restrict__ S, int64_t lds,
                                                   uint8_t* __restrict__ d, int64_t ldd, int g,
                                                   int dzero, int nr, int64_t sr, const float* __restrict__ xm) {
    __shared__ uint32_t red[4];
    const int row = blockIdx.x / nr, rg = blockIdx.x % nr;
    const int lane = threadIdx.x;
    x += (int64_t)rg * K;
    if (xm) xm += (int64_t)rg * K;
    q += (int64_t)rg * K;
    if (d) d += (int64_t)rg * (K / g);
    S += (int64_t)rg * sr;
    const float4* xr = reinterpret_cast<const float4*>(x + (int64_t)row * ldx);
    const float4* mr = xm ? reinterpret_cast<const float4*>(xm + (int64_t)row * ldx) : nullptr;
    const int nc = K >> 2;
    // the quantized operand: x, or the VOP MUL x * xm (FTZ RNE) when xm is given
    auto elem = [&](int c) {
        float4 v = xr[c];
        if (mr) {
            const float4 u = mr[c];
            v.x = fmul(v.x, u.x); v.y = fmul(v.y, u.y); v.z = fmul(v.z, u.z); v.w = fmul(v.w, u.w);
        }
        return v;
    };

    uint32_t m = 0;
    for (int c = lane; c < nc; c += 256) {
        float4 v = elem(c);
        m = max(m, fbits(ftz(v.x)) & 0x7FFFFFFFu);
        m = max(m, fbits(ftz(v.y)) & 0x7FFFFFFFu);
        m = max(m, fbits(ftz(v.z)) & 0x7FFFFFFFu);
        m = max(m, fbits(ftz(v.w)) & 0x7FFFFFFFu);
    }
    m = wave_max_dpp(m, 64);
    if ((lane & 63) == 0) red[lane >> 6] = m;
    __syncthreads();
    const uint32_t amax = max(max(red[0], red[1]), max(red[2], red[3]));
    const float fa = bitsf(amax);
    const float inv = amax ? fmul(127.0f, recip(fa)) : 0.0f;
    if (lane == 0) S[(int64_t)row * lds] = amax ? fmul(fa, bitsf(0x3C010204u)) : 0.0f;

    int8_t* qr = q + (int64_t)row * ldq;
    uint8_t* dr = d ? d + (int64_t)row * ldd : nullptr;
    for (int base = 0; base < nc; base += 256) {       // uniform trip count: shuffles converge
        const int c = base + lane;
        const bool ok = c < nc;
        float4 v = ok ? elem(c) : make_float4(0.f, 0.f, 0.f, 0.f);
        int dg = 0;
        if (GL > 0) {
            uint32_t gm = max(max(fbits(ftz(v.x)) & 0x7FFFFFFFu, fbits(ftz(v.y)) & 0x7FFFFFFFu),
                              max(fbits(ftz(v.z)) & 0x7FFFFFFFu, fbits(ftz(v.w)) & 0x7FFFFFFFu));
            gm = wave_max_dpp(gm, GL);
            if (gm) {
                dg = (int)(amax >> 23) - (int)(gm >> 23) - ((gm & 0x7FFFFFu) > (amax & 0x7FFFFFu));
                dg = dg < 0 ? 0 : (dg > 31 ? 31 : dg);
            }
        }
        if (ok) {
            const float sc = fmul(inv, pow2f(dg));
            uint32_t p = (uint32_t)(q8(fmul(v.x, sc)) & 0xFF) | ((uint32_t)(q8(fmul(v.y, sc)) & 0xFF) << 8)
                       | ((uint32_t)(q8(fmul(v.z, sc)) & 0xFF) << 16)
                       | ((uint32_t)(q8(fmul(v.w, sc)) & 0xFF) << 24);
            reinterpret_cast<uint32_t*>(qr)[c] = p;
            const int gl = GL > 0 ? GL : (g >> 2);
            if (dr && (c % gl) == 0) dr[c / gl] = (uint8_t)dg;
        }
    }
    if (dr && lane < dzero) dr[K / g + lane] = 0;      // scale-row padding (int8x rows)
}

}  // namespace otpu

using namespace otpu;

static int launch_qact(const float* x, int M, int K, int64_t ldx, int g, int row_mode, int8_t* q,
                       int64_t ldq, float* S, int64_t lds, uint8_t* d, int64_t ldd, int dzero,
                       hipStream_t s, int nr = 1, int64_t sr = 0, const float* xm = nullptr) {
    dim3 grid(M * nr), block(256);
#define OTPU_QACT_ARGS x, K, ldx, q, ldq, S, lds, d, ldd, g, dzero, nr, sr, xm
    if (row_mode) {
        qact_kernel<0><<<grid, block, 0, s>>>(OTPU_QACT_ARGS);
    } else {
        switch (g) {
            case 8: qact_kernel<2><<<grid, block, 0, s>>>(OTPU_QACT_ARGS); break;
            case 16: qact_kernel<4><<<grid, block, 0, s>>>(OTPU_QACT_ARGS); break;
            case 32: qact_kernel<8><<<grid, block, 0, s>>>(OTPU_QACT_ARGS); break;
            case 64: qact_kernel<16><<<grid, block, 0, s>>>(OTPU_QACT_ARGS); break;
            case 128: qact_kernel<32><<<grid, block, 0, s>>>(OTPU_QACT_ARGS); break;
            default: return otpu_fail(OTPU_EINVAL, "qact: group size %d", g);
        }
    }
#undef OTPU_QACT_ARGS
    return otpu_launch_check("qact");
}

static bool al(const void* p, int a) { return ((uintptr_t)p & (uintptr_t)(a - 1)) == 0; }

extern "C" int otpu_qact(const float* x, int M, int K, int64_t ldx, int g, int row_mode, int8_t* q,
                         int64_t ldq, float* S, uint8_t* d, int64_t ldd, otpu_stream_t stream) {
    if (M < 1 || K < 4 || K % 4 || ldx < K || ldq < K)
        return otpu_fail(OTPU_EINVAL, "qact: M %d, K %d, ldx %lld, ldq %lld", M, K, (long long)ldx,
                         (long long)ldq);
    if (!(g == 8 || g == 16 || g == 32 || g == 64 || g == 128) || K % g)
        return otpu_fail(OTPU_EINVAL, "qact: groups of %d over %d columns", g, K);
    if (!x || !q || !S || (!d && !row_mode))
        return otpu_fail(OTPU_EINVAL, "qact: a NULL operand");
    if (d && ldd < K / g) return otpu_fail(OTPU_EINVAL, "qact: ldd %lld < %d", (long long)ldd, K / g);
    if (!al(x, 16) || ldx % 4 || !al(q, 4) || ldq % 4 || !al(S, 4))
        return otpu_fail(OTPU_EALIGN, "qact: x 16-byte aligned, q 4-byte aligned, ldx and ldq multiples of 4");
    return launch_qact(x, M, K, ldx, g, row_mode, q, ldq, S, 1, d, ldd, 0, (hipStream_t)stream);
}

extern "C" int otpu_pack_int8(const float* W, int N, int K, int64_t ldw, int rsc, uint8_t* rows,
                              int64_t rs, uint8_t* srows, int64_t srs, otpu_stream_t stream) {
    if (N < 1 || K < OTPU_D || K % OTPU_D || ldw < K || rs < K)
        return otpu_fail(OTPU_EINVAL, "pack_int8: N %d, K %d, ldw %lld, rs %lld", N, K,
                         (long long)ldw, (long long)rs);
    const int KB = K / OTPU_D;
    const int64_t need = rsc ? 4 : 4 + 4 * ((KB + 3) / 4);
    if (srs < need || srs % 4)
        return otpu_fail(OTPU_EINVAL, "pack_int8: scale rows of %lld bytes, need %lld (a multiple of 4)",
                         (long long)srs, (long long)need);
    if (!al(W, 16) || ldw % 4 || !al(rows, 4) || rs % 4 || !al(srows, 4))
        return otpu_fail(OTPU_EALIGN, "pack_int8: alignment");
    float* S = reinterpret_cast<float*>(srows);
    if (rsc)
        return launch_qact(W, N, K, ldw, K, 1, (int8_t*)rows, rs, S, srs / 4, nullptr, 0, 0,
                           (hipStream_t)stream);
    return launch_qact(W, N, K, ldw, OTPU_D, 0, (int8_t*)rows, rs, S, srs / 4, srows + 4, srs,
                       (int)(srs - 4 - KB), (hipStream_t)stream);
}

extern "C" int otpu_qact_ranges(const float* x, const float* xmul, int M, int K, int64_t ldx, int width, int g,
                                int row_mode, int8_t* q, int64_t ldq, float* S, uint8_t* d, int64_t ldd,
                                otpu_stream_t stream) {
    if (width < 4 || K % width || width % 4)
        return otpu_fail(OTPU_EINVAL, "qact_ranges: ranges of %d over %d columns", width, K);
    if (M < 1 || ldx < K || ldq < K || !x || !q || !S || (!d && !row_mode))
        return otpu_fail(OTPU_EINVAL, "qact_ranges: M %d, K %d, ldx %lld, ldq %lld", M, K, (long long)ldx,
                         (long long)ldq);
    if (!(g == 8 || g == 16 || g == 32 || g == 64 || g == 128) || width % g)
        return otpu_fail(OTPU_EINVAL, "qact_ranges: groups of %d over ranges of %d", g, width);
    if (d && ldd < K / g) return otpu_fail(OTPU_EINVAL, "qact_ranges: ldd %lld < %d", (long long)ldd, K / g);
    if (!al(x, 16) || (xmul && !al(xmul, 16)) || ldx % 4 || !al(q, 4) || ldq % 4 || !al(S, 4))
        return otpu_fail(OTPU_EALIGN, "qact_ranges: alignment");
    const int nr = K / width;
    if ((int64_t)M * nr > 0x7FFFFFFF) return otpu_fail(OTPU_EINVAL, "qact_ranges: %d rows x %d ranges", M, nr);
    return launch_qact(x, M, width, ldx, g, row_mode, q, ldq, S, 1, d, ldd, 0, (hipStream_t)stream, nr, M, xmul);
}
