// QACT: the row / MX quantizer (fp32.quantize_mx, opentpu/fp32.py:321-343; docs/isa.md:163-178)
// with QACT's RSCALE / CSCALE pre-multiplies, its split (LO, HL) and ST records
// (opentpu/isasim.py:913-988, docs/isa.md:444-486), LDA (opentpu/isasim.py:990-1006), and the
// int8x / RSC weight packers built on it (opentpu/quant.py:316-322, runtime.py:66-76; QST LO).
//
// One workgroup of 256 lanes quantizes one row.  A lane owns float4 chunks, so a group of g
// elements is g/4 adjacent lanes and its maximum is a few xor-shuffles; the row maximum is a
// wave reduction plus one LDS exchange.  The row is read twice (max, then quantize), the
// second time from L2; q is written as packed 32-bit words.
#include "otpu_common.h"

namespace otpu {

// one QACT launch: x [rows, ldx] in nr ranges of K columns a row (range rg of row `row` starts at
// column rg * K); its S at S[rg * sr + row * lds]
struct QactArgs {
    const float* x; int64_t ldx;
    const float* xm;            // VOP MUL operand (same shape), or NULL
    const float* rsc;           // RSCALE: a factor per row, or NULL
    const float* csc;           // CSCALE: a factor per column of the whole row, or NULL
    int K, nr, g, dzero;
    int64_t sr;
    int8_t* q; int64_t ldq;
    float* S; int64_t lds;
    uint8_t* d; int64_t ldd;
    int part;                   // 0: q8 (hi), 1: q8lo (the split's lo part), 2: both (HL)
    int64_t qlo;                // HL: the lo bytes' offset in a q row
    float* Slo;                 // HL: the lo part's S, at Slo[row * lds]
    uint8_t* st; int64_t sts;   // QACT ST: rows of K bytes + K / 128 records of 8 bytes, or NULL
};

// the split's lo byte of a product p: sat127(rint(256 p) - 256 q8(p)), NaN -> 0; rint(256 p) is
// exact in fp32 (a power-of-two scaling) and clamped to +-2^16, past which the result saturates
// either way
__device__ __forceinline__ int q8lo(float p) {
    p = ftz(p);
    if (p != p) return 0;
    float t = __builtin_rintf(p * 256.0f);
    t = t > 65536.0f ? 65536.0f : (t < -65536.0f ? -65536.0f : t);
    int r = (int)t - 256 * q8(p);
    return r > 127 ? 127 : (r < -127 ? -127 : r);
}

template <int GL>   // lanes per group (g / 4); 0: row mode (every offset 0)
__global__ __launch_bounds__(256) void qact_kernel(QactArgs a) {
    __shared__ uint32_t red[4];
    const int row = blockIdx.x / a.nr, rg = blockIdx.x % a.nr;
    const int lane = threadIdx.x, K = a.K;
    const float4* xr = reinterpret_cast<const float4*>(a.x + (int64_t)row * a.ldx + (int64_t)rg * K);
    const float4* mr = a.xm ? reinterpret_cast<const float4*>(a.xm + (int64_t)row * a.ldx + (int64_t)rg * K) : nullptr;
    const float4* cr = a.csc ? reinterpret_cast<const float4*>(a.csc + (int64_t)rg * K) : nullptr;
    const float rf = a.rsc ? a.rsc[row] : 1.0f;
    const int nc = K >> 2;
    // the quantized operand: x, times xm (VOP MUL), then (x * r) * c (RSCALE, CSCALE), each an
    // FTZ RNE product
    auto elem = [&](int c) {
        float4 v = xr[c];
        if (mr) {
            const float4 u = mr[c];
            v.x = fmul(v.x, u.x); v.y = fmul(v.y, u.y); v.z = fmul(v.z, u.z); v.w = fmul(v.w, u.w);
        }
        if (a.rsc) { v.x = fmul(v.x, rf); v.y = fmul(v.y, rf); v.z = fmul(v.z, rf); v.w = fmul(v.w, rf); }
        if (cr) {
            const float4 u = cr[c];
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
    const float Shi = amax ? fmul(fa, bitsf(0x3C010204u)) : 0.0f;
    const float Slo = fmul(Shi, pow2f(-8));
    const float Sw = a.part == 1 ? Slo : Shi;                     // the written part's scale
    float* S = a.S + (int64_t)rg * a.sr;
    if (lane == 0) {
        S[(int64_t)row * a.lds] = Sw;
        if (a.part == 2) a.Slo[(int64_t)row * a.lds] = Slo;
    }

    int8_t* qr = a.q + (int64_t)row * a.ldq + (int64_t)rg * K;
    uint8_t* dr = a.d ? a.d + (int64_t)row * a.ldd + (int64_t)rg * (K / a.g) : nullptr;
    uint8_t* str = a.st ? a.st + (int64_t)row * a.sts : nullptr;
    if (str && lane < (K >> 7)) *reinterpret_cast<float*>(str + K + 8 * lane) = Sw;   // block records' S
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
            const float p0 = fmul(v.x, sc), p1 = fmul(v.y, sc), p2 = fmul(v.z, sc), p3 = fmul(v.w, sc);
            uint32_t ph = (uint32_t)(q8(p0) & 0xFF) | ((uint32_t)(q8(p1) & 0xFF) << 8)
                        | ((uint32_t)(q8(p2) & 0xFF) << 16) | ((uint32_t)(q8(p3) & 0xFF) << 24);
            uint32_t pl = 0;
            if (a.part) {
                pl = (uint32_t)(q8lo(p0) & 0xFF) | ((uint32_t)(q8lo(p1) & 0xFF) << 8)
                   | ((uint32_t)(q8lo(p2) & 0xFF) << 16) | ((uint32_t)(q8lo(p3) & 0xFF) << 24);
            }
            const uint32_t pw = a.part == 1 ? pl : ph;
            reinterpret_cast<uint32_t*>(qr)[c] = pw;
            if (a.part == 2) reinterpret_cast<uint32_t*>(qr + a.qlo)[c] = pl;
            if (str) reinterpret_cast<uint32_t*>(str)[c] = pw;
            const int gl = GL > 0 ? GL : (a.g >> 2);
            if ((c % gl) == 0) {
                const int grp = c / gl;
                if (dr) dr[grp] = (uint8_t)dg;
                if (str) str[K + 8 * (grp >> 2) + 4 + (grp & 3)] = (uint8_t)dg;   // record offsets (g 32)
            }
        }
    }
    if (dr && lane < a.dzero) dr[K / a.g + lane] = 0;      // scale-row padding (int8x rows)
}

// LDA: QACT ST rows back into an operand: row r's K = KB * 128 bytes to q[r], block k's record
// to S[k * rows + r] (its scale) and d[r, 4k .. 4k+3] (its offsets); one thread a (row, block)
__global__ __launch_bounds__(256) void lda_kernel(const uint8_t* __restrict__ st, int64_t sts, int rows, int KB,
                                                  int8_t* __restrict__ q, int64_t ldq, float* __restrict__ S,
                                                  uint8_t* __restrict__ d, int64_t ldd) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (int64_t)rows * KB) return;
    const int r = (int)(t / KB), k = (int)(t % KB);
    const uint8_t* src = st + (int64_t)r * sts;
    const uint4* s4 = reinterpret_cast<const uint4*>(src + 128 * k);
    uint4* q4 = reinterpret_cast<uint4*>(q + (int64_t)r * ldq + 128 * k);
#pragma unroll
    for (int i = 0; i < 8; ++i) q4[i] = s4[i];
    const uint2 rec = *reinterpret_cast<const uint2*>(src + 128 * KB + 8 * k);
    S[(int64_t)k * rows + r] = bitsf(rec.x);
    *reinterpret_cast<uint32_t*>(d + (int64_t)r * ldd + 4 * k) = rec.y;
}

}  // namespace otpu

using namespace otpu;

static int launch_qact(const QactArgs& a, int M, int row_mode, hipStream_t s) {
    dim3 grid(M * a.nr), block(256);
    if (row_mode) {
        qact_kernel<0><<<grid, block, 0, s>>>(a);
    } else {
        switch (a.g) {
            case 8: qact_kernel<2><<<grid, block, 0, s>>>(a); break;
            case 16: qact_kernel<4><<<grid, block, 0, s>>>(a); break;
            case 32: qact_kernel<8><<<grid, block, 0, s>>>(a); break;
            case 64: qact_kernel<16><<<grid, block, 0, s>>>(a); break;
            case 128: qact_kernel<32><<<grid, block, 0, s>>>(a); break;
            default: return otpu_fail(OTPU_EINVAL, "qact: group size %d", a.g);
        }
    }
    return otpu_launch_check("qact");
}

static QactArgs qact_args(const float* x, int K, int64_t ldx, int g, int8_t* q, int64_t ldq, float* S,
                          int64_t lds, uint8_t* d, int64_t ldd) {
    QactArgs a = {};
    a.x = x; a.ldx = ldx; a.K = K; a.nr = 1; a.g = g; a.q = q; a.ldq = ldq; a.S = S; a.lds = lds;
    a.d = d; a.ldd = ldd;
    return a;
}

static bool al(const void* p, int a) { return ((uintptr_t)p & (uintptr_t)(a - 1)) == 0; }

extern "C" int otpu_qact(const float* x, int M, int K, int64_t ldx, int g, int flags, const float* rscale,
                         const float* cscale, int8_t* q, int64_t ldq, float* S, uint8_t* d, int64_t ldd,
                         uint8_t* qrows, int64_t qrs, otpu_stream_t stream) {
    const int row_mode = flags & OTPU_Q_ROW, lo = (flags & OTPU_Q_LO) != 0, hl = (flags & OTPU_Q_HL) != 0;
    if (flags & ~(OTPU_Q_ROW | OTPU_Q_LO | OTPU_Q_HL)) return otpu_fail(OTPU_EINVAL, "qact: unknown flags %#x", flags);
    if (lo && hl) return otpu_fail(OTPU_EINVAL, "qact: HL with LO");
    if (hl && qrows) return otpu_fail(OTPU_EINVAL, "qact: ST with HL");
    if (M < 1 || K < 4 || K % 4 || ldx < K || ldq < (hl ? 2 * (int64_t)K : K))
        return otpu_fail(OTPU_EINVAL, "qact: M %d, K %d, ldx %lld, ldq %lld", M, K, (long long)ldx,
                         (long long)ldq);
    if (!(g == 8 || g == 16 || g == 32 || g == 64 || g == 128) || K % g)
        return otpu_fail(OTPU_EINVAL, "qact: groups of %d over %d columns", g, K);
    if (!x || !q || !S || (!d && !row_mode))
        return otpu_fail(OTPU_EINVAL, "qact: a NULL operand");
    if (d && ldd < K / g) return otpu_fail(OTPU_EINVAL, "qact: ldd %lld < %d", (long long)ldd, K / g);
    if (!al(x, 16) || ldx % 4 || !al(q, 4) || ldq % 4 || !al(S, 4) || (cscale && !al(cscale, 16)))
        return otpu_fail(OTPU_EALIGN, "qact: x and cscale 16-byte aligned, q 4-byte aligned, ldx and ldq multiples of 4");
    if (qrows) {
        if (g != 32 || K % OTPU_D || K > 256 * OTPU_D || !d)
            return otpu_fail(OTPU_EINVAL, "qact: ST records hold 4 offsets of 32 a block (g 32, K a multiple of 128, "
                             "at most 256 blocks)");
        const int64_t need = (int64_t)K + 8 * (K / OTPU_D);
        if (!al(qrows, OTPU_QALIGN) || (M > 1 && (qrs % OTPU_QALIGN || qrs < need)))
            return otpu_fail(OTPU_EINVAL, "qact: ST rows at multiples of %d bytes, %lld bytes each", OTPU_QALIGN,
                             (long long)need);
    }
    QactArgs a = qact_args(x, K, ldx, g, q, ldq, S, 1, d, ldd);
    a.rsc = rscale; a.csc = cscale;
    a.part = hl ? 2 : (lo ? 1 : 0);
    a.qlo = K; a.Slo = S + M;
    a.st = qrows; a.sts = qrs;
    return launch_qact(a, M, row_mode, (hipStream_t)stream);
}

extern "C" int otpu_lda(const uint8_t* qrows, int64_t qrs, int rows, int KB, int8_t* q, int64_t ldq, float* S,
                        uint8_t* d, int64_t ldd, otpu_stream_t stream) {
    if (rows < 1 || KB < 1 || !qrows || !q || !S || !d)
        return otpu_fail(OTPU_EINVAL, "lda: rows %d, KB %d, a NULL operand", rows, KB);
    const int64_t need = (int64_t)KB * (OTPU_D + 8);
    if (!al(qrows, OTPU_QALIGN) || (rows > 1 && (qrs % OTPU_QALIGN || qrs < need)))
        return otpu_fail(OTPU_EINVAL, "lda: rows at multiples of %d bytes, %lld bytes each", OTPU_QALIGN, (long long)need);
    if (ldq < (int64_t)KB * OTPU_D || ldq % 16 || !al(q, 16) || ldd < 4 * KB || ldd % 4 || !al(d, 4) || !al(S, 4))
        return otpu_fail(OTPU_EALIGN, "lda: q 16-byte aligned (ldq a multiple of 16), d 4-byte aligned");
    const int64_t n = (int64_t)rows * KB;
    lda_kernel<<<(unsigned)((n + 255) / 256), 256, 0, (hipStream_t)stream>>>(qrows, qrs, rows, KB, q, ldq, S, d, ldd);
    return otpu_launch_check("lda");
}

extern "C" int otpu_pack_int8(const float* W, int N, int K, int64_t ldw, int flags, uint8_t* rows,
                              int64_t rs, uint8_t* srows, int64_t srs, otpu_stream_t stream) {
    const int rsc = flags & OTPU_Q_ROW, lo = (flags & OTPU_Q_LO) != 0;
    if (flags & ~(OTPU_Q_ROW | OTPU_Q_LO)) return otpu_fail(OTPU_EINVAL, "pack_int8: unknown flags %#x", flags);
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
    QactArgs a = qact_args(W, K, ldw, rsc ? K : OTPU_D, (int8_t*)rows, rs, S, srs / 4,
                           rsc ? nullptr : srows + 4, srs);
    a.dzero = rsc ? 0 : (int)(srs - 4 - KB);
    a.part = lo ? 1 : 0;
    return launch_qact(a, N, rsc, (hipStream_t)stream);
}

extern "C" int otpu_qact_ranges(const float* x, const float* xmul, int M, int K, int64_t ldx, int width, int g,
                                int flags, const float* rscale, const float* cscale, int8_t* q, int64_t ldq, float* S,
                                uint8_t* d, int64_t ldd, otpu_stream_t stream) {
    const int row_mode = flags & OTPU_Q_ROW, lo = (flags & OTPU_Q_LO) != 0;
    if (flags & ~(OTPU_Q_ROW | OTPU_Q_LO)) return otpu_fail(OTPU_EINVAL, "qact_ranges: flags %#x (ROW, LO)", flags);
    if (width < 4 || K % width || width % 4)
        return otpu_fail(OTPU_EINVAL, "qact_ranges: ranges of %d over %d columns", width, K);
    if (M < 1 || ldx < K || ldq < K || !x || !q || !S || (!d && !row_mode))
        return otpu_fail(OTPU_EINVAL, "qact_ranges: M %d, K %d, ldx %lld, ldq %lld", M, K, (long long)ldx,
                         (long long)ldq);
    if (!(g == 8 || g == 16 || g == 32 || g == 64 || g == 128) || width % g)
        return otpu_fail(OTPU_EINVAL, "qact_ranges: groups of %d over ranges of %d", g, width);
    if (d && ldd < K / g) return otpu_fail(OTPU_EINVAL, "qact_ranges: ldd %lld < %d", (long long)ldd, K / g);
    if (!al(x, 16) || (xmul && !al(xmul, 16)) || (cscale && !al(cscale, 16)) || ldx % 4 || !al(q, 4) || ldq % 4 ||
        !al(S, 4))
        return otpu_fail(OTPU_EALIGN, "qact_ranges: alignment");
    const int nr = K / width;
    if ((int64_t)M * nr > 0x7FFFFFFF) return otpu_fail(OTPU_EINVAL, "qact_ranges: %d rows x %d ranges", M, nr);
    QactArgs a = qact_args(x, width, ldx, g, q, ldq, S, 1, d, ldd);
    a.nr = nr; a.sr = M; a.xm = xmul; a.rsc = rscale; a.csc = cscale;
    a.part = lo ? 1 : 0;
    return launch_qact(a, M, row_mode, (hipStream_t)stream);
}
