// MM SPL: one MM over a split operand's terms (opentpu/isasim.py:757-770, :849-852, :872-873;
// docs/isa.md:414-441), natural rows.  The operands are split by the quantizer (QACT HL for the
// activations, QST LO for the weights): x ~ (hi + lo / 256) S 2^-d.  One K-block (D = 128) of
// int8 RSC weights a part; advance k takes an activation block, a weight part and an extra
// offset e_k:
//   3 terms: (hi, w_hi, 0), (lo, w_hi, 8), (hi, w_lo, 8)      2 terms: (hi, w_hi, 0), (hi, w_lo, 8)
// acc = sum over advances and 32-groups of c << (16 - da - e_k) (a term whose shift is negative
// adds nothing), one exact integer an output, then the epilogue (i2f(acc) * Sw) * (Sa * 2^-16)
// with the hi part's Sa and Sw: the split product rounded once.
//
// A team of 16 lanes owns a weight row: a part is 8 pieces of 16 bytes, so the (at most) 24
// pieces of the advances are lane tl's tl and tl + 16.  The row's weight pieces stay in registers
// while the team walks the activation rows; a row's sum is a 16-lane reduction of exact int64s.
#include "otpu_common.h"

namespace otpu {

__global__ __launch_bounds__(256) void mm_spl_kernel(const int8_t* __restrict__ q, int64_t ldq,
                                                     const float* __restrict__ Sa, const uint8_t* __restrict__ da,
                                                     int64_t ldda, int M, int nterms, const uint8_t* __restrict__ w,
                                                     int64_t rs, int64_t hld, const uint8_t* __restrict__ ws,
                                                     int64_t srs, int N, int acc, float* __restrict__ out, int64_t ors) {
    const int lane = threadIdx.x & 63, tl = lane & 15;
    const int n = (int)(((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 4);
    const bool live = n < N;
    const int nr = live ? n : N - 1;                          // rows past N load row N-1, store nothing
    // advance table: activation block, weight part, extra offset
    const int np = 8 * nterms;
    int ablk[2], e[2], grp[2], off[2];
    bool on[2];
    uint4 wv[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int p = tl + 16 * i;
        on[i] = p < np;
        const int k = on[i] ? p >> 3 : 0;
        const int wpart = nterms == 3 ? (k == 2) : (k == 1);
        ablk[i] = nterms == 3 ? (k == 1) : 0;
        e[i] = k ? 8 : 0;
        off[i] = (p & 7) * 16;
        grp[i] = (p & 7) >> 1;
        wv[i] = on[i] ? *reinterpret_cast<const uint4*>(w + (int64_t)nr * rs + (wpart ? hld : 0) + off[i])
                      : make_uint4(0, 0, 0, 0);
    }
    const float sw = ftz(*reinterpret_cast<const float*>(ws + (int64_t)nr * srs));
    for (int j = 0; j < M; ++j) {
        int64_t t = 0;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            if (!on[i]) continue;
            const uint4 av = *reinterpret_cast<const uint4*>(q + (int64_t)j * ldq + 128 * ablk[i] + off[i]);
            int c = __builtin_amdgcn_sdot4((int)wv[i].x, (int)av.x, 0, false);
            c = __builtin_amdgcn_sdot4((int)wv[i].y, (int)av.y, c, false);
            c = __builtin_amdgcn_sdot4((int)wv[i].z, (int)av.z, c, false);
            c = __builtin_amdgcn_sdot4((int)wv[i].w, (int)av.w, c, false);
            const int sh = 16 - ((int)da[(int64_t)j * ldda + grp[i]] + e[i]);
            if (sh >= 0) t += (int64_t)c << sh;
        }
#pragma unroll
        for (int o = 8; o > 0; o >>= 1) t += __shfl_xor(t, o, 16);
        if (tl == 0 && live) {
            float y = fmul_f(fmul_f(i2f(t), sw), fmul(Sa[j], pow2f(-16)));
            float* op = out + (int64_t)j * ors + n;
            if (acc) y = fadd(*op, y);
            *op = y;
        }
    }
}

}  // namespace otpu

using namespace otpu;

static bool al(const void* p, int a) { return ((uintptr_t)p & (uintptr_t)(a - 1)) == 0; }

extern "C" int otpu_mm_spl(const int8_t* q, int64_t ldq, const float* Sa, const uint8_t* da, int64_t ldda, int M,
                           int nterms, const uint8_t* w, int64_t rs, int64_t hld, const uint8_t* ws, int64_t srs,
                           int N, int flags, float* out, int64_t ors, otpu_stream_t stream) {
    if (nterms != 2 && nterms != 3) return otpu_fail(OTPU_EINVAL, "mm_spl: %d terms (2 or 3)", nterms);
    if (!(flags & OTPU_RSC) || (flags & ~(OTPU_RSC | OTPU_ACC)))
        return otpu_fail(OTPU_EINVAL, "mm_spl: int8 RSC weights, no flags but ACC (not UNIT, PAIR, RMAX or ASCALE)");
    if (M < 1 || N < 1 || !q || !Sa || !da || !w || !ws || !out)
        return otpu_fail(OTPU_EINVAL, "mm_spl: M %d, N %d, a NULL operand", M, N);
    if (ldq < (nterms == 3 ? 256 : 128) || ldda < 4 || rs < 128 || hld < 128 || srs < 4 || ors < N)
        return otpu_fail(OTPU_EINVAL, "mm_spl: ldq %lld, ldda %lld, rs %lld, hld %lld, srs %lld, ors %lld",
                         (long long)ldq, (long long)ldda, (long long)rs, (long long)hld, (long long)srs, (long long)ors);
    if (!al(q, 16) || ldq % 16 || !al(w, 16) || rs % 16 || hld % 16 || !al(ws, 4) || srs % 4)
        return otpu_fail(OTPU_EALIGN, "mm_spl: q, w, rs, hld 16-byte aligned; ws, srs 4");
    const int64_t threads = (int64_t)N * 16;
    mm_spl_kernel<<<(unsigned)((threads + 255) / 256), 256, 0, (hipStream_t)stream>>>(
        q, ldq, Sa, da, ldda, M, nterms, w, rs, hld, ws, srs, N, (flags & OTPU_ACC) != 0, out, ors);
    return otpu_launch_check("mm_spl");
}
