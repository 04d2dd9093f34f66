// MM for few activation rows: the host side of the decode GEMV (argument checks, launch
// shapes, the C ABI entry points), the LM head with the greedy argmax fused into the GEMV
// epilogue, VOP ARGMAX and the small helper kernels.  The streaming kernel itself is
// gemv_impl.h.  Semantics: opentpu/isasim.py:706-910 (MM), :1141-1152 (ARGMAX).
#include <cstdlib>

#include "gemv_args.h"

namespace otpu {

// a fill kernel (graph-capture friendly, no memset nodes)
__global__ void fill_u32(uint32_t* p, int n, uint32_t v) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

__global__ void rmax_finish(uint32_t* k, int n) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) k[i] = fbits(unkey(k[i]));
}

// the ACC chain of R partial MM outputs: out = add(..add(add(old | part_0, part_1)..), part_R-1)
__global__ void sum_parts(const float* __restrict__ part, int64_t pstride, int R, int M, int N, int acc,
                          float* __restrict__ out, int64_t ors) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)M * N) return;
    const int j = (int)(i / N), n = (int)(i % N);
    const float* p = part + (int64_t)j * N + n;
    float* o = out + (int64_t)j * ors + n;
    float y = acc ? fadd(*o, p[0]) : p[0];
    for (int r = 1; r < R; ++r) y = fadd(y, p[r * pstride]);
    *o = y;
}

// the LM head's last step: the maximum over the running maxima (state[LM_STRIDE (1 + j)], one
// a lane) becomes the result state[0] and the token; the maxima are cleared for the next call
__global__ __launch_bounds__(64) void best_finish(uint64_t* state, int32_t* token) {
    static_assert(LM_WORDS == 64, "one word a lane");
    static_assert(8 * LM_STRIDE * (1 + LM_WORDS) == OTPU_LM_STATE_BYTES, "the state's size in otpu.h");
    uint64_t* w = state + LM_STRIDE * (1 + threadIdx.x);
    const uint64_t m = wave_max_u64(*w);
    *w = 0;
    if (threadIdx.x == 0) {
        state[0] = m;
        *token = (int32_t)~(uint32_t)(m & 0xFFFFFFFFull);
    }
}

// VOP ARGMAX: one workgroup per row; (max, i2f(index + base))
__global__ __launch_bounds__(256) void argmax_rows(const float* __restrict__ x, int cols, int64_t ldx,
                                                    int64_t base, float* pairs, int64_t drs) {
    __shared__ uint64_t red[4];
    const float* xr = x + (int64_t)blockIdx.x * ldx;
    uint64_t best = 0;
    for (int c = threadIdx.x; c < cols; c += 256) {
        uint64_t cand = ((uint64_t)fkey(xr[c]) << 32) | (uint32_t)~(uint32_t)c;
        best = cand > best ? cand : best;
    }
    best = wave_max_u64(best);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t b = red[0];
        for (int i = 1; i < 4; ++i) b = red[i] > b ? red[i] : b;
        const uint32_t idx = ~(uint32_t)(b & 0xFFFFFFFFu);
        float* o = pairs + (int64_t)blockIdx.x * drs;
        o[0] = unkey((uint32_t)(b >> 32));
        o[1] = i2f((int64_t)(int32_t)(uint32_t)((int64_t)idx + base));
    }
}

}  // namespace otpu

using namespace otpu;

static bool al(const void* p, int a) { return ((uintptr_t)p & (uintptr_t)(a - 1)) == 0; }

// the SimError-style checks of one MM (opentpu/isasim.py:767-822, the fields of isa.py:502-548)
static int check_mm(const char* who, const int8_t* q, int64_t ldq, const uint8_t* da, int64_t ldda,
                    int M, int K, const uint8_t* w, int64_t rs, const uint8_t* ws, int64_t srs,
                    int N, int fmt, int flags, int k0) {
    if (fmt < OTPU_INT8 || fmt > OTPU_NVFP4) return otpu_fail(OTPU_EFORMAT, "%s: weight format %d", who, fmt);
    if (M < 1 || N < 1 || K < OTPU_D || K % OTPU_D || k0 < 0)
        return otpu_fail(OTPU_EINVAL, "%s: M %d, N %d, K %d (a multiple of %d), k0 %d", who, M, N, K, OTPU_D, k0);
    if ((flags & OTPU_RSC) && fmt == OTPU_NVFP4) return otpu_fail(OTPU_EFORMAT, "%s: RSC does not take NVFP4", who);
    if ((flags & OTPU_ASCALE) && !((flags & OTPU_UNIT) && (flags & OTPU_ACC)))
        return otpu_fail(OTPU_EINVAL, "%s: ASCALE needs UNIT and ACC", who);
    if (flags & ~(OTPU_UNIT | OTPU_ACC | OTPU_RMAX | OTPU_ASCALE | OTPU_PAIR | OTPU_RSC))
        return otpu_fail(OTPU_EINVAL, "%s: unknown flags %#x", who, flags);
    const int KB = K / OTPU_D;
    const int64_t rowb = fmt == OTPU_INT8 ? K : K / 2;
    if (!q || !da || !w) return otpu_fail(OTPU_EINVAL, "%s: a NULL operand", who);
    if (ldq < K || ldda < K / 32 || rs < rowb)
        return otpu_fail(OTPU_EINVAL, "%s: ldq %lld, ldda %lld, rs %lld too small", who, (long long)ldq,
                         (long long)ldda, (long long)rs);
    if (!(flags & OTPU_UNIT)) {
        if (!ws) return otpu_fail(OTPU_EINVAL, "%s: NULL scale rows", who);
        int64_t need = 4;
        if (!(flags & OTPU_RSC))
            need = fmt == OTPU_INT8 ? 4 + k0 + KB : fmt == OTPU_NVFP4 ? 16 + 8 * (k0 + KB) : 8 + 4 * (k0 + KB);
        const int sal = fmt == OTPU_NVFP4 ? 16 : (fmt == OTPU_INT8 || (flags & OTPU_RSC)) ? 4 : 8;
        if (srs < need) return otpu_fail(OTPU_EINVAL, "%s: scale rows of %lld bytes, blocks k0 %d + %d need %lld",
                                         who, (long long)srs, k0, KB, (long long)need);
        if (!al(ws, 4) || srs % sal)
            return otpu_fail(OTPU_EALIGN, "%s: ssa and srs must be multiples of %d", who, sal);
    }
    if (!al(w, 16) || rs % 16 || !al(q, 16) || ldq % 16)
        return otpu_fail(OTPU_EALIGN, "%s: weight rows and activations 16-byte aligned (w, rs, q, ldq)", who);
    if (rs >= (1 << 24) || srs >= (1 << 24))
        return otpu_fail(OTPU_EINVAL, "%s: row strides of 16 MiB or more", who);
    if (K > KMAX_MM) return otpu_fail(OTPU_EINVAL, "%s: K %d (at most %d: fewer than 256 blocks)", who, K, KMAX_MM);
    return OTPU_OK;
}

// lanes per row: the team size in {64, 32, 16} that wastes the fewest lane pieces; a row of
// more than 64 LMAX pieces takes teams of 64 with LMAX pieces a lane, walked in segments
static void pick_team(int P, int* T, int* L, int* nseg = nullptr) {
    int bt = 64, bl = (P + 63) / 64, bw = bl * 64 - P;
    for (int t = 32; t >= 16; t >>= 1) {
        int l = (P + t - 1) / t, w = l * t - P;
        if (l <= LMAX && w < bw) { bt = t; bl = l; bw = w; }
    }
    if (bl == 7) bl = 8;                        // (no L = 7 instantiation: the eighth is masked)
    const int ns = bl > LMAX ? (bl + LMAX - 1) / LMAX : 1;
    if (bl > LMAX) bl = LMAX;
    *T = bt;
    *L = bl;
    if (nseg) *nseg = ns;
}

static int mr_max(int fmt, int L) {
    return fits_rt(fmt, 4, L) ? 4 : (fits_rt(fmt, 2, L) ? 2 : 1);
}

static int launch_gemv(MMArgs a, int fmt, int batch, hipStream_t s) {
    const int64_t rowb = fmt == OTPU_INT8 ? a.K : a.K / 2;
    a.P = (int)(rowb / 16);
    int L = 1;
    pick_team(a.P, &a.T, &L, &a.nseg);
    const int M = a.M, cap = mr_max(fmt, L);
    for (int j0 = 0; j0 < M; j0 += cap) {        // activation rows in chunks the registers hold
        MMArgs c = a;
        c.M = M - j0 < cap ? M - j0 : cap;
        const int mr = c.M == 1 ? 1 : (c.M == 2 ? 2 : 4);
        c.q = a.q + j0 * a.ldq;
        if (a.Sa) c.Sa = a.Sa + j0;
        c.da = a.da + j0 * a.ldda;
        if (c.out) c.out = a.out + j0 * a.ors;
        if (c.alpha) c.alpha = a.alpha + j0;
        if (c.rmax_key) c.rmax_key = a.rmax_key + j0;
        if (c.acc_out) c.acc_out = a.acc_out + (int64_t)j0 * a.N;
        switch (fmt) {
            case OTPU_INT8: launch_fmt<OTPU_INT8>(c, mr, L, batch, s); break;
            case OTPU_INT4: launch_fmt<OTPU_INT4>(c, mr, L, batch, s); break;
            case OTPU_FP4: launch_fmt<OTPU_FP4>(c, mr, L, batch, s); break;
            default: launch_fmt<OTPU_NVFP4>(c, mr, L, batch, s); break;
        }
    }
    return otpu_launch_check("mm");
}

static MMArgs make_args(const int8_t* q, int64_t ldq, const float* Sa, const uint8_t* da, int64_t ldda, int M,
                        int K, const uint8_t* w, int64_t rs, const uint8_t* ws, int64_t srs, int N, int flags,
                        int k0) {
    MMArgs a = {};
    a.q = q; a.ldq = ldq; a.Sa = Sa; a.da = da; a.ldda = ldda; a.M = M; a.K = K;
    a.w = w; a.rs = rs; a.ws = ws; a.srs = srs; a.N = N; a.flags = flags & ~OTPU_PAIR; a.k0 = k0;
    return a;
}

int otpu_gemm_try(const int8_t* q, int64_t ldq, const float* Sa, const uint8_t* da, int64_t ldda, int M, int K,
                  const uint8_t* w, int64_t rs, const uint8_t* ws, int64_t srs, int N, int fmt, int flags, int k0,
                  const float* alpha, float* out, int64_t ors, hipStream_t s);
int otpu_gemm4_try(const int8_t* q, int64_t ldq, const float* Sa, const uint8_t* da, int64_t ldda, int M, int K,
                   const uint8_t* w, int64_t rs, const uint8_t* ws, int64_t srs, int N, int fmt, int flags, int k0,
                   const float* alpha, float* out, int64_t ors, hipStream_t s);

extern "C" int otpu_mm(const int8_t* q, int64_t ldq, const float* Sa, const uint8_t* da, int64_t ldda,
                       int M, int K, const uint8_t* w, int64_t rs, const uint8_t* ws, int64_t srs, int N,
                       int fmt, int flags, int k0, const float* alpha, float* out, int64_t ors,
                       float* rowmax, otpu_stream_t stream) {
    int rc = check_mm("mm", q, ldq, da, ldda, M, K, w, rs, ws, srs, N, fmt, flags, k0);
    if (rc) return rc;
    if (!Sa || !out || ors < N) return otpu_fail(OTPU_EINVAL, "mm: Sa / out NULL or ors < N");
    if ((flags & OTPU_ASCALE) && !alpha) return otpu_fail(OTPU_EINVAL, "mm: ASCALE without alpha");
    if ((flags & OTPU_RMAX) && !rowmax) return otpu_fail(OTPU_EINVAL, "mm: RMAX without rowmax");
    hipStream_t s = (hipStream_t)stream;
    if (M > 4) {
        rc = otpu_gemm_try(q, ldq, Sa, da, ldda, M, K, w, rs, ws, srs, N, fmt, flags & ~OTPU_PAIR, k0, alpha,
                           out, ors, s);
        if (rc <= 0) return rc;                       // handled (or failed); > 0: not this path
        rc = otpu_gemm4_try(q, ldq, Sa, da, ldda, M, K, w, rs, ws, srs, N, fmt, flags & ~OTPU_PAIR, k0, alpha,
                            out, ors, s);
        if (rc <= 0) return rc;
    }
    MMArgs a = make_args(q, ldq, Sa, da, ldda, M, K, w, rs, ws, srs, N, flags, k0);
    a.alpha = alpha; a.out = out; a.ors = ors;
    if (flags & OTPU_RMAX) {
        a.rmax_key = reinterpret_cast<uint32_t*>(rowmax);
        fill_u32<<<(M + 255) / 256, 256, 0, s>>>(a.rmax_key, M, 0u);
    }
    rc = launch_gemv(a, fmt, 1, s);
    if (rc) return rc;
    if (flags & OTPU_RMAX) {
        rmax_finish<<<(M + 255) / 256, 256, 0, s>>>(a.rmax_key, M);
        return otpu_launch_check("mm rmax");
    }
    return OTPU_OK;
}

extern "C" int otpu_mm_acc(const int8_t* q, int64_t ldq, const uint8_t* da, int64_t ldda, int M, int K,
                           const uint8_t* w, int64_t rs, const uint8_t* ws, int64_t srs, int N, int fmt,
                           int flags, int k0, int64_t* acc, otpu_stream_t stream) {
    int rc = check_mm("mm_acc", q, ldq, da, ldda, M, K, w, rs, ws, srs, N, fmt,
                      flags & ~(OTPU_ACC | OTPU_ASCALE | OTPU_RMAX), k0);
    if (rc) return rc;
    if (!acc) return otpu_fail(OTPU_EINVAL, "mm_acc: NULL acc");
    MMArgs a = make_args(q, ldq, nullptr, da, ldda, M, K, w, rs, ws, srs, N,
                         flags & ~(OTPU_ACC | OTPU_ASCALE | OTPU_RMAX), k0);
    a.acc_out = acc;
    return launch_gemv(a, fmt, 1, (hipStream_t)stream);
}

extern "C" int otpu_mm_batched(int B, const int8_t* q, int64_t ldq, int64_t q_bstride, const float* Sa,
                               int64_t sa_bstride, const uint8_t* da, int64_t ldda, int64_t da_bstride, int M,
                               int K, const uint8_t* w, int64_t rs, int64_t w_bstride, const uint8_t* ws,
                               int64_t srs, int64_t ws_bstride, int N, int fmt, int flags, int k0, float* out,
                               int64_t ors, int64_t out_bstride, otpu_stream_t stream) {
    if (B < 1 || B > 65535) return otpu_fail(OTPU_EINVAL, "mm_batched: B %d", B);
    if (flags & (OTPU_ACC | OTPU_ASCALE | OTPU_RMAX))
        return otpu_fail(OTPU_EINVAL, "mm_batched: no ACC, ASCALE or RMAX");
    int rc = check_mm("mm_batched", q, ldq, da, ldda, M, K, w, rs, ws, srs, N, fmt, flags, k0);
    if (rc) return rc;
    if (!Sa || !out || ors < N) return otpu_fail(OTPU_EINVAL, "mm_batched: Sa / out NULL or ors < N");
    if (q_bstride % 16 || w_bstride % 16 || (!(flags & OTPU_UNIT) && ws_bstride % 4))
        return otpu_fail(OTPU_EALIGN, "mm_batched: batch strides keep the operands aligned");
    MMArgs a = make_args(q, ldq, Sa, da, ldda, M, K, w, rs, ws, srs, N, flags, k0);
    a.out = out; a.ors = ors;
    a.q_bs = q_bstride; a.sa_bs = sa_bstride; a.da_bs = da_bstride;
    a.w_bs = w_bstride; a.ws_bs = ws_bstride; a.out_bs = out_bstride;
    return launch_gemv(a, fmt, B, (hipStream_t)stream);
}

extern "C" int otpu_mm_ranges(const int8_t* q, int64_t ldq, const float* Sa, const uint8_t* da, int64_t ldda,
                              int M, int K, int width, const uint8_t* w, int64_t rs, const uint8_t* ws, int64_t srs,
                              int N, int fmt, int flags, int k0, float* part, float* out, int64_t ors,
                              otpu_stream_t stream) {
    const int chunk = fmt == OTPU_INT8 ? OTPU_D : 2 * OTPU_D;
    if (width < chunk || width % chunk || K % width)
        return otpu_fail(OTPU_EINVAL, "mm_ranges: ranges of %d over K %d (multiples of %d for this format)", width,
                         K, chunk);
    if (flags & (OTPU_ASCALE | OTPU_RMAX)) return otpu_fail(OTPU_EINVAL, "mm_ranges: no ASCALE or RMAX");
    const int R = K / width;
    const bool plain = (flags & (OTPU_UNIT | OTPU_RSC)) != 0;
    int rc = check_mm("mm_ranges", q, ldq, da, ldda, M, width, w, rs, ws, srs, N, fmt, flags & ~OTPU_ACC,
                      plain ? k0 : k0 + (K - width) / OTPU_D);
    if (rc) return rc;
    if (ldq < K || ldda < K / 32 || rs < (fmt == OTPU_INT8 ? K : K / 2))
        return otpu_fail(OTPU_EINVAL, "mm_ranges: ldq %lld, ldda %lld, rs %lld short of K %d", (long long)ldq,
                         (long long)ldda, (long long)rs, K);
    if (!Sa || !part || !out || ors < N) return otpu_fail(OTPU_EINVAL, "mm_ranges: Sa / part / out NULL or ors < N");
    if (!al(part, 4)) return otpu_fail(OTPU_EALIGN, "mm_ranges: part");
    hipStream_t s = (hipStream_t)stream;
    MMArgs a = make_args(q, ldq, Sa, da, ldda, M, width, w, rs, ws, srs, N, flags & ~OTPU_ACC, k0);
    a.out = part; a.ors = N;
    a.q_bs = width; a.sa_bs = M; a.da_bs = width / 32;
    a.w_bs = fmt == OTPU_INT8 ? width : width / 2; a.ws_bs = 0; a.out_bs = (int64_t)M * N;
    a.k0_bs = plain ? 0 : width / OTPU_D;
    rc = launch_gemv(a, fmt, R, s);
    if (rc) return rc;
    const int64_t tot = (int64_t)M * N;
    sum_parts<<<(unsigned)((tot + 255) / 256), 256, 0, s>>>(part, (int64_t)M * N, R, M, N, (flags & OTPU_ACC) != 0,
                                                            out, ors);
    return otpu_launch_check("mm_ranges");
}

namespace otpu {
// the checks and the argument block of one otpu_mm_qin (pieces a lane in *L; also the persistent
// chain's linears)
int qin_args(MMArgs* ap, int* Lp, const float* x, const float* xmul, const float* rscale, const float* cscale,
             int nsum, int64_t sum_stride, int K, int width, const uint8_t* w, int64_t rs, const uint8_t* ws,
             int64_t srs, int N, int fmt, int flags, int k0, float* out, int64_t ors, int64_t part_stride) {
    const int chunk = fmt == OTPU_INT8 ? OTPU_D : 2 * OTPU_D;
    if (width < chunk || width % chunk || K % width || width > QIN_KBIG)
        return otpu_fail(OTPU_EINVAL, "mm_qin: ranges of %d over K %d (multiples of %d, at most %d)", width, K, chunk,
                         QIN_KBIG);
    if (flags & (OTPU_ACC | OTPU_ASCALE | OTPU_RMAX)) return otpu_fail(OTPU_EINVAL, "mm_qin: no ACC, ASCALE or RMAX");
    if (!x || !out || nsum < 1 || nsum > QIN_NSUM_MAX || (nsum > 1 && sum_stride < K) || ors < N)
        return otpu_fail(OTPU_EINVAL, "mm_qin: x / out NULL, nsum %d, sum_stride %lld, ors %lld", nsum,
                         (long long)sum_stride, (long long)ors);
    if (!al(x, 16) || (xmul && !al(xmul, 16)) || (cscale && !al(cscale, 16)) || sum_stride % 4)
        return otpu_fail(OTPU_EALIGN, "mm_qin: x, xmul and cscale 16-byte aligned, sum_stride a multiple of 4");
    const int R = K / width;
    if (R > 1 && part_stride < N) return otpu_fail(OTPU_EINVAL, "mm_qin: part_stride %lld < N %d", (long long)part_stride, N);
    if (R > 65535) return otpu_fail(OTPU_EINVAL, "mm_qin: %d ranges", R);
    const bool plain = (flags & (OTPU_UNIT | OTPU_RSC)) != 0;
    // the operand checks of one range's MM (the activation operand is the fp32 row itself)
    int rc = check_mm("mm_qin", reinterpret_cast<const int8_t*>(x), width, reinterpret_cast<const uint8_t*>(x),
                      width / 32, 1, width, w, rs, ws, srs, N, fmt, flags, plain ? k0 : k0 + (K - width) / OTPU_D);
    if (rc) return rc;
    if (rs < (fmt == OTPU_INT8 ? K : K / 2)) return otpu_fail(OTPU_EINVAL, "mm_qin: rs %lld short of K %d", (long long)rs, K);
    MMArgs a = make_args(nullptr, width, nullptr, nullptr, width / 32, 1, width, w, rs, ws, srs, N, flags, k0);
    a.out = out; a.ors = ors; a.out_bs = part_stride;
    a.xin = x; a.xmul = xmul; a.nsum = nsum; a.sum_stride = sum_stride; a.xin_bs = width;
    a.rscale = rscale; a.cscale = cscale;
    a.w_bs = fmt == OTPU_INT8 ? width : width / 2; a.k0_bs = plain ? 0 : width / OTPU_D;
    a.P = (fmt == OTPU_INT8 ? width : width / 2) / 16;
    pick_team(a.P, &a.T, Lp, &a.nseg);
    *ap = a;
    return OTPU_OK;
}
}  // namespace otpu

extern "C" int otpu_mm_qin(const float* x, const float* xmul, const float* rscale, const float* cscale, int nsum,
                           int64_t sum_stride, int K, int width, const uint8_t* w, int64_t rs, const uint8_t* ws,
                           int64_t srs, int N, int fmt, int flags, int k0, float* out, int64_t ors, int64_t part_stride,
                           otpu_stream_t stream) {
    MMArgs a;
    int L = 1;
    const int rc = qin_args(&a, &L, x, xmul, rscale, cscale, nsum, sum_stride, K, width, w, rs, ws, srs, N, fmt, flags,
                            k0, out, ors, part_stride);
    if (rc) return rc;
    const int R = K / width;
    hipStream_t s = (hipStream_t)stream;
    switch (fmt) {
        case OTPU_INT8: launch_qin_fmt<OTPU_INT8>(a, L, R, s); break;
        case OTPU_INT4: launch_qin_fmt<OTPU_INT4>(a, L, R, s); break;
        case OTPU_FP4: launch_qin_fmt<OTPU_FP4>(a, L, R, s); break;
        default: launch_qin_fmt<OTPU_NVFP4>(a, L, R, s); break;
    }
    return otpu_launch_check("mm_qin");
}

namespace otpu {
void launch_fold(const MMArgs& a, int fmt, int L, hipStream_t s);   // gemv_fold.hip

// the checks and the argument block of one otpu_mm_qin_fold (pieces a lane in *L; also the
// persistent chain's down projections)
int fold_args(MMArgs* ap, int* Lp, const float* x, const float* xmul, const float* rscale, const float* cscale,
              int K, int width, const uint8_t* w, int64_t rs, const uint8_t* ws, int64_t srs, int N, int fmt, int flags,
              int k0, float* out) {
    if (fmt == OTPU_INT8) return otpu_fail(OTPU_EINVAL, "mm_qin_fold: 4-bit weights (F-chunks of 256)");
    if (flags & ~OTPU_PAIR) return otpu_fail(OTPU_EINVAL, "mm_qin_fold: no flags (weights with scale rows)");
    if (K < 256 || K % 256 || K > FOLD_KMAX)
        return otpu_fail(OTPU_EINVAL, "mm_qin_fold: K %d (a multiple of 256, at most %d)", K, FOLD_KMAX);
    if (width < 256 || width % 256 || K % width)
        return otpu_fail(OTPU_EINVAL, "mm_qin_fold: width %d (a multiple of 256 dividing K %d)", width, K);
    if (!x || !out) return otpu_fail(OTPU_EINVAL, "mm_qin_fold: x / out NULL");
    if (!al(x, 16) || (xmul && !al(xmul, 16)) || (cscale && !al(cscale, 16)))
        return otpu_fail(OTPU_EALIGN, "mm_qin_fold: x, xmul and cscale 16-byte aligned");
    int rc = check_mm("mm_qin_fold", reinterpret_cast<const int8_t*>(x), K, reinterpret_cast<const uint8_t*>(x),
                      K / 32, 1, K, w, rs, ws, srs, N, fmt, flags, k0);
    if (rc) return rc;
    if (rs < K / 2) return otpu_fail(OTPU_EINVAL, "mm_qin_fold: rs %lld short of K %d", (long long)rs, K);
    MMArgs a = make_args(nullptr, K, nullptr, nullptr, K / 32, 1, K, w, rs, ws, srs, N, flags & ~OTPU_PAIR, k0);
    a.out = out; a.ors = N;
    a.xin = x; a.xmul = xmul; a.nsum = 1;
    a.rscale = rscale; a.cscale = cscale;
    a.P = (K / 2) / 16;
    a.fold_c = width / 256;
    int L = 1;
    pick_team(a.P, &a.T, &L);
    if (L > 4) return otpu_fail(OTPU_EINVAL, "mm_qin_fold: K %d needs %d pieces a lane (at most 4)", K, L);
    *ap = a;
    *Lp = L;
    return OTPU_OK;
}
}  // namespace otpu

extern "C" int otpu_mm_qin_fold(const float* x, const float* xmul, const float* rscale, const float* cscale, int K,
                                int width, const uint8_t* w, int64_t rs, const uint8_t* ws, int64_t srs, int N,
                                int fmt, int flags, int k0, float* out, otpu_stream_t stream) {
    MMArgs a;
    int L = 1;
    const int rc = fold_args(&a, &L, x, xmul, rscale, cscale, K, width, w, rs, ws, srs, N, fmt, flags, k0, out);
    if (rc) return rc;
    launch_fold(a, fmt, L, (hipStream_t)stream);
    return otpu_launch_check("mm_qin_fold");
}

extern "C" int otpu_acc_rows(const float* parts, int R, int64_t pstride, int n, const float* old, float* out,
                             otpu_stream_t stream) {
    if (!parts || !out || R < 1 || n < 1 || (R > 1 && pstride < n))
        return otpu_fail(OTPU_EINVAL, "acc_rows: R %d, n %d, pstride %lld", R, n, (long long)pstride);
    hipStream_t s = (hipStream_t)stream;
    if (old && old != out) {
        hipError_t e = hipMemcpyAsync(out, old, sizeof(float) * n, hipMemcpyDeviceToDevice, s);
        if (e != hipSuccess) return otpu_fail(OTPU_ELAUNCH, "acc_rows: %s", hipGetErrorString(e));
    }
    sum_parts<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(parts, pstride, R, 1, n, old != nullptr, out, n);
    return otpu_launch_check("acc_rows");
}

extern "C" int otpu_lm_head_argmax(const int8_t* q, const float* Sa, const uint8_t* da, int K, const uint8_t* w,
                                   int64_t rs, const uint8_t* ws, int64_t srs, int N, int fmt, int flags, int k0,
                                   int64_t base, float* logits, uint64_t* best, int32_t* token,
                                   otpu_stream_t stream) {
    if (flags & (OTPU_ACC | OTPU_ASCALE | OTPU_RMAX))
        return otpu_fail(OTPU_EINVAL, "lm_head_argmax: no ACC, ASCALE or RMAX");
    int rc = check_mm("lm_head_argmax", q, K, da, K / 32, 1, K, w, rs, ws, srs, N, fmt, flags, k0);
    if (rc) return rc;
    if (!Sa || !best || !token) return otpu_fail(OTPU_EINVAL, "lm_head_argmax: NULL Sa, best or token");
    if (base < 0 || base + (int64_t)N > 0xFFFFFFFFll) return otpu_fail(OTPU_EINVAL, "lm_head_argmax: base %lld", (long long)base);
    if (!al(best, 16)) return otpu_fail(OTPU_EALIGN, "lm_head_argmax: best (the state) 16-byte aligned");
    hipStream_t s = (hipStream_t)stream;
    MMArgs a = make_args(q, K, Sa, da, K / 32, 1, K, w, rs, ws, srs, N, flags, k0);
    a.out = logits; a.ors = N; a.best = best + LM_STRIDE; a.base = base;
    rc = launch_gemv(a, fmt, 1, s);
    if (rc) return rc;
    best_finish<<<1, 64, 0, s>>>(best, token);
    return otpu_launch_check("lm_head_argmax");
}

extern "C" int otpu_argmax(const float* x, int rows, int cols, int64_t ldx, int64_t base, float* pairs,
                           int64_t drs, otpu_stream_t stream) {
    if (rows < 1 || cols < 1 || ldx < cols || !x || !pairs || (rows > 1 && drs < 2))
        return otpu_fail(OTPU_EINVAL, "argmax: rows %d, cols %d, ldx %lld, drs %lld", rows, cols,
                         (long long)ldx, (long long)drs);
    argmax_rows<<<rows, 256, 0, (hipStream_t)stream>>>(x, cols, ldx, base, pairs, drs);
    return otpu_launch_check("argmax");
}
