/* Oracle (C, OpenMP): MM / QACT / ARGMAX of openTPU on the CPU.  TEST INFRASTRUCTURE ONLY:
 * the fast checker at full sizes for tests/ and the CPU baseline timed by bench.py.
 *
 * The same functions as oracle/fp32.py and oracle/mm.py (which pin them), restated from:
 *   fp32 arithmetic, recip, q8, quantize_mx   opentpu/fp32.py:45-101, :162-172, :242-261, :295-343
 *   MM (natural layout, rows of one)          opentpu/isasim.py:706-910, docs/isa.md:226-305
 *   ARGMAX / greedy                           opentpu/isasim.py:1141-1152, opentpu/fp32.py:110-121
 * Built with -ffp-contract=off and SSE arithmetic (no excess precision): every float operation
 * is one IEEE binary32 RNE operation, flushed by hand like the machine's.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define D 128

static inline uint32_t fbits(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static inline float bitsf(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }
static inline float ftz(float x) {
    uint32_t u = fbits(x);
    if ((u & 0x7F800000u) == 0) u &= 0x80000000u;
    return bitsf(u);
}
static inline float fin(float r) {
    r = ftz(r);
    return (r != r) ? bitsf(0x7FC00000u) : r;
}
static inline float fmul(float a, float b) { return fin(ftz(a) * ftz(b)); }
static inline float fadd(float a, float b) { return fin(ftz(a) + ftz(b)); }
static inline float fsub(float a, float b) { return fin(ftz(a) - ftz(b)); }
static inline uint32_t fkey(float x) {
    uint32_t u = fbits(ftz(x));
    return (u >> 31) ? ~u : (u | 0x80000000u);
}

static float recip(float x) {
    x = ftz(x);
    uint32_t xb = fbits(x), mag = xb & 0x7FFFFFFFu, sign = xb & 0x80000000u;
    if (mag == 0) return 0.0f;
    if (mag >= 0x7E800000u) return bitsf(sign);
    float a = bitsf(0x3F800000u | (mag & 0x7FFFFFu));
    float y = bitsf(0x7EF311C3u - fbits(a));
    y = fmul(y, fsub(2.0f, fmul(a, y)));
    y = fmul(y, fsub(2.0f, fmul(a, y)));
    y = fadd(fmul(y, fsub(1.0f, fmul(a, y))), y);
    int32_t k = 127 - (int32_t)(mag >> 23);
    return bitsf((uint32_t)((int32_t)fbits(y) + k * (1 << 23)) | sign);
}

static inline int8_t q8(float x) {
    x = ftz(x);
    if (x != x) return 0;
    float r = rintf(x);                 /* the default rounding mode: half to even */
    if (r > 127.0f) r = 127.0f;
    if (r < -127.0f) r = -127.0f;
    return (int8_t)r;
}

static inline float pow2f(int d) { return bitsf((uint32_t)(d + 127) << 23); }

int otpu_cpu_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
    return omp_get_max_threads();
#else
    (void)n;
    return 1;
#endif
}

/* recip of n values: the C restatement's own recip, exported so that the tests can check it
 * against the reference's golden vectors directly (QACT's bytes rarely show a one-ulp slip). */
void otpu_cpu_recip(const float* x, long n, float* y) {
    #pragma omp parallel for schedule(static)
    for (long i = 0; i < n; ++i) y[i] = recip(x[i]);
}

/* quantize_mx of M rows of K: q int8 [M, ldq], S [M], d [M, ldd] (K/g offsets a row). */
int otpu_cpu_qact(const float* x, int M, int K, long ldx, int g, int row_mode,
                  int8_t* q, long ldq, float* S, uint8_t* d, long ldd) {
    if (M < 1 || K < 1 || g < 1 || K % g) return -1;
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < M; ++r) {
        const float* xr = x + (long)r * ldx;
        uint32_t amax = 0;
        for (int i = 0; i < K; ++i) {
            uint32_t a = fbits(ftz(xr[i])) & 0x7FFFFFFFu;
            if (a > amax) amax = a;
        }
        float fa = bitsf(amax);
        float s = amax ? fmul(fa, bitsf(0x3C010204u)) : 0.0f;
        float inv = amax ? fmul(127.0f, recip(fa)) : 0.0f;
        S[r] = s;
        for (int g0 = 0; g0 < K; g0 += g) {
            int dg = 0;
            if (!row_mode) {
                uint32_t ga = 0;
                for (int i = g0; i < g0 + g; ++i) {
                    uint32_t a = fbits(ftz(xr[i])) & 0x7FFFFFFFu;
                    if (a > ga) ga = a;
                }
                if (ga) {
                    dg = (int)(amax >> 23) - (int)(ga >> 23) - ((ga & 0x7FFFFFu) > (amax & 0x7FFFFFu));
                    dg = dg < 0 ? 0 : (dg > 31 ? 31 : dg);
                }
            }
            d[(long)r * ldd + g0 / g] = (uint8_t)dg;
            float sc = fmul(inv, pow2f(dg));
            for (int i = g0; i < g0 + g; ++i) q[(long)r * ldq + i] = q8(fmul(xr[i], sc));
        }
    }
    return 0;
}

static const int8_t DEC4[3][16] = {
    {0, 1, 2, 3, 4, 5, 6, 7, -8, -7, -6, -5, -4, -3, -2, -1},
    {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12},
    {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12},
};

enum { F_UNIT = 1, F_ACC = 2, F_RMAX = 4, F_ASCALE = 8, F_RSC = 0x80 };

/* MM: out[j, n] (ors floats apart) for M activation rows x N weight rows; acc_out (optional)
 * the exact accumulators int64 [M, N]; rowmax (optional, RMAX) [M]. */
int otpu_cpu_mm(const int8_t* q, long ldq, const float* Sa, const uint8_t* da, long ldda,
                int M, int K, const uint8_t* w, long rs, const uint8_t* ws, long srs, int N,
                int fmt, int flags, int k0, const float* alpha, float* out, long ors,
                float* rowmax, int64_t* acc_out) {
    if (M < 1 || N < 1 || K < D || K % D || fmt < 0 || fmt > 3) return -1;
    if ((flags & F_ASCALE) && !((flags & F_UNIT) && (flags & F_ACC))) return -2;
    if ((flags & F_RSC) && fmt == 3) return -3;
    const int KB = K / D, G = fmt == 3 ? 8 : 4, gs = D / G;
    const int W = fmt == 0 ? 16 : fmt == 3 ? 13 : 11;
    const int unit = flags & F_UNIT, rsc = flags & F_RSC;
    #pragma omp parallel
    {
        int8_t* wv = (int8_t*)malloc((size_t)K);
        int* dw = (int*)malloc(sizeof(int) * KB * G);
        int* mw = (int*)malloc(sizeof(int) * KB * G);
        #pragma omp for schedule(static)
        for (int n = 0; n < N; ++n) {
            const uint8_t* row = w + (long)n * rs;
            const uint8_t* srow = ws + (long)n * srs;
            if (fmt == 0) memcpy(wv, row, (size_t)K);
            else
                for (int i = 0; i < K; ++i)
                    wv[i] = DEC4[fmt - 1][(row[i >> 1] >> ((i & 1) * 4)) & 15];
            float Sw = 1.0f;
            if (!unit) memcpy(&Sw, srow, 4);
            for (int k = 0; k < KB; ++k)
                for (int g = 0; g < G; ++g) {
                    int dv = 0, mv = 1;
                    if (!unit && !rsc) {
                        int kk = k0 + k;
                        if (fmt == 0) dv = srow[4 + kk];
                        else if (fmt < 3) {
                            uint32_t word;
                            memcpy(&word, srow + 8 + 4 * kk, 4);
                            dv = (int)(word & 0xFF);
                            mv = (int)((word >> (8 + 6 * g)) & 63);
                        } else {
                            int e4 = srow[16 + 8 * kk + g], E = (e4 >> 3) & 15, Mt = e4 & 7;
                            dv = 15 - (E > 1 ? E : 1);
                            mv = E ? 8 + Mt : Mt;
                        }
                    }
                    dw[k * G + g] = dv;
                    mw[k * G + g] = mv;
                }
            for (int j = 0; j < M; ++j) {
                const int8_t* qj = q + (long)j * ldq;
                const uint8_t* daj = da + (long)j * ldda;
                int64_t acc = 0;
                for (int t = 0; t < KB * G; ++t) {
                    int32_t c = 0;
                    const int8_t* a = qj + t * gs;
                    const int8_t* b = wv + t * gs;
                    for (int i = 0; i < gs; ++i) c += (int32_t)a[i] * (int32_t)b[i];
                    int sh = W - dw[t] - (int)daj[(t * gs) / 32];
                    if (sh >= 0) acc += ((int64_t)mw[t] << sh) * (int64_t)c;
                }
                if (acc_out) acc_out[(long)j * N + n] = acc;
                float y = fmul(fmul((float)acc, Sw), fmul(Sa[j], pow2f(-W)));
                float* o = out + (long)j * ors + n;
                if (flags & F_ASCALE) y = fadd(fmul(*o, alpha[j]), y);
                else if (flags & F_ACC) y = fadd(*o, y);
                *o = y;
            }
        }
        free(wv); free(dw); free(mw);
    }
    if ((flags & F_RMAX) && rowmax)
        for (int j = 0; j < M; ++j) {
            const float* o = out + (long)j * ors;
            uint32_t best = fkey(o[0]);
            float bv = ftz(o[0]);
            for (int n = 1; n < N; ++n)
                if (fkey(o[n]) > best) { best = fkey(o[n]); bv = ftz(o[n]); }
            rowmax[j] = bv;
        }
    return 0;
}

/* Greedy over n logits: best = max over i of (key << 32 | ~i), token = the first maximal i. */
int otpu_cpu_argmax(const float* x, long n, uint64_t* best, int32_t* token) {
    if (n < 1) return -1;
    uint64_t b = 0;
    #pragma omp parallel for reduction(max : b) schedule(static)
    for (long i = 0; i < n; ++i) {
        uint64_t v = ((uint64_t)fkey(x[i]) << 32) | (uint32_t)~(uint32_t)i;
        if (v > b) b = v;
    }
    *best = b;
    *token = (int32_t)~(uint32_t)(b & 0xFFFFFFFFu);
    return 0;
}
