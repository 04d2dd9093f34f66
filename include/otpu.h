/* opentpu_amd: the C ABI of the MI355X quantized-linear hot path (openTPU's MM, QACT and
 * greedy ARGMAX as HIP kernels for gfx950).
 *
 * Conventions
 *   - Every pointer is device memory owned by the caller (hipMalloc or a torch tensor's
 *     data_ptr()); sizes and strides are in elements of the pointed-to type unless the name
 *     says bytes (`rs`, `srs` are bytes, like the reference's).
 *   - Every call is asynchronous on `stream` (a hipStream_t; NULL = the null stream) and
 *     allocates nothing.
 *   - Return value: OTPU_OK (0) or a negative OTPU_E* code; the message of the last failure
 *     on the calling thread is otpu_last_error().  The argument checks mirror the reference
 *     simulator's SimError checks (opentpu/isasim.py:767-822).
 *   - Layouts are the reference's byte for byte, so packed weights from
 *     opentpu/quant.py:quantize_mxu load unchanged (opentpu/quant.py:287-449, docs/isa.md:277-304).
 */
#ifndef OTPU_H
#define OTPU_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* otpu_stream_t; /* hipStream_t */

enum {
    OTPU_OK = 0,
    OTPU_EINVAL = -1,   /* a shape, stride or field out of range */
    OTPU_EALIGN = -2,   /* a pointer or stride not aligned as the kernels need */
    OTPU_EFORMAT = -3,  /* an unknown weight format or a format / flag combination refused */
    OTPU_ELAUNCH = -4,  /* a HIP launch error */
    OTPU_ENODEV = -5    /* no usable gfx950 device */
};

/* Weight formats (opentpu/isa.py:26-28: W8, W4I, W4F, WNV; shift windows 16, 11, 11, 13). */
enum { OTPU_INT8 = 0, OTPU_INT4 = 1, OTPU_FP4 = 2, OTPU_NVFP4 = 3 };

/* MM flags, the reference's bits (opentpu/isa.py:21, :29-30). PAIR changes no result bit
 * (a scheduling mode of the MXU) and is accepted and ignored. */
enum {
    OTPU_UNIT = 0x1,
    OTPU_ACC = 0x2,
    OTPU_RMAX = 0x4,
    OTPU_ASCALE = 0x8,
    OTPU_PAIR = 0x40,
    OTPU_RSC = 0x80
};

/* QACT / QST flags (the reference's QACT bits: opentpu/isa.py, docs/isa.md:444-460).  CSCALE,
 * RSCALE and ST are given by their operands (non-NULL cscale, rscale, qrows); DUP (the operand
 * layout of MM PAIR) changes no result and has no counterpart. */
enum {
    OTPU_Q_ROW = 0x1,   /* one scale a row: every group offset 0 */
    OTPU_Q_LO = 0x10,   /* the split's lo part: q8lo bytes and the scale S * 2^-8 (SPLITQ) */
    OTPU_Q_HL = 0x20    /* both parts from one read: hi bytes at q[r, 0..K), lo at q[r, K..2K) */
};
#define OTPU_QALIGN 64  /* QACT ST / LDA rows: addresses and stride multiples of it (isa.py:40) */

/* The ABI's version: otpu_version() returns OTPU_ABI_VERSION of the header the library was built
 * with.  It changes whenever an entry point's signature or an operand's size changes, so a caller
 * built against another header can refuse the library (opentpu_amd/_lib.py does). */
#define OTPU_ABI_VERSION 3

const char* otpu_last_error(void);
int otpu_version(void);

/* QACT: fp32.quantize_mx(x', g, row_mode, lo) of M rows of K (opentpu/fp32.py:321-343; the
 * instruction: opentpu/isasim.py:913-959, opentpu/isa.py:551, docs/isa.md:444-486), x' the rows
 * after QACT's pre-multiplies: x' = (x * rscale[r]) * cscale[c] (RSCALE, CSCALE; either may be
 * NULL: RMSNorm's x * r * gamma folded into the quantizer).
 *   x [M, ldx] fp32 -> q [M, ldq] int8, S [M] fp32 (amax * f32(1/127)), d [M, ldd] uint8
 *   (K/g power-of-two group offsets; all 0 with OTPU_Q_ROW).  g in {8, 16, 32, 64, 128}
 *   (QACT: 32 = D/4; QST and the int8x weight packer: 128 = D), K a multiple of g and of 4.
 *   OTPU_Q_LO: q holds q8lo's bytes and S the scale S * 2^-8 (fp32.q8lo, opentpu/fp32.py:175-185).
 *   OTPU_Q_HL: ldq >= 2K; q[r, 0..K) the hi bytes, q[r, K..2K) the lo bytes; S [2M]: S[r] hi's,
 *   S[M + r] lo's; the same offsets d.
 *   qrows (may be NULL; not with HL): QACT ST's rows, row r at qrows + r * qrs bytes: its K bytes
 *   as q holds them, then block k's 8-byte record at K + 8k (S little-endian, the block's 4
 *   offsets); g 32, K a multiple of 128 (at most 256 blocks), qrows and qrs (with M > 1)
 *   multiples of OTPU_QALIGN, qrs >= K + 8 K/128 (opentpu/isasim.py:962-988, isa.py:577-580). */
int otpu_qact(const float* x, int M, int K, int64_t ldx, int g, int flags, const float* rscale,
              const float* cscale, int8_t* q, int64_t ldq, float* S, uint8_t* d, int64_t ldd,
              uint8_t* qrows, int64_t qrs, otpu_stream_t stream);

/* LDA (opentpu/isasim.py:990-1006): QACT ST's rows of KB blocks back into an MM operand:
 * q [rows, ldq] the bytes, d [rows, ldd] the offsets (4 a block), S [KB, rows] (block k's record
 * scale of row r at S[k * rows + r]: the MM over blocks from k on takes Sa = S + k * rows). */
int otpu_lda(const uint8_t* qrows, int64_t qrs, int rows, int KB, int8_t* q, int64_t ldq, float* S,
             uint8_t* d, int64_t ldd, otpu_stream_t stream);

/* QACT over K / width equal column ranges of each row in one launch: one QACT instruction per
 * range (opentpu/isasim.py:927-959), as the reference quantizes a down projection's input in
 * F-chunks (opentpu/kernels/mlp.py:8-30, :87-120).  Range r of row j: q[j, r*width ..], its
 * scale S[r * M + j], its offsets d[j, r*width/g ..].  xmul (may be NULL): quantize the VOP MUL
 * x * xmul instead of x (same shape and stride; the SwiGLU product g * u of mlp.py:101-104);
 * then RSCALE / CSCALE as otpu_qact (cscale indexed by the row's column, over all ranges).
 * flags: OTPU_Q_ROW, OTPU_Q_LO. */
int otpu_qact_ranges(const float* x, const float* xmul, int M, int K, int64_t ldx, int width, int g,
                     int flags, const float* rscale, const float* cscale, int8_t* q, int64_t ldq,
                     float* S, uint8_t* d, int64_t ldd, otpu_stream_t stream);

/* VOP MUL (opentpu/isasim.py:1181, V_MUL; fp32.mul, opentpu/fp32.py:100): out = a * b, one IEEE RNE
 * product with flush-to-zero on operands and result, over n elements. */
int otpu_vmul(const float* a, const float* b, float* out, int64_t n, otpu_stream_t stream);

/* MM (opentpu/isasim.py:749-910, opentpu/isa.py:502; semantics docs/isa.md:226-305), natural
 * row layout, rows of one:
 *   q [M, ldq] int8, Sa [M], da [M, ldda] uint8 (an offset per 32 of K): the operand one QACT
 *   range wrote; w: N weight rows `rs` bytes apart (int8: K bytes; 4-bit: K/2 bytes, element
 *   2i in the low nibble); ws: N scale rows `srs` bytes apart (ignored with UNIT); the MM's
 *   block k uses the scale rows' block k0 + k.  out [M, ors] fp32:
 *     out[j, n] = (i2f(acc) * Sw[n]) * (Sa[j] * 2^-W)   (then ACC / ASCALE as the flags say)
 *   with acc the exact integer sum over 32-groups of (m << (W - dw - da)) * c (dropped where
 *   the shift is negative).  alpha [M] (ASCALE only), rowmax [M] (RMAX only; may be NULL
 *   otherwise).  K a multiple of 128; w, rs multiples of 16 bytes; ws, srs multiples of 4. */
int otpu_mm(const int8_t* q, int64_t ldq, const float* Sa, const uint8_t* da, int64_t ldda,
            int M, int K, const uint8_t* w, int64_t rs, const uint8_t* ws, int64_t srs, int N,
            int fmt, int flags, int k0, const float* alpha, float* out, int64_t ors,
            float* rowmax, otpu_stream_t stream);

/* The same MM's exact accumulators acc [M, N] (int64), no epilogue (parity and debugging:
 * the int64 row sums of opentpu/isasim.py:879-898). */
int otpu_mm_acc(const int8_t* q, int64_t ldq, const uint8_t* da, int64_t ldda, int M, int K,
                const uint8_t* w, int64_t rs, const uint8_t* ws, int64_t srs, int N, int fmt,
                int flags, int k0, int64_t* acc, otpu_stream_t stream);

/* Builder.dot's per-range MMs (opentpu/compiler.py:2686-2720; swiglu_down's chunks,
 * opentpu/kernels/mlp.py:87-120): K / width MMs, range r over columns r*width .. of q / da
 * (offsets) and of the weight rows (scale blocks k0 + r*width/128), its activation scale
 * Sa[r * M + j] (otpu_qact_ranges' layout), accumulated in range order as the ACC chain
 * out = add(..add(add(old | y_0, y_1)..), y_R-1) (old with ACC; else y_0 starts it).
 * part: a caller's workspace of R * M * N fp32 (the per-range MM outputs).  width a multiple
 * of 128 (int8) or 256 (4-bit: ranges start on whole 128-byte chunks).  No ASCALE / RMAX. */
int otpu_mm_ranges(const int8_t* q, int64_t ldq, const float* Sa, const uint8_t* da, int64_t ldda,
                   int M, int K, int width, const uint8_t* w, int64_t rs, const uint8_t* ws,
                   int64_t srs, int N, int fmt, int flags, int k0, float* part, float* out,
                   int64_t ors, otpu_stream_t stream);

/* QACT + MM of one activation row in one launch (the chained decode's linear): quantize the fp32
 * row as QACT does (fp32.quantize_mx(x, 32), opentpu/fp32.py:321-343) and run the MM on it
 * (opentpu/isasim.py:749-910), in K / width ranges each with its own QACT, as
 * otpu_qact_ranges + otpu_mm_ranges do without their ACC fold: range r writes its MM output
 * row to out + r * part_stride (one range: out).  The row quantized is x[0..K) folded with
 * nsum - 1 more rows sum_stride apart in order (x_0 + x_1 + ..: the ACC chain of a previous
 * per-range MM, opentpu/isasim.py:899-905), times xmul when given (VOP MUL), then QACT's
 * RSCALE and CSCALE products (x * rscale[0]) * cscale[c] when given (rscale: one float, the
 * row's factor; cscale [K]; docs/isa.md:447-452).  No ACC / ASCALE / RMAX; width at most 4096,
 * a multiple of 128 (int8) or 256 (4-bit); nsum at most 16. */
int otpu_mm_qin(const float* x, const float* xmul, const float* rscale, const float* cscale, int nsum,
                int64_t sum_stride, int K, int width, const uint8_t* w, int64_t rs, const uint8_t* ws,
                int64_t srs, int N, int fmt, int flags, int k0, float* out, int64_t ors, int64_t part_stride,
                otpu_stream_t stream);

/* The chained layer's down projection folded in one launch (Builder.dot's per-range MMs with
 * their ACC, opentpu/compiler.py:2686-2720; swiglu_down's chunk loop,
 * opentpu/kernels/mlp.py:87-120): the fp32 row mul(x, xmul) (xmul may be NULL; then RSCALE and
 * CSCALE as otpu_mm_qin, either may be NULL) in K / width ranges of width columns (the 4-bit down
 * chunk, opentpu/kernels/mlp.py:8-30: 256 at F = 3072, 768 at F = 6144), each quantized by its
 * own QACT and multiplied by its weight columns, and the ranges' outputs added in range order into
 * out[0..N): otpu_mm_qin's ranges and the fold of their rows, bit for bit.  4-bit weights with
 * scale rows only (INT4, FP4, NVFP4; no flags but PAIR); K a multiple of 256, at most 8192; width
 * a multiple of 256 that divides K. */
int otpu_mm_qin_fold(const float* x, const float* xmul, const float* rscale, const float* cscale, int K,
                     int width, const uint8_t* w, int64_t rs, const uint8_t* ws, int64_t srs, int N, int fmt,
                     int flags, int k0, float* out, otpu_stream_t stream);

/* MM SPL (split terms: opentpu/isasim.py:757-770, :849-852, :872-873; docs/isa.md:414-441): one
 * MM over a split operand's terms, one K-block (128) of int8 RSC weights a part, natural rows.
 *   q [M, ldq]: the activations' hi part at q[j, 0..128), with nterms 3 also the lo part at
 *   q[j, 128..256) (otpu_qact OTPU_Q_HL's layout); Sa [M] and da [M, ldda] (4 offsets) the hi
 *   part's; w: N hi weight rows rs bytes apart, their lo rows hld bytes after them (otpu_pack_int8
 *   with OTPU_Q_ROW, then OTPU_Q_ROW | OTPU_Q_LO); ws: the hi rows' scale words Sw, srs apart.
 *   nterms 3: hi.w_hi + lo.w_hi + hi.w_lo; nterms 2: hi.w_hi + hi.w_lo; each lo term's offsets
 *   + 8 (dropped where 16 - da - 8 < 0); one exact integer an output and one fp32 epilogue
 *   (i2f(acc) * Sw) * (Sa * 2^-16): the split product rounded once (not the sum of the separate
 *   MMs).  flags: OTPU_RSC (required) and OTPU_ACC. */
int otpu_mm_spl(const int8_t* q, int64_t ldq, const float* Sa, const uint8_t* da, int64_t ldda, int M,
                int nterms, const uint8_t* w, int64_t rs, int64_t hld, const uint8_t* ws, int64_t srs,
                int N, int flags, float* out, int64_t ors, otpu_stream_t stream);

/* The ACC fold of R rows of n (opentpu/isasim.py:899-905 applied in order): out = add(..add(
 * add(old | p_0, p_1)..), p_R-1) with FTZ adds, rows pstride apart; old may be NULL. */
int otpu_acc_rows(const float* parts, int R, int64_t pstride, int n, const float* old, float* out,
                  otpu_stream_t stream);

/* The fused, folded decode chain in one persistent launch (per layer: MM qkv, MM o on q, MM
 * gate/up, the folded down projection on mul(g, u), each with its input row's QACT in the
 * prologue: opentpu/kernels/mlp.py's layer and Builder.dot's per-range MMs + ACC,
 * opentpu/compiler.py:2686-2720), bit for bit the outputs of otpu_mm_qin x 3 + otpu_mm_qin_fold a
 * layer.  The reference runs this as an ISA program; this is the same computation as one launch
 * of one workgroup a CU, the phases handing rows to each other through the plan's memory.
 *   otpu_chain_plan_bytes: the plan's size (-1 for bad dimensions).
 *   otpu_chain_plan: checks every phase as its one-launch entry point would and writes the plan
 *   (synchronous; plan device memory, 256-byte aligned).  w / rs / ws / srs / outs: 4 a layer in
 *   the order qkv, o, gu, down (each layer's strides equal layer 0's); rnorm: RSCALE factors
 *   [layers, 2] (device) or NULL; cscale: 2 a layer (gamma of the qkv and the gate/up QACTs,
 *   device, entries may be NULL) or NULL; x: the step's input row [hidden]; outs: the phases' fp32
 *   output rows (qkv [q_dim + 2 kv_dim], o [hidden], gu [2 F], down [hidden]); down_width: the
 *   down projection's QACT range (a multiple of 256 dividing F; the reference's chunk rule gives
 *   256 at F = 3072, 768 at F = 6144).  int4x, fp4x6 or nvfp4 weights; hidden <= 2048, q_dim <= 2048, F
 *   a multiple of 256 and <= 8192 (hidden <= 1024 and F <= 4096, Qwen3-0.6B's sizes, run teams of
 *   one and two pieces a lane, larger shapes up to Qwen3-1.7B's two and four), hidden and q_dim
 *   multiples of 32.
 *   otpu_chain_step: one step (reads x, writes every output row); capturable in a HIP graph.
 *   Steps on one plan must not overlap (issue them on one stream).  It launches the kernel
 *   otpu_chain_plan picked for the plan (a plan built at that address in this process; else
 *   OTPU_EINVAL).  A step needs all of its workgroups (one a CU) resident at once: the plan
 *   refuses (OTPU_ELAUNCH) a device whose occupancy for its kernel cannot hold them; kernels
 *   beside it on other streams can still hold CUs back, and its waits then run out of polls
 *   (they are bounded: no hang).
 *   otpu_chain_error: the plan's error word (0: every hand-off completed; 1: a wait ran out of
 *   polls, the outputs since are invalid), synchronous.  It stays set until the plan is
 *   written again. */
int64_t otpu_chain_plan_bytes(int layers, int hidden, int q_dim, int kv_dim, int F);
int otpu_chain_plan(int layers, int hidden, int q_dim, int kv_dim, int F, int down_width, int fmt,
                    const uint8_t* const* w, const int64_t* rs, const uint8_t* const* ws, const int64_t* srs,
                    const float* rnorm, const float* const* cscale, const float* x, float* const* outs,
                    void* plan, int64_t plan_bytes);
int otpu_chain_step(const void* plan, otpu_stream_t stream);
int otpu_chain_error(const void* plan, uint32_t* err);
/* Profiling: clock stamps of every phase and workgroup into stamps [4 layers][grid][16]
 * (uint64, the 100 MHz clock: phase start, weights issued, input row in, QACT done, rows stored,
 * and the counts of polls of the hand-off waits; NULL stops).  Only a library built with the stamps (python -m opentpu_amd.build --stamps); others
 * refuse (OTPU_EINVAL).  Synchronous. */
int otpu_chain_stamps(void* plan, uint64_t* stamps);

/* B independent MMs of one shape in one launch (a layer stack's or an expert set's decode
 * GEMVs): problem b's operands start at the given pointers plus b times the *_bstride
 * (elements of each pointer's type; bytes for w and ws).  No ACC / ASCALE / RMAX. */
int otpu_mm_batched(int B, const int8_t* q, int64_t ldq, int64_t q_bstride, const float* Sa,
                    int64_t sa_bstride, const uint8_t* da, int64_t ldda, int64_t da_bstride,
                    int M, int K, const uint8_t* w, int64_t rs, int64_t w_bstride,
                    const uint8_t* ws, int64_t srs, int64_t ws_bstride, int N, int fmt,
                    int flags, int k0, float* out, int64_t ors, int64_t out_bstride,
                    otpu_stream_t stream);

/* LM head + greedy: one activation row (M = 1) times N vocabulary rows, the logits' total-order
 * maximum with the first index (opentpu/llm/qwen3.py:2052-2088 + opentpu/llm/generate.py:251-286
 * + VOP ARGMAX opentpu/isasim.py:1141-1152).  best is the call's state, OTPU_LM_STATE_BYTES
 * 16-byte aligned: best[0] = max over n of (key(y_n) << 32 | ~(base+n)) (a u64 whose low word
 * is the complement of the index); token = base + that n.  The rest holds the running maxima
 * the GEMV's workgroups raise: zero before the first call (e.g. allocated zeroed), and every
 * call leaves it zero again.  Calls on one state must not overlap.  logits may be NULL.  Two
 * kernels. */
#define OTPU_LM_STATE_BYTES 16640  /* 64 maxima 256 bytes apart, after the result's 256 */
int otpu_lm_head_argmax(const int8_t* q, const float* Sa, const uint8_t* da, int K,
                        const uint8_t* w, int64_t rs, const uint8_t* ws, int64_t srs, int N,
                        int fmt, int flags, int k0, int64_t base, float* logits,
                        uint64_t* best, int32_t* token, otpu_stream_t stream);

/* VOP ARGMAX (opentpu/isasim.py:1141-1152, opentpu/isa.py:633): per row of x [rows, ldx] the
 * (maximum, i2f(first column + base)) fp32 pair into pairs[r * drs + 0..1]. */
int otpu_argmax(const float* x, int rows, int cols, int64_t ldx, int64_t base, float* pairs,
                int64_t drs, otpu_stream_t stream);

/* Weight packers, bit-exact with opentpu/quant.py:quantize_mxu (no counterpart kernel in the
 * reference: it packs on the host in numpy).
 *   otpu_pack_int8: int8x (quant.py:316-322, flags 0; scale rows of 4 + 4*ceil(KB/4) bytes) or
 *   RSC rows (runtime.py:66-76 with row=True, flags OTPU_Q_ROW; scale rows of 4 bytes); with
 *   OTPU_Q_LO the split's lo rows (QST LO: q8lo bytes, Sw * 2^-8; the weights' lo part of MM SPL).
 *   otpu_pack_x4: int4x / fp4x6 (quant.py:325-367; fmt OTPU_INT4 or OTPU_FP4) or nvfp4 with a
 *   per-row scale (quant.py:368-400; fmt OTPU_NVFP4): element rows of ceil(K/256)*128 bytes,
 *   scale rows of 8 + 8*ceil(KB/2) bytes (nvfp4: 16 + 16*ceil(KB/2)). */
int otpu_pack_int8(const float* W, int N, int K, int64_t ldw, int flags, uint8_t* rows,
                   int64_t rs, uint8_t* srows, int64_t srs, otpu_stream_t stream);
int otpu_pack_x4(const float* W, int N, int K, int64_t ldw, int fmt, uint8_t* rows, int64_t rs,
                 uint8_t* srows, int64_t srs, otpu_stream_t stream);

/* A weight image in the reference machine's grouped layout (docs/isa.md "Weight groups";
 * opentpu/quant.py:634-808: group_rows / hash_rows / group_scales for a machine of wg lanes)
 * back to the natural rows every MM entry point streams: the inverses of group_rows (with the
 * channel hash of hash_rows when at >= 0: the image's byte address on that machine, a multiple
 * of wg * 128) and of group_scales.  data: ceil(N / R) groups of grp_row_bytes (R = wg int8,
 * 2 wg 4-bit; wg = 1 the natural rows); rows: N rows of rs >= row_bytes(K); areas: the groups'
 * scale areas; srows: N scale rows of srs >= scale_bytes(K).  kt: the image is in MM KT's
 * pairs (docs/isa.md "K tail", opentpu/quant.py:829-880: groups 2p and 2p + 1 share their last
 * block's chunk, (2 KB - 1) chunks a pair; the odd groups' scale entries in chunk order, the tail
 * block's first): K = KB D the padded K, the natural rows come out with block KB-1's upper half
 * zero; int8, int4 and fp4 at wg > 1.  The tail block's 4-bit scale word comes out as the KT
 * image stores it: its sub-blocks 2 and 3 carry copies of sub-blocks 0 and 1's multipliers
 * (opentpu/quant.py:861-880), not quantize_mxu's, so a KT image does not ungroup to
 * quantize_mxu's scale rows byte for byte; every MM result is the same, because the elements
 * those multipliers scale are the zero upper half. */
int otpu_ungroup_rows(const uint8_t* data, int N, int K, int wg, int fmt, int kt, int64_t at,
                      uint8_t* rows, int64_t rs, otpu_stream_t stream);
int otpu_ungroup_scales(const uint8_t* areas, int N, int K, int wg, int fmt, int rsc, int kt,
                        uint8_t* srows, int64_t srs, otpu_stream_t stream);

/* Checkpoint imports, exact (opentpu/quant.py:1070-1182, import_mxfp4 / import_nvfp4; the
 * reference converts on the host in numpy).  codes: one E2M1 code (0..15, sign bit 3) a byte,
 * [N, K] at ldc; rows / srows as otpu_pack_x4 writes them for fp4 / nvfp4.  status[n]: the
 * reasons row n does not come in exactly in the asked format (0: it does):
 *   otpu_import_mxfp4: e8m0 [N, K/32] at lde; fmt OTPU_FP4 or OTPU_NVFP4; status bits 1 an E8M0
 *   NaN, 2 a K-block spanning more than 5 octaves (no fp4), 4 an fp4 dw above 255, 8 fp4's Sw
 *   outside fp32's normal range, 16 a row spanning more than 17 octaves (no nvfp4; set by the
 *   nvfp4 call), 32 nvfp4's Sw outside the normal range (nvfp4 call).
 *   otpu_import_nvfp4: scales [N, K/16] E4M3 bytes at lds, ts the tensor scale; status bits 1 a
 *   negative scale, 2 an E4M3 NaN, 4 a scale too far below the row's largest, 8 Sw outside
 *   fp32's normal range. */
int otpu_import_mxfp4(const uint8_t* codes, int64_t ldc, const uint8_t* e8m0, int64_t lde, int N, int K,
                      int fmt, uint8_t* rows, int64_t rs, uint8_t* srows, int64_t srs, int32_t* status,
                      otpu_stream_t stream);
int otpu_import_nvfp4(const uint8_t* codes, int64_t ldc, const uint8_t* scales, int64_t lds, float ts,
                      int N, int K, uint8_t* rows, int64_t rs, uint8_t* srows, int64_t srs,
                      int32_t* status, otpu_stream_t stream);

/* The sampled decode's pick after the LM head (opentpu/llm/generate.py:323-337 Sampler and
 * :492-557 reference_pick at one slice; the reference's device sampler, in its fp32 arithmetic):
 * logits [V] (the LM head's, e.g. otpu_lm_head_argmax's logits output); pa / pb [V] the
 * repetition penalty's factors (1/R and R at the context's ids, 1 elsewhere; both NULL: none);
 * softcap c (0: none); top_k k in 1..64; itemp = f32(log2(e) / temperature); top_p; u [nu]
 * uniforms, one pick each, to ids [nu].  status[0] = 1 when top_p keeps no token (the
 * reference raises), else 0.  work: otpu_sample_work_bytes(V) bytes (also holds the km
 * candidate values and ids after the call, km = k rounded up to 8).  Two kernels. */
int64_t otpu_sample_work_bytes(int V);
int otpu_sample(const float* logits, int V, const float* pa, const float* pb, double softcap, int k,
                float itemp, float top_p, const float* u, int nu, void* work, int32_t* ids,
                int32_t* status, otpu_stream_t stream);

/* otpu_sample with no work argument and no allocation.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture, serving loops that
 * forbid it).  The work area is the library's own static device array (1,066,496 bytes on each
 * device the library runs on, held until the process ends), looked up once per device with that
 * device current; so V is at most 262144 (larger: OTPU_EINVAL, use otpu_sample).  The candidate
 * values and ids of the last call stay in that array.  Calls that overlap on one device (two
 * streams, two threads) race on the one array: serialize them. */
int otpu_sample_static(const float* logits, int V, const float* pa, const float* pb, double softcap,
                       int k, float itemp, float top_p, const float* u, int nu, int32_t* ids,
                       int32_t* status, otpu_stream_t stream);

/* The reference's float64 emulation (opentpu/quant.py:895-1067), for checking model code
 * against the operator:
 *   otpu_fake_act: quant.fake_act of x [M, K] fp32 in ranges of n columns (K a multiple of n),
 *   groups of g (16, 32 = QACT, 64, 128 = QST; row_mode: every offset 0): values v [M, K] float64
 *   and da [M, K/16] (each 16-element group's offset).  otpu_fake_act_f64: the same of float64 x
 *   (the reference quantizes x as float64; its tie rule reads x rounded to fp32).
 *   otpu_dequant: quant.dequantize_mxu (values [N, K] float64, exact) and quant.group_offsets
 *   (dw [N, K/16]) of element rows and scale rows (rsc: scale rows of Sw alone; srows NULL:
 *   UNIT, the elements themselves and offsets 0; out NULL: the offsets alone, rows unread;
 *   dw NULL: the values alone).
 *   otpu_mx_matmul: quant.mx_matmul: y [M, N] float64 = h [M, K] @ w [N, K]^T over the
 *   16-element groups MM's window W keeps (da[j, g] + dw[n, g] <= W; da NULL: every group;
 *   dw NULL: offsets 0; dw_rows 1: one offset row for every n). */
int otpu_fake_act(const float* x, int M, int K, int64_t ldx, int n, int g, int row_mode, double* v,
                  int64_t ldv, uint8_t* da, int64_t ldda, otpu_stream_t stream);
int otpu_fake_act_f64(const double* x, int M, int K, int64_t ldx, int n, int g, int row_mode, double* v,
                      int64_t ldv, uint8_t* da, int64_t ldda, otpu_stream_t stream);
int otpu_dequant(const uint8_t* rows, int64_t rs, const uint8_t* srows, int64_t srs, int N, int K, int fmt,
                 int rsc, double* out, int64_t ldo, uint8_t* dw, int64_t lddw, otpu_stream_t stream);
int otpu_mx_matmul(const double* h, int64_t ldh, const uint8_t* da, int64_t ldda, const double* w,
                   int64_t ldw, const uint8_t* dw, int64_t lddw, int dw_rows, int W, int M, int N, int K,
                   double* y, int64_t ldy, otpu_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* OTPU_H */
