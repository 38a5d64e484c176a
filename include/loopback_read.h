/*
 * loopback_read.h -- C ABI of libloopback_read.so, the MI355X (gfx950) kernels of the Loopback depth-attention
 * read ("delta_attnres"): the write step, the read step (scores stored at write time, or computed online), the
 * backward and the RMS-scale gradient.
 *
 * Conventions (every entry point):
 *   - device pointers are plain addresses of device memory; tensors are row-major and contiguous, one row of d
 *     elements per token; every vector pointer (updates, h, x, base, out, g, dv, q rows) is 16-byte aligned;
 *   - n_tok = b * t tokens, d the width (a multiple of 8, at most LDR_MAX_WIDTH); n_tok = 0 is a valid batch, for
 *     which the token-sized buffers may be NULL (as empty tensors give them): nothing is read or written but the
 *     per-read outputs (next_prior);
 *   - dtype is LDR_F32, LDR_BF16 or LDR_F16 and applies to the update-shaped tensors (updates, base, out, g, dv,
 *     h, x), which are loaded into fp32 and rounded back to dtype (round to nearest even, the fp32 result rounded);
 *     every scale, score, coefficient and gradient scalar is fp32;
 *   - per-source arrays (src_v, src_r, ...) are HOST arrays of n device addresses, copied into the kernel
 *     arguments (no device pointer table, no host-to-device copy); n <= LDR_MAX_SOURCES;
 *   - except for the *_any entry points at the end, which take what the others reject: any width d >= 1, rows
 *     aligned to their element size only, up to LDR_ANY_MAX_SOURCES sources, whose addresses come as DEVICE arrays
 *     (n uint64 in device memory, read by the kernels; the caller keeps them until the launch has run);
 *   - stream is a hipStream_t; nothing synchronizes with the host, nothing allocates device memory;
 *   - the return value is 0, a negative LDR_E_* code (rejected before any launch), or a positive hipError_t
 *     from the launch; ldr_strerror() names it.
 * The reference's Python module launches Triton kernels; the entry points below replace those launches one for one
 * (file:line into yancyou/Loopback's fused_dattn.py).
 */
#ifndef LOOPBACK_READ_H
#define LOOPBACK_READ_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LDR_F32 0
#define LDR_BF16 1
#define LDR_F16 2

#define LDR_MAX_SOURCES 64
#define LDR_MAX_WIDTH 8192
#define LDR_MAX_QUERIES 64
#define LDR_ANY_MAX_SOURCES 1024   /* the *_any entry points */

#define LDR_OK 0
#define LDR_E_ARG (-1)    /* null pointer, negative size, bad flag */
#define LDR_E_SHAPE (-2)  /* d not a multiple of 8 or too wide; n or nq out of range (*_any: d < 1, n) */
#define LDR_E_ALIGN (-3)  /* a vector pointer is not 16-byte aligned (*_any: not element-aligned) */
#define LDR_E_DTYPE (-4)  /* dtype is none of LDR_F32, LDR_BF16, LDR_F16 */

/* Version of this ABI; bumped on any signature change or change of what an entry point accepts. A caller compares
 * ldr_abi_version() of the library it loaded with the LDR_ABI_VERSION of the header it was compiled with. */
#define LDR_ABI_VERSION 16
int ldr_abi_version(void);

/* Human-readable text for a return code of any entry point (static storage). */
const char* ldr_strerror(int code);

/* The row layout the kernels use for width d: each row of d/8 eight-element vectors is covered by *tpr lanes
 * holding *vpt vectors each. Exposed for tests; returns LDR_E_SHAPE for an unsupported d. */
int ldr_row_layout(int64_t d, int* vpt, int* tpr);

/* Number of dq partial rows ldr_read_bwd1 writes for (n_tok, d): the caller allocates parts * d fp32. */
int64_t ldr_read_bwd1_parts(int64_t n_tok, int64_t d);

/* r[tok] = rsqrt(sum_k x[tok,k]^2 / d + eps).
 * Replaces _rstd_fwd_kernel and its launches (fused_dattn.py:206-215, 240, 705). Any d >= 1 and any alignment, as
 * the reference's masked kernel: rows the vector layout does not take (d not a multiple of 8 or above
 * LDR_MAX_WIDTH, x not 16-byte aligned) run on scalar loads. */
int ldr_rstd_fwd(const void* x, float* r, int64_t n_tok, int64_t d, float eps, int dtype, void* stream);

/* gx[tok,:] = gr[tok] * (-r[tok]^3) / d * x[tok,:], rounded to dtype.
 * Replaces _rstd_bwd_kernel (fused_dattn.py:218-229, 252). Any d >= 1, alignment and dtype, as ldr_rstd_fwd. */
int ldr_rstd_bwd(const void* x, const float* r, const float* gr, void* gx, int64_t n_tok, int64_t d, int dtype,
                 void* stream);

/* The write step of update s: v_out = round(h - x); r_out[tok] = rsqrt(mean(v_out^2) + eps) of the rounded update
 * (summed in ldr_rstd_fwd's order, so the same bits); and the scores of the update against the read queries
 * j_lo .. nq - 1 of the pass: dots[(j - j_lo) * dots_jstride + tok] = q[j, :] . v_out[tok, :] (dots points at query
 * j_lo's score slice for source s; j_lo == nq: no scores). The scores are formed on the matrix cores from qb, the
 * operand table ldr_split_queries made of the nq fp32 queries, for every dtype: a bf16 update is its own operand, an
 * fp16 one the exact sum of two bf16 values, an fp32 one the sum of three (the six products of parts whose orders
 * sum to at most two). q, the fp32 queries [nq, d], is read only by a build with LDR_WRITE_VALU=1 (the scores on
 * the vector units, a comparison build); it may be NULL otherwise. Replaces _write_stk_kernel (fused_dattn.py:561-585,
 * launched at 684-687; its tensor-core product is tl.dot with tf32x3, 583). */
int ldr_write_dots(const void* h, const void* x, void* v_out, float* r_out, const float* q, const void* qb,
                   int64_t nq, int64_t j_lo, float* dots, int64_t n_tok, int64_t d, int64_t dots_jstride, float eps,
                   int dtype, void* stream);

/* Size of the operand table of nq fp32 queries of width d, in bf16 elements (0 for nq or d out of range). */
int64_t ldr_query_parts_elems(int64_t nq, int64_t d);

/* The matrix-core operand table of nq fp32 queries q [nq, d] (16-byte aligned, ldr_query_parts_elems(nq, d) bf16):
 * each value split into three bf16 parts q = hi + mid + lo (exact to ~2^-24 relative), laid out in the order the
 * write's matrix-core product loads them -- per 64-column chunk, 16-query block, part and k-group half, the 64 lanes'
 * 16-byte operands consecutive (lane l: query 16 b + l mod 16, columns 64 c + 8 (l / 16) + 32 hf .. + 8; zeros past
 * the last query and past d). Replaces the reference's zero-padded transposed query operand QT
 * (fused_dattn.py:657-660). */
int ldr_split_queries(const float* q, int64_t nq, int64_t d, void* qb, void* stream);

/* Online scores: out[i * out_stride + tok] = q . v_i[tok, :] for the n sources (fp32). Together with
 * ldr_read_fwd it is the read without stored scores (replaces the score half of _dattn_fwd_stk_kernel,
 * fused_dattn.py:410-456, and of the list layout's _dattn_fwd_kernel, 55-108). */
int ldr_dots_online(const uint64_t* src_v, int64_t n, const float* q, float* out, int64_t out_stride,
                    int64_t n_tok, int64_t d, int dtype, void* stream);

/* The coefficient inputs of a read (ldr_read_fwd, ldr_read_bwd1) come as the read takes them -- cbar [n_tok, n]
 * and c0 [n] with cbar_cols = c0_cols = n and lam = 1 -- or as the previous read left them, fused with the caller's
 * bookkeeping (looped_transformer.py:383-391): coeffs [n_tok, n-1] and prior [n-1] with cbar_cols = c0_cols = n-1,
 * the newest source's entries implied, cbar = lam * [coeffs, 1] and c0 = lam * [prior, 1] (lam = 1 - beta at an
 * iteration end, 1 otherwise). */

/* The read step over n sources from their raw scores dots[i * dots_stride + tok] = q . v_i:
 *   l_i = dots_i * r_i * inv_sqrt_d + log(max(c0_i, 1e-8));  p = softmax_i(l);  p0 = softmax_i(lc)
 *   tc_i = c0_i + M (p_i - p0_i),  M = sum_i c0_i
 *   out = round(base + sum_i (tc_i - cbar_i) v_i)   (fp32 accumulation, one rounding)
 * (softmax as exp(l - max) / sum). With h0 != NULL (an iteration end, fused with looped_transformer.py:380-381) base
 * is the proposal and the read first forms round(base + round(beta * round(h0 - base))), the caller's own rounding
 * sequence. Stores tc [n_tok, n], the probabilities p [n_tok, n] for the backward (p may be NULL: a read without a
 * backward), and c0 into next_prior [n] when not NULL (the caller's next prior). Replaces _dattn_fwd_dots_kernel (fused_dattn.py:588-625, launched at 748-751)
 * and the weighted-sum half of _dattn_fwd_stk_kernel / _dattn_fwd_kernel (410-456 / 55-108). */
int ldr_read_fwd(const uint64_t* src_v, const uint64_t* src_r, int64_t n, const float* dots, int64_t dots_stride,
                 const void* base, const void* h0, float beta, const float* cbar, int64_t cbar_cols, const float* c0,
                 int64_t c0_cols, float lam, float inv_sqrt_d, void* out, float* tc, float* p, float* next_prior,
                 int64_t n_tok, int64_t d, int dtype, void* stream);

/* The read step without stored scores, in one pass over the sources: the raw scores q . v_i are formed as the
 * sources stream and stored into dots[i * dots_stride + tok] (for the backward; required), and the outputs are
 * those of ldr_read_fwd on those scores (out up to fp32 summation order: the weighted sum runs as an online softmax
 * against a running maximum; tc and p from the same softmax as ldr_read_fwd, so a zero query with cbar == c0 gives
 * tc == c0 and out == base bitwise). q is the read's query, fp32 [d]. Rows wider than one wave (d > 2048)
 * take two passes inside the call (ldr_dots_online, then ldr_read_fwd). Replaces _dattn_fwd_stk_kernel
 * (fused_dattn.py:410-456, the stacked read with LOOP_DATTN_DOTS=0) and the list layout's _dattn_fwd_kernel
 * (55-108), each one pass over the sources. */
int ldr_read_fwd_online(const uint64_t* src_v, const uint64_t* src_r, int64_t n, const float* q, float* dots,
                        int64_t dots_stride, const void* base, const void* h0, float beta, const float* cbar,
                        int64_t cbar_cols, const float* c0, int64_t c0_cols, float lam, float inv_sqrt_d, void* out,
                        float* tc, float* p, float* next_prior, int64_t n_tok, int64_t d, int dtype, void* stream);

/* Backward pass 1 of a read (the only re-read of the sources), with g = dL/dout, gt = dL/dtc (NULL = zeros), and
 * the forward's p and raw scores dots (as ldr_read_fwd took them):
 *   gd_i = g . v_i,  gp_i = M (gd_i + gt_i),  Sacc = sum_i p_i gp_i,  dz_i = p_i (gp_i - Sacc)
 *   dcbar[tok, i] = -lam gd_i for i < dcbar_cols (the gradient of cbar, or with dcbar_cols = n-1 that of the
 *     previous coefficients through the caller's bookkeeping)
 *   dr_i[tok] (+)= dz_i dots_i inv_sqrt_d   (= dz_i z_i / r_i; added when dr_accum != 0)
 *   wz[(i * wz_stride + tok) * 2 + {0,1}] = (tc_i - cbar_i, dz_i r_i inv_sqrt_d)   (the pass-2 scalars)
 *   dq_part[p * dq_part_stride + c] = per-workgroup partial of sum_tok sum_i dz_i r_i v_i inv_sqrt_d
 *     (ldr_read_bwd1_parts rows p; dq_part_stride >= d: with a stride of k d, k reads' partials interleave as
 *     [p][read][d] and one ldr_reduce_rows over rows of k d sums them all)
 *   with g_prop and / or g_h0 (each may be NULL): the iteration-end blend's gradients g_h0 = round(beta g),
 *     g_prop = round(g - g_h0), rounded as autograd rounds them
 * Replaces _dattn_bwd1_stk_kernel (fused_dattn.py:459-493, launched at 777-779) and pass 1 of _dattn_bwd_kernel
 * (111-151); dr is also the dR update of _dattn_bwd2_stk_kernel (532-535). */
int ldr_read_bwd1(const uint64_t* src_v, const uint64_t* src_r, int64_t n, const void* g, const float* gt,
                  const float* p, const float* dots, int64_t dots_stride, const float* tc, const float* cbar,
                  int64_t cbar_cols, const float* c0, int64_t c0_cols, float lam, float inv_sqrt_d, float* dcbar,
                  int64_t dcbar_cols, const uint64_t* dr, int dr_accum, float* wz, int64_t wz_stride,
                  float* dq_part, int64_t dq_part_stride, void* g_prop, void* g_h0, float beta, int64_t n_tok,
                  int64_t d, int dtype, void* stream);

/* Backward pass 1 and its query gradient in one call that allocates nothing and takes no workspace: every output
 * of ldr_read_bwd1 (same arguments) except the partials, and dq[c] = sum_tok sum_i dz_i r_i v_i[c] inv_sqrt_d
 * (fp32, d; zeros for an empty batch) -- the bits of ldr_read_bwd1 followed by ldr_reduce_rows over its partials.
 * No counterpart in the reference: it is for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops, harnesses that forbid allocation). The partials go to a device array the library holds on
 * each GPU it runs on (LDR_B1_GRID x LDR_MAX_WIDTH fp32: 512 x 8192 x 4 B = 16 MiB with the default launch settings,
 * kept until the process ends; its address is looked up once per device on the first call there, so under HIP graph
 * capture make one call on that device first, outside capture -- an empty batch, n_tok = 0, suffices). Calls that
 * overlap on one GPU (on two streams, or from two threads) share that array and race: serialize them. Returns
 * LDR_E_SHAPE for a width or batch whose partials would not fit the array (none with d <= LDR_MAX_WIDTH at the
 * default launch settings). */
int ldr_read_bwd1_noalloc(const uint64_t* src_v, const uint64_t* src_r, int64_t n, const void* g, const float* gt,
                          const float* p, const float* dots, int64_t dots_stride, const float* tc, const float* cbar,
                          int64_t cbar_cols, const float* c0, int64_t c0_cols, float lam, float inv_sqrt_d,
                          float* dcbar, int64_t dcbar_cols, const uint64_t* dr, int dr_accum, float* wz,
                          int64_t wz_stride, float* dq, void* g_prop, void* g_h0, float beta, int64_t n_tok, int64_t d,
                          int dtype, void* stream);

/* out[c] = sum_p part[p * d + c] in a fixed order (deterministic).
 * Replaces the torch dq_part.sum(0) (fused_dattn.py:317, 785). */
int ldr_reduce_rows(const float* part, int64_t rows, int64_t d, float* out, void* stream);

/* Backward pass 2 of the list layout: dv_i = w_i g + dzr_i q (w, dzr from ldr_read_bwd1's wz), written to the
 * n per-source gradient tensors, or added (accum != 0) as prev + round(dv_i), rounded again: autograd's own
 * accumulation of per-read gradients. Replaces pass 2 of _dattn_bwd_kernel (fused_dattn.py:152-181). */
int ldr_read_bwd2_list(const uint64_t* dv, int64_t n, int accum, const void* g, const float* q, const float* wz,
                       int64_t wz_stride, int64_t n_tok, int64_t d, int dtype, void* stream);

/* The stacked layout's gradient of update i, formed once after every read of it has run its backward:
 *   dv[tok,:] = round( sum_e ( w_e[tok] g_e[tok,:] + dzr_e[tok] q_e[:] ) + gr[tok] (-r[tok]^3) / d * v[tok,:] )
 * over the m reads e that hold update i: g_e that read's output gradient, (w_e, dzr_e) its wz pair for source i
 * (float2 per token), q_e its query (fp32, d). One fp32 sum, one rounding; gr may be NULL (no scale gradient).
 * dv_neg (may be NULL) receives -dv, the write's gradient to x (fused_dattn.py:694-695). With add != NULL (another
 * gradient of the write's h, e.g. the read that took h as its proposal) dv holds round(dv + a) instead, the sum
 * autograd would form, with a = add, or, when add_beta != 0 (add being the output gradient g of a read whose base
 * was the iteration-end blend), the blend's share of it a = round(add - round(add_beta * add)); dv_neg stays -dv.
 * per_read = 1 rounds as the list layout does instead: each read's share round(w_e g_e + dzr_e q_e) (one fused
 * multiply-add over the rounded product dzr q, as ldr_read_bwd2_list) added to the running gradient in dtype, in
 * table order, then round(gr (-r^3) / d * v) added last -- autograd's accumulation of the per-read gradients when the
 * table lists the reads from the last to the first (the reference's stack read-modify-writes dV the same way,
 * fused_dattn.py:528-531); per_read = 0 (the default) forms one fp32 sum rounded once.
 * Replaces the dV read-modify-write of _dattn_bwd2_stk_kernel (fused_dattn.py:496-536, launched at 781-784) and
 * _rstd_bwd_acc_kernel (539-552, launched at 717-719). */
int ldr_dv_assemble(const uint64_t* g, const uint64_t* wz, const uint64_t* q, int64_t m, const void* v,
                    const float* r, const float* gr, const void* add, float add_beta, int per_read, void* dv,
                    void* dv_neg, int64_t n_tok, int64_t d, int dtype, void* stream);

/* out = round( sum_j round(beta * g_j) ) over m update-shaped tensors (fp32 sum): the gradient of h0 from the m
 * iteration-end blends of a pass (looped_transformer.py:380-381, base = proposal + beta (h0 - proposal)), formed
 * once from the reads' output gradients instead of one tensor per blend added up by autograd; per_read = 1 adds the
 * rounded shares in dtype in table order instead, as autograd adds them (list the blends from the last to the
 * first). No reference counterpart (the reference leaves these adds to autograd). */
int ldr_blend_sum(const uint64_t* g, int64_t m, float beta, int per_read, void* out, int64_t n_tok, int64_t d,
                  int dtype, void* stream);

/* ---- any-shape entry points ----------------------------------------------------------------------------------
 * The same computations for the shapes the entry points above reject -- the reference's kernels mask any width
 * and any source count (BLOCK_D = next_pow2(d), BLOCK_N = next_pow2(n): fused_dattn.py:60-63, 191-194) -- with
 * per-source addresses in device arrays (see the conventions at the top). One wave per token row; they are the
 * general path, not the fast one (the module routes to them only for such shapes). */

/* ldr_read_fwd (q == NULL: dots holds the stored raw scores) and ldr_read_fwd_online (q != NULL: the scores are
 * formed and stored into dots) for any shape: the same outputs and formulas; a zero query with cbar == c0 gives
 * tc == c0 and out == base bitwise. q, when given, is fp32 [d]. Replaces _dattn_fwd_kernel (fused_dattn.py:55-108),
 * _dattn_fwd_stk_kernel (410-456) and _dattn_fwd_dots_kernel (588-625) at the shapes ldr_read_fwd does not take. */
int ldr_read_fwd_any(const uint64_t* src_v, const uint64_t* src_r, int64_t n, const float* q, float* dots,
                     int64_t dots_stride, const void* base, const void* h0, float beta, const float* cbar,
                     int64_t cbar_cols, const float* c0, int64_t c0_cols, float lam, float inv_sqrt_d, void* out,
                     float* tc, float* p, float* next_prior, int64_t n_tok, int64_t d, int dtype, void* stream);

/* ldr_read_bwd1 for any shape (dr a device array too): the same outputs, with the query-gradient partials in
 * dq_parts rows of dq_part (1 <= dq_parts <= 65535, chosen by the caller; every row is written, zeros where a
 * workgroup had no token; row stride dq_part_stride >= d, so reads' partials can interleave as for ldr_read_bwd1),
 * summed by ldr_reduce_rows over dq_parts rows. wz must be 8-byte aligned. Replaces _dattn_bwd1_stk_kernel
 * (fused_dattn.py:459-493) and pass 1 of _dattn_bwd_kernel (111-151) at the shapes ldr_read_bwd1 does not take. */
int ldr_read_bwd1_any(const uint64_t* src_v, const uint64_t* src_r, int64_t n, const void* g, const float* gt,
                      const float* p, const float* dots, int64_t dots_stride, const float* tc, const float* cbar,
                      int64_t cbar_cols, const float* c0, int64_t c0_cols, float lam, float inv_sqrt_d, float* dcbar,
                      int64_t dcbar_cols, const uint64_t* dr, int dr_accum, float* wz, int64_t wz_stride,
                      float* dq_part, int64_t dq_parts, int64_t dq_part_stride, void* g_prop, void* g_h0, float beta,
                      int64_t n_tok, int64_t d, int dtype, void* stream);

/* ldr_dv_assemble for any shape (g, wz, q device arrays; 0 <= m <= LDR_ANY_MAX_SOURCES): the same roundings in the
 * same order, so the bits of ldr_dv_assemble for the same tables. Replaces _dattn_bwd2_stk_kernel
 * (fused_dattn.py:496-536) and _rstd_bwd_acc_kernel (539-552) at the shapes ldr_dv_assemble does not take. */
int ldr_dv_assemble_any(const uint64_t* g, const uint64_t* wz, const uint64_t* q, int64_t m, const void* v,
                        const float* r, const float* gr, const void* add, float add_beta, int per_read, void* dv,
                        void* dv_neg, int64_t n_tok, int64_t d, int dtype, void* stream);

/* ldr_read_bwd2_list for any shape (dv a device array). Replaces pass 2 of _dattn_bwd_kernel (fused_dattn.py:
 * 152-181) at the shapes ldr_read_bwd2_list does not take. */
int ldr_read_bwd2_list_any(const uint64_t* dv, int64_t n, int accum, const void* g, const float* q, const float* wz,
                           int64_t wz_stride, int64_t n_tok, int64_t d, int dtype, void* stream);

/* ldr_blend_sum for any shape (g a device array): the same sum in the same order. No reference counterpart (the
 * reference leaves these adds to autograd, looped_transformer.py:380-381). */
int ldr_blend_sum_any(const uint64_t* g, int64_t m, float beta, int per_read, void* out, int64_t n_tok, int64_t d,
                      int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LOOPBACK_READ_H */
