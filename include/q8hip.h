/*
 * q8hip.h -- C ABI of libq8hip.so, the MI355X (gfx950) implementation of the
 * INT8 group-quantized, weight-only (W8A32) linear-layer path.
 *
 * The reference keeps weights in one u16 "weight arena" and activations in
 * one f32 "activation arena" and addresses tensors by element offsets into
 * them (src/resident.mojo:15-58, src/llama_common.mojo:578-606).  This ABI
 * keeps that convention: buffers are opaque handles, and every tensor is a
 * (buffer, offset) pair with offsets in the arena's element units (u16 for
 * weights, f32 for activations).  Only plain integers and pointers cross the
 * boundary, so Mojo's sys.ffi (or ctypes, cgo, ...) can bind every entry
 * point without struct-by-value.
 *
 * Packed row layout (qwen3_mojo/scripts/quantize.py:4-12,41-43):
 *     [ (m/G) scales | m int8 codes ]          as little-endian u16 elements
 * scale_dtype Q8_SCALE_F16 stores each scale as one binary16 (the reference
 * layout, G = 64); Q8_SCALE_F32 stores each scale as an f32 (two u16).
 * Supported group sizes: 32 and 64.
 *
 * Every call validates its arguments on the host before any HIP call and
 * returns a status (0 = OK, < 0 = error); q8_last_error(ctx) gives the
 * message.  Compute calls are asynchronous on the context's stream and a
 * context must not be used from two threads at once (the reference runs one
 * in-order queue per DeviceContext).
 */
#ifndef Q8HIP_H
#define Q8HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---------------------------------------------------- */
#define Q8_OK              0
#define Q8_ERR_ARG        -1   /* null handle, negative size, bad enum      */
#define Q8_ERR_SHAPE      -2   /* m % G != 0, s/n/m out of range            */
#define Q8_ERR_RANGE      -3   /* offset + extent beyond the buffer         */
#define Q8_ERR_HIP        -4   /* HIP runtime error                         */
#define Q8_ERR_NOMEM      -5   /* device allocation failed                  */
#define Q8_ERR_NODEVICE   -6   /* arguments valid, but the context is a     */
                               /* host-only validation context (device -1)  */
#define Q8_ERR_UNSUPPORTED -7  /* valid request this build does not handle  */

/* ---- enums ------------------------------------------------------------ */
#define Q8_SCALE_F16 1         /* binary16 scale per group (reference)      */
#define Q8_SCALE_F32 2         /* f32 scale per group                       */
#define Q8_SRC_BF16  1         /* pack input dtype                          */
#define Q8_SRC_F32   2

#define Q8_DEVICE_NONE (-1)    /* q8_create: host-only validation context   */

typedef struct q8_ctx q8_ctx;
typedef struct q8_buf q8_buf;

/* ---- library / context ------------------------------------------------ */

/* ABI version of this header (major * 100 + minor). */
int q8_version(void);

/* Packed row length in u16 elements for m inputs; 0 if (m, G, scale_dtype)
 * is invalid.  Replaces q8_rowstride (src/llama_q8.mojo:26-28). */
uint64_t q8_rowstride_u16(int64_t m, int G, int scale_dtype);

/* Create a context on HIP device `device_ordinal` owning one HIP stream.
 * Q8_DEVICE_NONE creates a host-only context: buffers carry sizes only and
 * compute calls validate their arguments and return Q8_ERR_NODEVICE.
 * Replaces DeviceContext() + Q8Kernels(ctx) (src/llama_q8.mojo:115-121). */
int q8_create(int device_ordinal, q8_ctx **out);
void q8_destroy(q8_ctx *ctx);

/* Run subsequent calls on an existing hipStream_t (NULL: the context's own
 * stream).  The caller keeps ownership of the stream. */
int q8_set_stream(q8_ctx *ctx, void *hip_stream);
void *q8_get_stream(q8_ctx *ctx);

/* Wait for all work queued on the context's stream (ctx.synchronize()). */
int q8_sync(q8_ctx *ctx);

/* Message of the last failing call on this context ("" if none).  With
 * ctx == NULL: the last error of a failed q8_create or q8_linear_noalloc on
 * this thread. */
const char *q8_last_error(q8_ctx *ctx);

/* ---- buffers (arenas) --------------------------------------------------- */

/* Library-owned device allocation (enqueue_create_buffer,
 * src/resident.mojo:22, src/llama_common.mojo:588). */
int q8_buf_alloc(q8_ctx *ctx, uint64_t nbytes, q8_buf **out);
/* Non-owning view of caller device memory (e.g. a torch tensor). */
int q8_buf_wrap(q8_ctx *ctx, void *device_ptr, uint64_t nbytes, q8_buf **out);
void q8_buf_free(q8_ctx *ctx, q8_buf *buf);
uint64_t q8_buf_size(const q8_buf *buf);
void *q8_buf_device_ptr(const q8_buf *buf);

/* Host <-> device copies, synchronous with respect to the host
 * (map_to_host + memcpy, src/resident.mojo:32-58). */
int q8_buf_upload(q8_ctx *ctx, q8_buf *buf, uint64_t byte_off,
                  const void *src, uint64_t nbytes);
int q8_buf_download(q8_ctx *ctx, q8_buf *buf, uint64_t byte_off,
                    void *dst, uint64_t nbytes);

/* ---- the Q8 path ---------------------------------------------------------- */

/* Quantize and pack n rows of m weights (bf16 or f32, at element offset
 * src_off of src) into packed rows at u16 offset dst_off of dst.  Codes and
 * scales are bit-identical to pack_q8 (qwen3_mojo/scripts/quantize.py:31-43)
 * for G = 64 / Q8_SCALE_F16.  Q8_SCALE_F32 keeps the scale in f32. */
int q8_quantize_pack(q8_ctx *ctx, q8_buf *src, uint64_t src_off, int src_dtype,
                     int64_t n, int64_t m, q8_buf *dst, uint64_t dst_off_u16,
                     int G, int scale_dtype);

/* y[s, n] = x[s, m] . deq(W[n, m])^T in f32, with x at f32 offset ox and y
 * at f32 offset oy of the activation arena `a`, and W's packed rows at u16
 * offset owt of the weight arena `w` -- the k_mm_q8 / mm_q8_op contract
 * (src/llama_q8.mojo:54-93,124-141).  y must not overlap x.  The caller
 * allocates y (Acts.alloc), as mm_q8_op does.  One row runs the f32 GEMV
 * and 2 .. 4 rows f32 4x4-block MFMA, both with f32 products of x and the
 * codes; 5 .. 31 rows split each x into two bf16 terms hi + lo (x - hi - lo
 * below 2^-17 |x|, so x is carried to that bound, not exactly) whose
 * products with the codes are exact on bf16 MFMA; all three stay within
 * 1e-5 of float64.  s >= 32 runs the dequant-GEMM on f16 MFMA (binary16 x
 * rows after a power-of-two scaling, binary16 q * s), whose max-rel-err
 * stays near 2e-4. */
int q8_linear(q8_ctx *ctx, q8_buf *w, uint64_t owt_u16, q8_buf *a,
              uint64_t ox_f32, uint64_t oy_f32, int64_t s, int64_t m, int64_t n,
              int G, int scale_dtype);

/* Prefill variant with bf16 activations: x bf16 [s, m] at element offset ox
 * of buffer x, y f32 [s, n] at f32 offset oy of buffer y.  Runs as the
 * dequant-GEMM on f16 MFMA: each x row scaled by a power of two into
 * binary16 (exact for bf16 values), weights q * s rounded once to binary16
 * (twice with f32 scales), f32 accumulation; max-rel-err stays near 2e-4.
 * No reference counterpart (the reference is W8A32 only); it is the
 * M = 512 bf16-activation prefill case. */
int q8_linear_bf16act(q8_ctx *ctx, q8_buf *w, uint64_t owt_u16, q8_buf *x,
                      uint64_t ox_bf16, q8_buf *y, uint64_t oy_f32, int64_t s,
                      int64_t m, int64_t n, int G, int scale_dtype);

/* q8_linear on raw device pointers, without any allocation.  No counterpart
 * in the reference: it is for callers that cannot call hipMalloc (code under
 * HIP graph capture, tight serving loops, harnesses that forbid it), who
 * need no context.  y[s, n] = x[s, m] . deq(W[n, m])^T exactly as q8_linear
 * computes it (same kernels and split decisions, so the same bits, except
 * from s = 32 on when the rows do not fit the 16 MiB activation buffer at
 * once: they then run in chunks, within the same 1e-3 contract), on
 * hip_stream (NULL: the null stream), which must belong to the current
 * device.  w points at packed row 0 (rows back to back) and must be 2-byte
 * aligned; x and y are f32, 4-byte aligned, and must not overlap (else
 * Q8_ERR_ARG).
 * Scratch: one fixed __device__ array of Q8_NOALLOC_SCRATCH_BYTES (32 MiB)
 * per GPU, resident on every GPU where the library's code object is loaded
 * until the process ends, used or not (16 MiB of split-K partials and a
 * 16 MiB binary16 activation buffer for s >= 32, which takes the rows in
 * chunks).
 * Limit: from s = 32 on, one activation row (2 m + 4 bytes) plus 4 n bytes
 * must fit in 16 MiB, else Q8_ERR_SHAPE.  Every call on a GPU shares that
 * GPU's array: calls that overlap on one GPU (two streams, two threads)
 * race; calls in one stream's order do not.  Errors: status code, message in
 * q8_last_error(NULL) on the calling thread. */
#define Q8_NOALLOC_SCRATCH_BYTES (33554432LL)   /* 16 MiB + 16 MiB */
int q8_linear_noalloc(void *hip_stream, const void *w, const float *x, float *y, int64_t s,
                      int64_t m, int64_t n, int G, int scale_dtype);

/* y[i, c] = f32(q[id_i, c]) * f32(scale[id_i, c / G]) for i < s, c < d:
 * embedding rows gathered from packed rows (k_embed_gather_q8,
 * src/llama_q8.mojo:96-109).  ids are int32 at element offset oids of `ids`;
 * `vocab` is the number of packed rows at oemb.  An id outside [0, vocab)
 * yields a row of NaN instead of an out-of-bounds read. */
int q8_embed_gather(q8_ctx *ctx, q8_buf *w, uint64_t oemb_u16, q8_buf *ids,
                    uint64_t oids_i32, q8_buf *a, uint64_t oy_f32, int64_t s,
                    int64_t d, int64_t vocab, int G, int scale_dtype);

/* ---- decode-step layer kernels ------------------------------------------------
 * The non-linear parts of run_layer_q8 and of the token loop
 * (src/llama_q8.mojo:144-230, qwen3_mojo/src/qwen_q8.mojo:127-162), over the
 * same arenas: f32 activations at float offsets of `a`, bf16 norm vectors at
 * u16 offsets of the weight arena `w`.  The KV cache is a separate binary16
 * buffer `kv` (the reference keeps an f32 cache in the activation arena).
 * Outputs may coincide exactly with an input (in place) but must not
 * otherwise overlap one. */

/* One-row Q8 linear with its neighbours folded into the same launch (the
 * decode step's s = 1 GEMVs).  How x is read (pre):
 *   Q8_PRE_NONE:    x (m floats)
 *   Q8_PRE_RMSNORM: rmsnorm(x) as q8_rmsnorm, with the d = m bf16 weights at
 *                   onorm of `w` and eps; the norm factor is applied to each
 *                   output (W (wn x / r) = (W (wn x)) / r), so results match
 *                   q8_rmsnorm + q8_linear to float rounding, not to the bit
 *   Q8_PRE_SWIGLU:  x = [g | u] (2m floats), read as silu(g) * u (as q8_swiglu)
 * What is stored (post):
 *   Q8_POST_STORE:    y = W x~ (n floats)
 *   Q8_POST_RESIDUAL: y = res + W x~, res = n floats at ores, may be y itself
 *   Q8_POST_SWIGLU:   rows [0, n/2) are gate rows and [n/2, n) up rows (the
 *                     fused gate|up weights); y = silu(W_g x~) * (W_u x~), n/2
 *                     floats (as q8_linear + q8_swiglu)
 * x must not overlap y.  Without Q8_PRE_RMSNORM the results equal the
 * separate calls to the bit.  Needs m % 32 == 0, 16-byte aligned rows and
 * x, 8-byte aligned norm weights and, with a prologue, m <= 16384
 * (Q8_ERR_UNSUPPORTED otherwise).
 * Replaces rmsnorm_op + mm_q8_op, mm_q8_op + swiglu_mul_op and mm_q8_op +
 * res_add_op / add_op of run_layer_q8 (src/llama_q8.mojo:144-230). */
#define Q8_PRE_NONE 0
#define Q8_PRE_RMSNORM 1
#define Q8_PRE_SWIGLU 2
#define Q8_POST_STORE 0
#define Q8_POST_RESIDUAL 1
#define Q8_POST_SWIGLU 2
int q8_linear_fused(q8_ctx *ctx, q8_buf *w, uint64_t owt_u16, q8_buf *a,
                    uint64_t ox_f32, uint64_t oy_f32, int64_t m, int64_t n, int G,
                    int scale_dtype, int pre, uint64_t onorm_u16, float eps,
                    int post, uint64_t ores_f32);

/* y = W (silu(g) * u) for s rows of gate g (s x m floats at og) and up u
 * (s x m at ou): the prompt path's swiglu folded into the binary16 pre-pass
 * of the dequant-GEMM (the same bits as q8_swiglu into g, then q8_linear on
 * g; g and u are left as they were).  s >= 32 (fewer rows: q8_swiglu, then
 * q8_linear); g, u and the weight rows 16-byte aligned, m a multiple of 8.
 * Row i of g and of u starts at og + i*ld and ou + i*ld (ld = 0: m; else
 * at least m and a multiple of 4 -- gate|up from one stacked q8_linear of
 * 2m outputs: ou = og + m, ld = 2m).
 * Replaces swiglu_mul_op + the down projection's mm_q8_op of run_layer_q8
 * (src/llama_q8.mojo:221-225) for prompt rows. */
int q8_linear_swiglu(q8_ctx *ctx, q8_buf *w, uint64_t owt_u16, q8_buf *a, uint64_t og_f32,
                     uint64_t ou_f32, uint64_t oy_f32, int64_t s, int64_t m, int64_t n, int G,
                     int scale_dtype, int64_t ld);

/* y = W rmsnorm(h) for s rows (s x m floats at ox), h = x, or with has_res
 * h = x + res (res: s x m at ores), h then also stored at oh (which may be
 * x or res itself): the prompt path's RMSNorm (and residual add) folded into
 * the binary16 pre-pass of the dequant-GEMM.  Norm weights: m bf16 values at
 * onorm_u16 of w.  The same bits as q8_rmsnorm (or q8_add_rmsnorm) into a
 * temporary, then q8_linear on it; the normalised rows are not stored.
 * s >= 32 and m <= 16384 (otherwise the two calls); x and the weight rows
 * 16-byte aligned, m a multiple of 8; y may not overlap x, res or h.
 * Replaces rmsnorm_op + mm_q8_op (q|k|v, src/llama_q8.mojo:159-170) and
 * k_res_add + rmsnorm_op + mm_q8_op (gate|up, :207-220) of run_layer_q8
 * for prompt rows. */
int q8_linear_rmsnorm(q8_ctx *ctx, q8_buf *w, uint64_t owt_u16, uint64_t onorm_u16, float eps,
                      q8_buf *a, uint64_t ox_f32, int has_res, uint64_t ores_f32,
                      uint64_t oh_f32, uint64_t oy_f32, int64_t s, int64_t m, int64_t n, int G,
                      int scale_dtype);

/* The end of a token step in two launches: logits y (n floats at oy) = W
 * rmsnorm(x) over the lm_head's n packed rows (norm weights at onorm of w;
 * as q8_linear_fused with Q8_PRE_RMSNORM), their argmax (as q8_argmax: the
 * lowest index of the largest value, 0 when y[0] is NaN) written to
 * ids[oid], the position at posbuf[opos] advanced by pos_step (posbuf NULL:
 * none) and, with gather != 0, the embedding row of that id -- from the n
 * packed rows of m at oemb of w, as q8_embed_gather -- written to x_next
 * (m floats at onext of a), ready for the next step.  The argmax partials
 * live in the context's workspace.  Needs m <= 16384, m % 32 == 0 and the
 * alignment of q8_linear_fused.
 * Replaces the final rmsnorm_op + lm_head mm_q8_op + argmax_op + the next
 * embed of the token loop (qwen3_mojo/src/qwen_q8.mojo:110-162). */
int q8_head_argmax(q8_ctx *ctx, q8_buf *w, uint64_t owt_u16, uint64_t onorm_u16, float eps,
                   q8_buf *a, uint64_t ox_f32, uint64_t oy_f32, int64_t m, int64_t n, int G,
                   int scale_dtype, q8_buf *ids, uint64_t oid_i32, q8_buf *posbuf,
                   uint64_t opos_i32, int64_t pos_step, int gather, uint64_t oemb_u16,
                   uint64_t onext_f32);

/* y = bf16(wn) * x / sqrt(mean(x^2) + eps) for `rows` rows of d, wn = d bf16
 * values at owt (k_rmsnorm_w / rmsnorm_op, src/llama_common.mojo:197-225,
 * 690-696). */
int q8_rmsnorm(q8_ctx *ctx, q8_buf *w, uint64_t owt_u16, q8_buf *a,
               uint64_t ox_f32, uint64_t oy_f32, int64_t rows, int64_t d,
               float eps);

/* Per-head RMSNorm (k_rmsnorm2_w, src/llama_common.mojo:228-270: the q and k
 * head norms of Qwen3) of `heads` consecutive head rows of head_dim in each
 * of `tokens` rows, token rows ld floats apart (ld = 0: heads * head_dim),
 * e.g. the q or k heads inside stacked q|k|v rows; y has x's layout and may
 * be x itself (in place), else it may not overlap x.  Each head row gets the
 * bits q8_rmsnorm gives it as a dense row. */
int q8_head_rmsnorm(q8_ctx *ctx, q8_buf *w, uint64_t owt_u16, q8_buf *a, uint64_t ox_f32,
                    uint64_t oy_f32, int64_t tokens, int64_t heads, int64_t head_dim, int64_t ld,
                    float eps);

/* h = x + o stored at oh, then y = rmsnorm(h): k_res_add then k_rmsnorm_w
 * (src/llama_common.mojo:354-359,197-225) in one dispatch. */
int q8_add_rmsnorm(q8_ctx *ctx, q8_buf *w, uint64_t owt_u16, q8_buf *a,
                   uint64_t ox_f32, uint64_t oo_f32, uint64_t oh_f32,
                   uint64_t oy_f32, int64_t rows, int64_t d, float eps);

/* RoPE (rotate_half; head_dim/2 inverse frequencies at oinv) in place on
 * q [s, nheads*head_dim] at oq and k [s, nkv*head_dim] at ok, and append the
 * rotated k and the v [s, nkv*head_dim] at ov to cache rows pos0 .. pos0+s-1
 * of the layer's K block (maxlen rows of nkv*head_dim binary16 at f16 offset
 * okc of kv) and V block (at ovc) -- k_rope_qk_copy2
 * (src/llama_common.mojo:299-342).  With posbuf != NULL the position is
 * instead the int32 at element offset opos of posbuf, read by the kernel
 * (a captured step then serves every position; rows past maxlen are dropped,
 * and attention clamps its context to maxlen).  ld = 0: q, k and v are dense
 * row-major; ld > 0: row i of each sits ld floats after row i-1 (q|k|v
 * stacked in rows of one q8_linear output, ok = oq + nheads*head_dim,
 * ov = ok + nkv*head_dim, ld = their sum); ld must be at least each row
 * width, and k's columns must not meet q's at that stride (Q8_ERR_ARG). */
int q8_rope_kv(q8_ctx *ctx, q8_buf *a, uint64_t oq_f32, uint64_t ok_f32,
               uint64_t ov_f32, uint64_t oinv_f32, q8_buf *kv, uint64_t okc_f16,
               uint64_t ovc_f16, int64_t maxlen, int64_t s, int64_t pos0,
               q8_buf *posbuf, uint64_t opos_i32, int nheads, int nkv,
               int head_dim, int64_t ld);

/* Floats of activation-arena scratch q8_attention needs (0 from s = 16 on,
 * where attention is one pass on the matrix cores). */
uint64_t q8_attention_scratch_floats(int64_t s, int nheads, int head_dim,
                                     int64_t maxlen);

/* out [s, nheads*head_dim] at oy = causal GQA attention of the rotated
 * q at oq (query row i at position pos0 + i attends cache rows
 * 0 .. pos0 + i; head h reads KV head h / (nheads / nkv); scores scaled by
 * 1/sqrt(head_dim)) -- k_scores, k_softmax_rows and k_att_out
 * (src/llama_common.mojo:402-473) with their score buffer replaced by an
 * online softmax: for s >= 16 one MFMA pass per (16..128-row block, KV
 * head), below that per-split partials in q8_attention_scratch_floats()
 * floats at oscratch (oscratch is unused when that is 0).  head_dim 64 or
 * 128, nheads / nkv in {1, 2, 4, 8}.  Position as in q8_rope_kv.  Row i of q
 * at oq + i*ldq (ldq = 0: nheads*head_dim, dense); out is dense.  From
 * s = 16 on, q and out must start 16-byte aligned and ldq be a multiple of 4
 * (Q8_ERR_UNSUPPORTED otherwise). */
int q8_attention(q8_ctx *ctx, q8_buf *a, uint64_t oq_f32, q8_buf *kv,
                 uint64_t okc_f16, uint64_t ovc_f16, int64_t maxlen,
                 uint64_t oy_f32, uint64_t oscratch_f32, int64_t s, int64_t pos0,
                 q8_buf *posbuf, uint64_t opos_i32, int nheads, int nkv,
                 int head_dim, int64_t ldq);

/* Decode step of one new token (s = 1): with wn non-null, per-head RMSNorm
 * of q and of k first (the head_dim bf16 weights at oqnorm / oknorm of wn,
 * eps; k_rmsnorm2_w, src/llama_common.mojo:228-270, the same values as
 * q8_rmsnorm over the head rows); RoPE of q at oq and k at ok, append of the
 * rotated k and of v at ov to cache row pos0 (as q8_rope_kv) and causal
 * attention of the token over rows 0 .. pos0 into out at oy (as
 * q8_attention), in two launches (context splits, then their merge).  q and
 * k in the arena are left as they were.  The split records live in the
 * context's workspace, so calls on one context must not overlap (they do
 * not when issued on its stream).  head_dim 64 or 128, nheads / nkv in
 * {1, 2, 4, 8}; a cache block must stay under 2 GiB; position as in
 * q8_rope_kv.
 * Replaces the per-token attention of run_layer_q8 (src/llama_q8.mojo:171-205:
 * k_rmsnorm2_w, k_rope_qk_copy2, k_scores, k_softmax_rows, k_att_out). */
int q8_decode_attention(q8_ctx *ctx, q8_buf *a, uint64_t oq_f32, uint64_t ok_f32,
                        uint64_t ov_f32, uint64_t oinv_f32, q8_buf *kv, uint64_t okc_f16,
                        uint64_t ovc_f16, int64_t maxlen, uint64_t oy_f32, int64_t pos0,
                        q8_buf *posbuf, uint64_t opos_i32, int nheads, int nkv, int head_dim,
                        q8_buf *wn, uint64_t oqnorm_u16, uint64_t oknorm_u16, float eps);

/* g = silu(g) * u in place over n values (k_swiglu_mul,
 * src/llama_common.mojo:476-481). */
int q8_swiglu(q8_ctx *ctx, q8_buf *a, uint64_t og_f32, uint64_t ou_f32, int64_t n);

/* y = x + o (k_res_add, src/llama_common.mojo:354-359). */
int q8_res_add(q8_ctx *ctx, q8_buf *a, uint64_t ox_f32, uint64_t oo_f32,
               uint64_t oy_f32, int64_t n);

/* y += x (k_add, src/llama_common.mojo:397-400). */
int q8_add(q8_ctx *ctx, q8_buf *a, uint64_t ox_f32, uint64_t oy_f32, int64_t n);

/* Index of the largest of n f32 at ox, stored as an int32 at element offset
 * oid of ids (k_argmax / argmax_op, src/llama_common.mojo:493-519,783-789):
 * a value must be strictly greater to win (NaN never wins), equal maxima go
 * to the lowest index. */
int q8_argmax(q8_ctx *ctx, q8_buf *a, uint64_t ox_f32, int64_t n, q8_buf *ids,
              uint64_t oid_i32);

/* The int32 position at element offset opos of posbuf += s, on the stream
 * (the device side of n_cached += s, qwen3_mojo/src/qwen_q8.mojo:138). */
int q8_pos_advance(q8_ctx *ctx, q8_buf *posbuf, uint64_t opos_i32, int64_t s);

/* ---- HIP graphs ------------------------------------------------------------ */

/* Capture every call issued on the context's stream between begin and end
 * into a hipGraph, then replay it with q8_graph_launch.  Used to amortise
 * the launch cost of a whole decode step.  *graph is an opaque handle. */
int q8_graph_begin(q8_ctx *ctx);
int q8_graph_end(q8_ctx *ctx, void **graph);
int q8_graph_launch(q8_ctx *ctx, void *graph);
void q8_graph_destroy(void *graph);

/* ---- packed checkpoint files (safetensors) -----------------------------------
 * Host code; no context needed except for q8_st_upload.  Errors return a
 * Q8_ERR_* code with the message in q8_st_error() (per thread). */
typedef struct q8_st q8_st;
typedef struct q8_stw q8_stw;

/* Open a safetensors model: a file, or a directory holding either
 * model.safetensors.index.json (shards in order of first appearance in its
 * weight_map) or model.safetensors.  Every header is parsed and checked
 * (offsets inside the file, bytes = shape x dtype size).
 * Replaces SafeTensors.__init__ (src/safetensors.mojo:36-84). */
int q8_st_open(const char *path, q8_st **out);
void q8_st_close(q8_st *st);
const char *q8_st_error(void);
/* Number of tensors (-1 for a null handle); index of `name` or -1
 * (SafeTensors.num_tensors / has / get, src/safetensors.mojo:86-95). */
int64_t q8_st_count(const q8_st *st);
int64_t q8_st_find(const q8_st *st, const char *name);
/* Tensor i: name, dtype string ("F16", "BF16", ...), rank and shape, shard
 * path, absolute byte offset in that shard and byte count (TensorInfo,
 * src/safetensors.mojo:17-33).  Any output pointer may be null; the
 * strings and shape live until q8_st_close. */
int q8_st_info(const q8_st *st, int64_t i, const char **name, const char **dtype, int *ndim,
               const int64_t **shape, const char **path, uint64_t *begin, uint64_t *nbytes);
/* The first shard's __metadata__ entries, in file order. */
int64_t q8_st_metadata_count(const q8_st *st);
int q8_st_metadata(const q8_st *st, int64_t i, const char **key, const char **value);
/* Bytes [byte_off, byte_off + nbytes) of tensor i into host memory. */
int q8_st_read(const q8_st *st, int64_t i, uint64_t byte_off, void *dst, uint64_t nbytes);
/* Bytes [src_off, src_off + nbytes) of tensor i to byte offset byte_off of
 * a device buffer, through the context's pinned staging (file reads
 * overlap the copies); returns when the bytes are on the device.
 * Replaces the per-tensor read + memcpy of Weights.upload_all
 * (src/resident.mojo:30-58). */
int q8_st_upload(q8_ctx *ctx, const q8_st *st, int64_t i, uint64_t src_off, uint64_t nbytes,
                 q8_buf *buf, uint64_t byte_off);

/* Write a safetensors file laid out as the safetensors library's
 * serializer lays it out (the writer behind quantize.py's save_file,
 * qwen3_mojo/scripts/quantize.py:59-61): tensors sorted by dtype (U64, I64,
 * F64, F32, U32, I32, BF16, F16, U16, I16, F8_E4M3, F8_E5M2, I8, U8, BOOL),
 * then by name; compact JSON, "__metadata__" (given key/value pairs, in the
 * given order) first; header padded with spaces to a multiple of 8.  shapes
 * holds the tensors' dims back to back.  The header is written at open;
 * q8_stw_put writes tensor i (caller's order) in any order; q8_stw_close
 * fails if a tensor was never written. */
int q8_stw_open(const char *path, int64_t count, const char *const *names,
                const char *const *dtypes, const int *ndims, const int64_t *shapes,
                int64_t nmeta, const char *const *meta_keys, const char *const *meta_values,
                q8_stw **out);
int q8_stw_put(q8_stw *w, int64_t i, const void *data, uint64_t nbytes);
int q8_stw_close(q8_stw *w);

#ifdef __cplusplus
}
#endif

#endif /* Q8HIP_H */
