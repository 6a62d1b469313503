// q8_launch.h -- host-side launchers of the gfx950 kernels (internal).
//
// The C ABI (q8hip_api.cpp) validates every argument, resolves buffer
// offsets to device pointers and then calls one of these.  Each launcher
// only picks a kernel variant and a grid; it trusts its arguments.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace q8 {

struct PackArgs {
  const void *src;       // first element of row 0 (bf16 or f32)
  int src_is_f32;
  int64_t n, m;
  uint8_t *dst;          // byte address of packed row 0
  int64_t dst_row_bytes; // packed row stride in bytes
  int G, kind;
};
hipError_t launch_pack(const PackArgs &a, hipStream_t st);

struct LinearArgs {
  const uint8_t *w;      // byte address of packed row 0
  int64_t row_bytes;     // packed row stride in bytes
  const void *x;         // activations [s, m] (f32 or bf16), row stride m
  int x_is_bf16;
  float *y;              // outputs [s, n] f32, row stride n
  int64_t s, m, n;
  int G, kind;
  // Split-K workspace for the GEMM (null: no split): room for ws_floats
  // partial sums.
  float *ws = nullptr;
  int64_t ws_floats = 0;
  // GEMM only, f32 x: with up set, x holds gate rows [s, m], up rows
  // [s, m] sit at up, and the linear reads silu(gate) * up (the values
  // swiglu_kernel stores).
  const float *up = nullptr;
  int64_t ldx = 0;   // GEMM only: row stride of x (and up) in elements; 0: m
  // GEMM only, f32 x, dense rows: with wn set the rows read are
  // rmsnorm(x + res) with bf16 weights wn (res null: rmsnorm(x)), formed as
  // rmsnorm_kernel forms them; with res set, x + res is also stored to hout
  // (which may be x or res itself).
  const uint16_t *wn = nullptr;
  float eps = 0.0f;
  const float *res = nullptr;
  float *hout = nullptr;
};
// Decode path (s small, f32 x): VALU GEMV.
hipError_t launch_gemv(const LinearArgs &a, hipStream_t st);
// One-row GEMV with its neighbours folded in (decode step, s = 1).
// Prologue (how x is read):
//   PRE_RMSNORM: rmsnorm(x) with bf16 weights wn; staged as wn * x, the
//                factor 1 / sqrt(mean(x^2) + eps) applied to each output;
//   PRE_SWIGLU:  x holds [gate | up] (2m floats), read as silu(gate) * up.
// Epilogue (what is stored):
//   POST_RESIDUAL: y = res + W x (res may be y itself);
//   POST_SWIGLU:   rows [0, n/2) are gate rows and [n/2, n) up rows; stores
//                  y[j] = silu(g_j) * u_j for j < n/2.
enum { PRE_NONE = 0, PRE_RMSNORM = 1, PRE_SWIGLU = 2 };
//   POST_ARGMAX:   y stored; each workgroup also writes its largest y and
//                  its row (strict > in row order, so the lowest row among
//                  equal values; NaN never wins) to part[blockIdx] and
//                  ((int *)part)[grid + blockIdx]: the partials that
//                  launch_argmax_finish reduces.
enum { POST_STORE = 0, POST_RESIDUAL = 1, POST_SWIGLU = 2, POST_ARGMAX = 3 };
struct FusedLinearArgs {
  LinearArgs lin;        // s = 1, f32 x, aligned rows
  int pre, post;
  const uint16_t *wn;    // PRE_RMSNORM: m bf16 norm weights
  float eps;
  const float *res;      // POST_RESIDUAL: residual [n]
  float *part = nullptr; // POST_ARGMAX: 2 x kArgmaxMaxBlocks words
  int *grid_out = nullptr;   // POST_ARGMAX: receives the workgroup count
};
constexpr int kArgmaxMaxBlocks = 8192;
// False when the shape cannot take the fused path (x staged in LDS).
bool gemv_fused_supported(const FusedLinearArgs &f);
hipError_t launch_gemv_fused(const FusedLinearArgs &a, hipStream_t st);
// Prefill path, dequant-GEMM on f16 MFMA: x (bf16 or f32) is first written
// as binary16 rows scaled by a power of two to x16 [s, m] with the
// exponents in ex [s]; with f32 scales and `weights` set the same launch
// writes each weight row's scale exponent to ew [n] (a later row chunk of
// the same call passes weights = false and reuses them); then the weights
// are dequantized to binary16 in registers.
hipError_t launch_gemm(const LinearArgs &a, uint16_t *x16, int *ex, int *ew, bool weights,
                       hipStream_t st);
// y[i] = sum over z < splits of ws[z * count + i] (split-K partial sums).
hipError_t launch_splitk_reduce(const float *ws, float *y, int64_t count, int splits,
                                hipStream_t st);
// Small batches (s <= 32, f32 x; the C ABI sends it 5 <= s < 32): bf16 MFMA
// over zero-padded 16-row tiles with x split into two bf16 terms.
hipError_t launch_skinny(const LinearArgs &a, hipStream_t st);
// A few rows (2 <= s <= kSkinny4MaxRows, f32 x): f32 4x4 MFMA blocks over
// 16-code runs, exact f32 products.
constexpr int kSkinny4MaxRows = 4;
hipError_t launch_skinny4(const LinearArgs &a, hipStream_t st);

struct GatherArgs {
  const uint8_t *w;      // byte address of packed row 0 of the table
  int64_t row_bytes;
  const int32_t *ids;
  float *y;
  int64_t s, d, vocab;
  int G, kind;
};
hipError_t launch_embed_gather(const GatherArgs &a, hipStream_t st);

// ---- decode-step layer kernels (q8_layer.hip) ------------------------------
// RMSNorm of `rows` rows of d; with res != null the rows are x + res, also
// stored to h_out.  per > 0: rows in groups of per consecutive rows of d,
// groups ld elements apart (x, res, h_out and y alike); else dense rows.
hipError_t launch_rmsnorm(const uint16_t *wn, const float *x, const float *res, float *h_out,
                          float *y, int64_t rows, int64_t d, float eps, hipStream_t st,
                          int64_t per = 0, int64_t ld = 0);
// RoPE on q [s, nheads*head_dim] (row stride ldq) and k [s, nkv*head_dim]
// (row stride ldk, also v's) in place; rotated k and v go to binary16 cache
// rows pos0 .. pos0+s-1 (pos0 = *posp if posp).
hipError_t launch_rope_kv(float *q, float *k, const float *v, __half *kc, __half *vc,
                          const float *inv, int s, const int *posp, int pos0, int nheads, int nkv,
                          int head_dim, int64_t maxlen, int64_t ldq, int64_t ldk,
                          hipStream_t st);
struct AttnArgs {
  const float *q;        // [s, nheads * head_dim], rotated, row i at q + i * ldq
  const __half *kc, *vc; // [maxlen, nkv * head_dim]
  float *part;           // scratch (s < kPrefillMinRows only):
                         //   s * nheads * nsplit * (head_dim + 2) floats
  float *out;            // [s, nheads * head_dim]
  int s, nheads, nkv, head_dim, nsplit;
  const int *posp;       // device position (or null: pos0)
  int pos0;
  int maxlen;            // cache rows; positions past it are clamped
  int64_t ldq;           // q row stride in floats (nheads * head_dim when dense)
};
// Row counts from which attention runs as one MFMA pass per (row block, KV
// head) with no scratch; below it, as (KV head, 64-key split) partials
// merged by a second kernel.
constexpr int kPrefillMinRows = 16;
// Causal GQA attention of s query rows at positions pos0 .. pos0+s-1 over
// cache rows 0 .. pos0+i; nsplit = ceil(maxlen / 64).
hipError_t launch_attention(const AttnArgs &a, hipStream_t st);
struct DecodeAttnArgs {
  const float *q, *k, *v;  // one new token: q [nheads*hd], k, v [nkv*hd] (unrotated)
  const float *inv;        // head_dim / 2 inverse frequencies
  __half *kc, *vc;         // cache blocks [maxlen, nkv*hd]
  float *out;              // [nheads*hd]
  float *part;             // scratch: nsplit * nheads * (hd + 2) floats
  const uint16_t *qnorm = nullptr, *knorm = nullptr;   // per-head RMSNorm weights (hd bf16)
  float eps = 0.0f;
  int nheads, nkv, head_dim, nsplit;
  const int *posp;         // device position (or null: pos0)
  int pos0, maxlen;
};
// Per-head RMSNorm of q and k (with qnorm / knorm), RoPE of q and k, append
// of k and v at cache row pos0 and attention of the one new token over rows
// 0 .. pos0: one launch of nsplit x nkv blocks over
// context splits, then (nsplit > 1) a merge launch.  Calls that share
// `part` must not overlap.
// Keys per chunk (one wave's unit of work), waves per block, head slots of
// a block and the split count.  Head slots: heads per wave GRP / slots,
// waves per head waves / slots (the chunks a block spans).
//   * 64-dim heads: one head per wave; in groups of 4, 8 waves over two
//     32-key chunks (the 64 keys a block of 4 waves over one 64-key chunk
//     took, each wave's chain halved: Llama-3.2-1B at 1030 tokens 7.02 ->
//     6.99 us per call, at 6000 10.78 -> 10.19 us; step 0.5054-0.5063 ->
//     0.5041-0.5054 ms), else 4 waves over 64-key chunks (8 waves over two
//     64-key chunks lose: 7.17 -> 7.73 us);
//   * 128-dim heads, 32-key chunks: in groups of 8, 4 waves serving 4 heads
//     each, so the K/V rows of a chunk are loaded once and the block's
//     waves work on different chunks (measured on the Llama-3.1-8B step at
//     2300 cached tokens; slower on the 1B step); in groups of 4, 8 waves,
//     two per chunk with 2 heads each, which halves each wave's chain of
//     dot products and softmax work for the same blocks (Llama-3.1-8B at
//     2300 tokens: 9.98 -> 9.75 us per call, the same bits); in groups of
//     2, 8 waves of one head each over 4 chunks instead of 4 waves over 2
//     chunks each, so no wave walks a second chunk (Qwen3-0.6B at 128
//     tokens: 7.29 -> 6.05 us per call, step 0.6525 -> 0.6179 ms).
// Splits: one chunk per wave and head slot (blocks of waves / slots
// chunks) up to 32 blocks per KV head, then more chunks per block.  Every
// launched block reads the position before it can leave and a launch of
// 256 blocks takes about 1.4 us to start them all, so the grid holds no
// more blocks than the longest context keeps busy.  A cache of at most 4
// chunks per wave gets one block per KV head, which writes the output
// itself, and no merge launch (the merge costs more than the chunks:
// Qwen3-0.6B at 128 cached tokens).
constexpr int kDecodeAttnOneBlockChunks = 4;
constexpr int kDecodeAttnMaxSplit = 32;   // bound of the merge's per-thread loads
constexpr int decode_attn_chunk(int head_dim, int grp) {
  return (head_dim > 64 || grp == 4) ? 32 : 64;
}
constexpr int decode_attn_waves(int hd, int grp) {
  return ((hd >= 128 && (grp == 4 || grp == 2)) || (hd == 64 && grp == 4)) ? 8 : 4;
}
constexpr int decode_head_slots(int hd, int grp) {
  return (hd >= 128 && grp == 4) ? 2 : (hd >= 128 && grp > 4) ? grp / 4 : (grp < 4 ? grp : 4);
}
inline int decode_attn_nsplit(int64_t maxlen, int head_dim, int grp) {
  const int64_t kc = decode_attn_chunk(head_dim, grp);
  const int64_t wph = decode_attn_waves(head_dim, grp) / decode_head_slots(head_dim, grp);
  const int64_t n = ((maxlen + kc - 1) / kc + wph - 1) / wph;
  return (int)(n <= kDecodeAttnOneBlockChunks ? 1 : n > 32 ? 32 : n);
}
hipError_t launch_decode_attention(const DecodeAttnArgs &a, hipStream_t st);
hipError_t launch_swiglu(float *g, const float *u, int64_t n, hipStream_t st);
hipError_t launch_res_add(const float *x, const float *o, float *y, int64_t n, hipStream_t st);
hipError_t launch_add(const float *x, float *y, int64_t n, hipStream_t st);
hipError_t launch_argmax(const float *v, int64_t n, int32_t *out, hipStream_t st);
// Reduce the POST_ARGMAX partials of `nblocks` workgroups (the argmax of the
// n logits, as launch_argmax: index 0 when logits[0] is NaN or nothing beats
// it), write it to ids[0], add pos_step to *pos (pos may be null) and, with
// emb non-null, gather that id's embedding row (d floats) into xnext.
struct ArgmaxFinishArgs {
  const float *part;
  int nblocks;
  const float *logits;
  int32_t *ids;
  int *pos;
  int pos_step;
  const uint8_t *emb;    // packed table (vocab rows) or null
  int64_t row_bytes, vocab, d;
  int G, kind;
  float *xnext;
};
hipError_t launch_argmax_finish(const ArgmaxFinishArgs &a, hipStream_t st);
hipError_t launch_pos_advance(int *pos, int s, hipStream_t st);

}  // namespace q8
