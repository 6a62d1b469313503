// q8_layer.hip -- decode-step layer kernels around the Q8 linears (gfx950).
//
// The non-linear parts of one pre-norm GQA transformer block and of the
// token loop, over the same arenas as the Q8 linears: f32 activations
// addressed by float offsets and bf16 norm vectors in the u16 weight arena.
// Reference kernels (src/llama_common.mojo):
//   rmsnorm          k_rmsnorm_w         :197-225
//   add + rmsnorm    k_res_add + k_rmsnorm_w (two dispatches there)
//   rope + KV append k_rope_qk_copy2     :299-342
//   attention        k_scores / k_softmax_rows / k_att_out  :402-473
//   swiglu           k_swiglu_mul        :476-481
//   res_add / add    k_res_add :354-359, k_add :397-400
//   argmax           k_argmax            :493-519
// Deliberate differences from the reference:
//   * the KV cache is binary16 (half the cache bytes per step);
//   * attention is one pass per (KV head, context split) with an online
//     softmax over the group's query heads plus a small combine, instead of
//     a materialised score matrix;
//   * positions can come from a device counter, so one captured HIP graph
//     serves every decode step.
#include <hip/hip_fp16.h>

#include "q8_device.h"
#include "q8_launch.h"

namespace q8 {
namespace {

// cos and sin of a RoPE angle through one sincosf call, so every kernel that
// rotates gets bit-identical values (separate cosf / sinf calls may be
// lowered differently from one kernel to the next).
__device__ __forceinline__ void rope_cs(float freq, float &c, float &sn) {
  sincosf(freq, &sn, &c);
}

// RoPE of one pair, written with explicit FMAs so every kernel that rotates
// (rope_kv_kernel, attn_decode_kernel) rounds identically.  The rotated pair
// is pinned in f32 registers (empty asm): otherwise the compiler may merge
// the last FMA with a later binary16 conversion (v_fma_mix*), rounding once
// to f16 where another kernel rounds to f32 first.
__device__ __forceinline__ void rotate(float x0, float x1, float c, float sn, float &y0, float &y1) {
  float a = __builtin_fmaf(x0, c, -(x1 * sn));
  float b = __builtin_fmaf(x1, c, x0 * sn);
  __asm__ volatile("" : "+v"(a), "+v"(b));
  y0 = a;
  y1 = b;
}

// ---- RMSNorm (k_rmsnorm_w): y = bf16(w) * x * 1/sqrt(mean(x^2) + eps) -------
// One 256-thread block per row.  With res != null the row is h = x + res,
// stored to h_out, and normalised (k_res_add followed by k_rmsnorm_w).
// Rows come in groups of `per` consecutive rows of d, groups `ld` elements
// apart (per = 1, ld = d: dense rows; per heads of a token row at stride
// ld: the per-head norms of q or k inside stacked q|k|v rows, k_rmsnorm2_w).
__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t *__restrict__ wn,
                                                      const float *x, const float *res,
                                                      float *h_out, float *y, int64_t d,
                                                      float eps, int64_t per, int64_t ld) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int64_t base = (row / per) * ld + (row % per) * d;
  const float *xr = x + base;
  const float *rr = res ? res + base : nullptr;
  float ss = 0.0f;
  for (int64_t k = threadIdx.x; k < d; k += 256) {
    float v = xr[k];
    if (rr) {
      v += rr[k];
      h_out[base + k] = v;
    }
    ss = __builtin_fmaf(v, v, ss);
  }
  ss = block_sum256(ss, red);
  const float inv = 1.0f / sqrtf(ss / (float)d + eps);
  const float *src = rr ? h_out + base : xr;
  for (int64_t k = threadIdx.x; k < d; k += 256)
    y[base + k] = bf16_bits_to_f32(wn[k]) * src[k] * inv;
}

// ---- RoPE on q and k + KV append (k_rope_qk_copy2) ----------------------------
// HF rotate_half RoPE in place on q [s, qdim] and k [s, kvdim] (row i of q
// at q + i*ldq, of k and v at + i*ldk); the rotated k and the unrotated v of
// row i are stored as binary16 at cache row pos0 + i (rows past maxlen are
// dropped).  One thread per rotated pair and one per v element.
__global__ __launch_bounds__(256) void rope_kv_kernel(float *q, float *k, const float *v,
                                                      __half *kc, __half *vc,
                                                      const float *inv, int s, const int *posp,
                                                      int pos0_host, int nheads, int nkv,
                                                      int head_dim, int64_t maxlen,
                                                      int64_t ldq, int64_t ldk) {
  const int half = head_dim / 2;
  const int nall = nheads + nkv;
  const int64_t nrope = (int64_t)s * nall * half;
  const int kvdim = nkv * head_dim;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int pos0 = posp ? *posp : pos0_host;
  if (idx < nrope) {
    const int i = (int)(idx / (nall * half));
    const int r = (int)(idx % (nall * half));
    const int h = r / half, d = r % half;
    const float freq = (float)(pos0 + i) * inv[d];
    float c, sn;
    rope_cs(freq, c, sn);
    if (h < nheads) {
      float *base = q + (int64_t)i * ldq + h * head_dim;
      float y0, y1;
      rotate(base[d], base[half + d], c, sn, y0, y1);
      base[d] = y0;
      base[half + d] = y1;
    } else {
      const int hk = h - nheads;
      float *base = k + (int64_t)i * ldk + hk * head_dim;
      float y0, y1;
      rotate(base[d], base[half + d], c, sn, y0, y1);
      base[d] = y0;
      base[half + d] = y1;
      const int64_t row = pos0 + i;
      if (row < maxlen) {
        __half *cb = kc + row * kvdim + hk * head_dim;
        cb[d] = __float2half_rn(y0);
        cb[half + d] = __float2half_rn(y1);
      }
    }
  } else if (idx < nrope + (int64_t)s * kvdim) {
    const int64_t vi = idx - nrope;
    const int64_t i = vi / kvdim;
    const int64_t row = pos0 + i;
    if (row < maxlen) vc[row * kvdim + vi % kvdim] = __float2half_rn(v[i * ldk + vi % kvdim]);
  }
}

// ---- attention, pass 1 (k_scores + k_softmax_rows + k_att_out) ---------------
// Block (g, sp, i): KV head g, context split sp (keys [sp*64, sp*64+64)),
// query row i (position pos0 + i, causal over keys 0 .. pos0 + i).  Wave w
// of the block is query head g*GRP + w; lane j holds key sp*64 + j for the
// scores, then output dims j (and j + 64) for P V.  Writes the split's
// unnormalised output, its max score and its sum of exponentials.
template <int HD, int GRP>
__global__ __launch_bounds__(64 * GRP) void attn_split_kernel(const float *__restrict__ q,
                                                              const __half *__restrict__ kc,
                                                              const __half *__restrict__ vc,
                                                              float *__restrict__ part, int nheads,
                                                              int nkv, const int *posp,
                                                              int pos0_host, int nsplit,
                                                              int maxlen, int64_t ldq) {
  constexpr int KC = 64;                       // keys per split
  constexpr int PW = HD + 2;                   // partial record: o[HD], m, l
  __shared__ float qs[GRP][HD];
  __shared__ float ps[GRP][KC];
  const int g = blockIdx.x, sp = blockIdx.y, i = blockIdx.z;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int h = g * GRP + w;
  const int kvdim = nkv * HD;
  const int pos0 = posp ? *posp : pos0_host;
  const int nctx = pos0 + i + 1 < maxlen ? pos0 + i + 1 : maxlen;   // cache rows that exist
  float *rec = part + (((int64_t)i * nheads + h) * nsplit + sp) * PW;
  const int j0 = sp * KC;
  if (j0 >= nctx) {                            // split past the context: empty
    if (lane == 0) {
      rec[HD] = -INFINITY;
      rec[HD + 1] = 0.0f;
    }
    return;
  }
  for (int d = lane; d < HD; d += 64) qs[w][d] = q[(int64_t)i * ldq + h * HD + d];
  __syncthreads();
  const float rd = sqrtf((float)HD);
  const int j = j0 + lane;
  float sc = -INFINITY;
  if (j < nctx) {
    const __half2 *kr = reinterpret_cast<const __half2 *>(kc + (int64_t)j * kvdim + g * HD);
    float acc = 0.0f;
#pragma unroll 8
    for (int d2 = 0; d2 < HD / 2; ++d2) {
      const float2 kv = __half22float2(kr[d2]);
      acc = __builtin_fmaf(qs[w][2 * d2], kv.x, acc);
      acc = __builtin_fmaf(qs[w][2 * d2 + 1], kv.y, acc);
    }
    sc = acc / rd;
  }
  const float mx = wave_max(sc);
  const float p = j < nctx ? expf(sc - mx) : 0.0f;
  const float l = wave_sum(p);
  ps[w][lane] = p;
  __syncthreads();
  const int nk = nctx - j0 < KC ? nctx - j0 : KC;
#pragma unroll
  for (int d = lane; d < HD; d += 64) {
    float o = 0.0f;
    for (int t = 0; t < nk; ++t)
      o = __builtin_fmaf(ps[w][t], __half2float(vc[(int64_t)(j0 + t) * kvdim + g * HD + d]), o);
    rec[d] = o;
  }
  if (lane == 0) {
    rec[HD] = mx;
    rec[HD + 1] = l;
  }
}

// ---- attention, pass 2: merge the splits of each (row, head) ----------------
template <int HD>
__global__ __launch_bounds__(64) void attn_combine_kernel(const float *__restrict__ part,
                                                          float *__restrict__ out, int nheads,
                                                          const int *posp, int pos0_host,
                                                          int nsplit, int maxlen) {
  constexpr int PW = HD + 2;
  const int h = blockIdx.x, i = blockIdx.y;
  const int pos0 = posp ? *posp : pos0_host;
  const int nctx = pos0 + i + 1 < maxlen ? pos0 + i + 1 : maxlen;
  const int nsp = (nctx + 63) / 64 < nsplit ? (nctx + 63) / 64 : nsplit;
  const float *rec = part + ((int64_t)i * nheads + h) * nsplit * PW;
  float mx = -INFINITY;
  for (int sp = 0; sp < nsp; ++sp) mx = fmaxf(mx, rec[sp * PW + HD]);
  float l = 0.0f;
  float o[HD / 64];
#pragma unroll
  for (int e = 0; e < HD / 64; ++e) o[e] = 0.0f;
  for (int sp = 0; sp < nsp; ++sp) {
    const float f = expf(rec[sp * PW + HD] - mx);
    l = __builtin_fmaf(rec[sp * PW + HD + 1], f, l);
#pragma unroll
    for (int e = 0; e < HD / 64; ++e) o[e] = __builtin_fmaf(rec[sp * PW + threadIdx.x + 64 * e], f, o[e]);
  }
  const float il = 1.0f / l;
#pragma unroll
  for (int e = 0; e < HD / 64; ++e)
    out[(int64_t)i * nheads * HD + h * HD + threadIdx.x + 64 * e] = o[e] * il;
}

// ---- multi-row causal attention on the matrix cores (prompt rows) -----------
// One block of 4 waves serves one KV head and PB = 4 * (32 / GRP) consecutive
// query rows, grid (nkv, row blocks) with the last rows' blocks first: a
// block's key tiles grow with its rows, and blocks are dispatched in index
// order, so the longest ones start first and the short ones fill in behind
// them (row blocks in order left the longest for the end: 2048 rows, 128-dim
// heads 32 / 8, 202 -> 127 us).  Each wave owns 32 columns, a column being one (row, query head)
// pair of the group.  Per tile of 64 keys the block stages K row-major and V
// transposed in LDS, and each wave forms S^T = K Q^T and O^T += V^T P^T with
// v_mfma_f32_32x32x16_f16 and an online softmax over its columns.
// The f32 operands enter as binary16 hi + lo pairs: q scaled per column by a
// power of two (largest |q| in [2^14, 2^15), so lo keeps its bits), p by
// 2^14; K and V are binary16 already, so the products are exact and scores
// and sums carry f32-level error.  Scores are kept in the log2 domain
// (scaled by log2(e) / sqrt(head_dim)), so the softmax uses exp2.
// Lane layout of the 32x32x16 MFMA (lane l, h = l / 32): A element i is
// A[l % 32][8h + i], B element i is B[8h + i][l % 32], and accumulator
// element v is D[8(v / 4) + 4h + v % 4][l % 32].  The keys of a P^T column
// held by a lane follow the accumulator layout, so V^T stores each 16-key
// chunk permuted (key 8a + 4h + b at 8h + 4a + b) to make one lane's eight
// keys of an MFMA step contiguous.
typedef _Float16 half8 __attribute__((ext_vector_type(8)));

constexpr int kPrefillBK = 64;   // keys per staged tile

__device__ __forceinline__ void split_f16(float a, _Float16 &hi, _Float16 &lo) {
  hi = (_Float16)a;
  lo = (_Float16)(a - (float)hi);
}

// Two waves per SIMD (two blocks per CU): at most 256 registers per wave, so
// the accumulators stay in VGPRs (no AGPR copies around the rescale) and one
// block's MFMAs run beside the other's softmax (2048 rows, 128-dim heads
// 32 / 8: 126 -> 113 us; one block per CU took 328 registers).
template <int HD, int GRP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void attn_prefill_kernel(const float *__restrict__ q,
                                                           const __half *__restrict__ kc,
                                                           const __half *__restrict__ vc,
                                                           float *__restrict__ out, int s,
                                                           int nheads, int nkv, const int *posp,
                                                           int pos0_host, int maxlen,
                                                           int64_t ldq) {
  constexpr int BK = kPrefillBK;
  constexpr int KS = HD / 16;                    // 16-dim steps of a score tile
  constexpr int DT = HD / 32;                    // 32-dim tiles of the output
  constexpr int PW = 32 / GRP;                   // query rows per wave
  constexpr int PB = 4 * PW;                     // query rows per block
  constexpr int KST = HD + 8;                    // K row stride in LDS (halves)
  constexpr int VST = BK + 8;                    // V^T row stride in LDS (halves)
  constexpr int KCH = BK * (HD / 8) / 256;       // 16-byte K chunks per thread
  constexpr int VCH = (BK / 2) * (HD / 8) / 256; // V key pairs x 8 dims per thread
  static_assert(KCH >= 1 && VCH >= 1, "tile too small for 256 threads");
  __shared__ __attribute__((aligned(16))) _Float16 ks[BK * KST];
  __shared__ __attribute__((aligned(16))) _Float16 vt[HD * VST];

  const int g = blockIdx.x;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int col = lane & 31, hf = lane >> 5;
  const int pos0 = posp ? *posp : pos0_host;
  const int qdim = nheads * HD, kvdim = nkv * HD;
  const int row0 = ((int)gridDim.y - 1 - (int)blockIdx.y) * PB;   // longest rows first
  const int nkeys = min(pos0 + min(row0 + PB, s), maxlen);   // keys any row of the block sees
  const int ntiles = nkeys > 0 ? (nkeys + BK - 1) / BK : 0;
  const int wend = min(pos0 + min(row0 + w * PW + PW, s), maxlen);   // ... any row of the wave
  const int wfull = min(pos0 + min(row0 + w * PW, s - 1) + 1, maxlen);  // ... every row of it
  const int i = row0 + w * PW + col / GRP;       // this lane's column: row i, head
  const int head = g * GRP + col % GRP;
  const int irow = min(i, s - 1);
  const int kend = min(pos0 + irow + 1, maxlen); // keys 0 .. kend-1 are visible to it

  // q of the column: dims 16ks + 8h + 0..7, scaled by 2^e, split hi + lo
  half8 qh[KS], ql[KS];
  float cs;
  {
    const float *qr = q + (int64_t)irow * ldq + head * HD + 8 * hf;
    f32x4 qv[KS][2];
    float mx = 0.0f;
#pragma unroll
    for (int k = 0; k < KS; ++k) {
      qv[k][0] = *reinterpret_cast<const f32x4 *>(qr + 16 * k);
      qv[k][1] = *reinterpret_cast<const f32x4 *>(qr + 16 * k + 4);
#pragma unroll
      for (int c = 0; c < 4; ++c) mx = fmaxf(mx, fmaxf(fabsf(qv[k][0][c]), fabsf(qv[k][1][c])));
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const int ex = (int)((__builtin_bit_cast(uint32_t, mx) >> 23) & 255u) - 127;
    const int e = min(max(14 - ex, -126), 126);
    const float qsc = __builtin_ldexpf(1.0f, e);
    cs = __builtin_ldexpf(1.44269504088896341f / sqrtf((float)HD), -e);
#pragma unroll
    for (int k = 0; k < KS; ++k)
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        _Float16 hi, lo;
        split_f16(qv[k][c >> 2][c & 3] * qsc, hi, lo);
        qh[k][c] = hi;
        ql[k][c] = lo;
      }
  }

  // staging: registers hold the next tile while the current one is used
  u32x4 kreg[KCH], vreg[VCH][2];
  auto load_tile = [&](int kt) {
    const int k0 = kt * BK;
    const int nk = min(BK, nkeys - k0);
    // keys k0 .. k0+nk-1 of this KV head; chunks of keys past them read as zero
    const uint32_t nbytes = (uint32_t)(((int64_t)(nk - 1) * kvdim + HD) * 2);
    const rsrc_t rk = make_rsrc(kc + (int64_t)k0 * kvdim + g * HD, nbytes);
    const rsrc_t rv = make_rsrc(vc + (int64_t)k0 * kvdim + g * HD, nbytes);
#pragma unroll
    for (int u = 0; u < KCH; ++u) {
      const int c = threadIdx.x + 256 * u;
      const int key = c / (HD / 8), dg = c % (HD / 8);
      kreg[u] = bload16(rk, (uint32_t)((key * kvdim + dg * 8) * 2));
    }
#pragma unroll
    for (int u = 0; u < VCH; ++u) {
      const int c = threadIdx.x + 256 * u;
      const int kp = c % (BK / 2), dg = c / (BK / 2);
      const uint32_t off = (uint32_t)((2 * kp * kvdim + dg * 8) * 2);
      vreg[u][0] = bload16(rv, off);
      vreg[u][1] = bload16(rv, off + (uint32_t)(kvdim * 2));
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int u = 0; u < KCH; ++u) {
      const int c = threadIdx.x + 256 * u;
      const int key = c / (HD / 8), dg = c % (HD / 8);
      *reinterpret_cast<u32x4 *>(&ks[key * KST + dg * 8]) = kreg[u];
    }
#pragma unroll
    for (int u = 0; u < VCH; ++u) {
      const int c = threadIdx.x + 256 * u;
      const int kp = c % (BK / 2), dg = c / (BK / 2);
      const int key = 2 * kp, r = key & 15;
      const int at = (key & ~15) + 8 * ((r >> 2) & 1) + 4 * (r >> 3) + (r & 3);
#pragma unroll
      for (int d2 = 0; d2 < 4; ++d2) {
        // dims 8dg + 2d2 and +1: (key, key + 1) pairs as one 32-bit word each
        const uint32_t a = vreg[u][0][d2], b = vreg[u][1][d2];
        *reinterpret_cast<uint32_t *>(&vt[(dg * 8 + 2 * d2) * VST + at]) =
            __builtin_amdgcn_perm(b, a, 0x05040100u);
        *reinterpret_cast<uint32_t *>(&vt[(dg * 8 + 2 * d2 + 1) * VST + at]) =
            __builtin_amdgcn_perm(b, a, 0x07060302u);
      }
    }
  };

  f32x16 o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int v = 0; v < 16; ++v) o[t][v] = 0.0f;
  float m = -INFINITY, l = 0.0f;
  if (ntiles > 0) load_tile(0);
  for (int kt = 0; kt < ntiles; ++kt) {
    __syncthreads();                             // every wave is done with the last tile
    store_tile();
    __syncthreads();
    if (kt + 1 < ntiles) load_tile(kt + 1);
    const int k0 = kt * BK;
    if (k0 >= wend) continue;                    // past every row of this wave
    f32x16 sc[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int v = 0; v < 16; ++v) sc[t][v] = 0.0f;
#pragma unroll
      for (int k = 0; k < KS; ++k) {
        const half8 a = *reinterpret_cast<const half8 *>(&ks[(32 * t + col) * KST + 16 * k + 8 * hf]);
        sc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qh[k], sc[t], 0, 0, 0);
        sc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, ql[k], sc[t], 0, 0, 0);
      }
    }
    // online softmax of the column over this tile (the other 32 keys of the
    // tile live in lane l ^ 32); a tile every row of the wave sees whole
    // needs no causal mask
    float tmax = -INFINITY;
    if (k0 + BK <= wfull) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float x = sc[t][v] * cs;
          sc[t][v] = x;
          tmax = fmaxf(tmax, x);
        }
    } else {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int key = k0 + 32 * t + 8 * (v >> 2) + 4 * hf + (v & 3);
          const float x = key < kend ? sc[t][v] * cs : -INFINITY;
          sc[t][v] = x;
          tmax = fmaxf(tmax, x);
        }
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
    const float mn = fmaxf(m, tmax);             // finite: key 0 is visible to every column
    const float alpha = exp2f(m - mn);
    m = mn;
    float ps = 0.0f;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float p = exp2f(sc[t][v] - mn);
        sc[t][v] = p;
        ps += p;
      }
    l = __builtin_fmaf(l, alpha, ps);
    // alpha is exactly 1 where the column's maximum did not move: the
    // rescale is skipped when that holds for the whole wave (same bits)
    if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
      for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[t][v] *= alpha;
    }
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        half8 bh, bl;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          _Float16 hi, lo;
          split_f16(sc[t][8 * j + c] * 16384.0f, hi, lo);
          bh[c] = hi;
          bl[c] = lo;
        }
#pragma unroll
        for (int d = 0; d < DT; ++d) {
          const half8 a =
              *reinterpret_cast<const half8 *>(&vt[(32 * d + col) * VST + 32 * t + 16 * j + 8 * hf]);
          o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bh, o[d], 0, 0, 0);
          o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bl, o[d], 0, 0, 0);
        }
      }
  }
  l += __shfl_xor(l, 32);
  if (i < s) {
    const float il = 1.0f / (l * 16384.0f);
    float *orow = out + (int64_t)i * qdim + head * HD + 4 * hf;
#pragma unroll
    for (int d = 0; d < DT; ++d)
#pragma unroll
      for (int vb = 0; vb < 4; ++vb) {
        f32x4 r;
#pragma unroll
        for (int c = 0; c < 4; ++c) r[c] = o[d][4 * vb + c] * il;
        *reinterpret_cast<f32x4 *>(orow + 32 * d + 8 * vb) = r;
      }
  }
}

// ---- decode attention: RoPE + KV append + attention of one new token --------
// (chunk, head slots and split count: decode_attn_chunk, decode_head_slots
// and decode_attn_nsplit; the merge kernel derives the active splits from
// the same values)

// Sum over aligned groups of N consecutive lanes (N = 8 or 16), in every lane.
template <int N>
__device__ __forceinline__ float lane_group_sum(float v) {
  v += dpp_mov<0xb1>(v);                    // quad_perm [1,0,3,2]
  v += dpp_mov<0x4e>(v);                    // quad_perm [2,3,0,1]
  v += dpp_mov<0x141>(v);                   // row_half_mirror
  if constexpr (N == 16) v += dpp_mov<0x140>(v);   // row_mirror
  return v;
}

// Grid (nkv, nsplit), NW = decode_attn_waves(HD, GRP) waves.  Block
// (g, split) serves KV head g and its GRP query heads over the key chunks
// [split * cpb, (split + 1) * cpb) of KC = decode_attn_chunk(HD, GRP) keys,
// cpb = max(waves per head, ceil(chunks / nsplit)).  The waves form
// decode_head_slots(HD, GRP) head slots: wave w serves the GRP / slots query
// heads of slot w % slots over chunk w / slots of the block's chunks (then
// every NW / slots-th after it), so the block's waves share each chunk's K
// and V rows through the cache.  Rows are read as
// 16-byte pieces, HD/8 lanes per row (full 128- or 256-byte runs): a lane
// multiplies its 8 dims of a key by the query and the row's lanes sum with
// DPP; for P V a lane accumulates its 8 dims over its rows.  Online softmax
// per wave; the block merges its waves (and their row slots) in LDS.  With
// one active block per KV head the block writes the output; otherwise it
// writes one partial record (o[HD], m, l) per head and attn_merge_kernel,
// the next launch, merges the records.
//
// Every block rotates q and the new k itself and takes cache row pos0 from
// LDS (rounded to binary16 exactly as cached); split 0 writes the new k and
// v to cache row pos0, and no block reads that row from memory.  Every
// global load of the prologue (q, k, v, frequencies, norm weights) and the
// first chunk's loads are issued before the position is read, so the
// prologue waits for one round trip, not one per dependent load.
template <int HD, int GRP>
__global__ __launch_bounds__(64 * decode_attn_waves(HD, GRP)) void attn_decode_kernel(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
    const float *__restrict__ inv, __half *__restrict__ kc, __half *__restrict__ vc,
    float *__restrict__ part, float *__restrict__ out, int nkv, const int *posp, int pos0_host,
    int maxlen, const uint16_t *__restrict__ qnw, const uint16_t *__restrict__ knw, float eps) {
  constexpr int KC = decode_attn_chunk(HD, GRP), NW = decode_attn_waves(HD, GRP), NT = 64 * NW;
  constexpr int LPR = HD / 8;           // lanes per row (8 dims each)
  constexpr int RPI = 64 / LPR;         // rows per load instruction (row slots)
  constexpr int NI = KC / RPI;          // load instructions per chunk
  constexpr int half = HD / 2;
  constexpr int PR = HD + 2;            // partial record per head: o[HD], m, l
  constexpr int HS = decode_head_slots(HD, GRP);   // head slots per block
  constexpr int HPW = GRP / HS;             // heads per wave
  constexpr int WPH = NW / HS;              // waves per head
  __shared__ float qs[GRP][HD];
  __shared__ __align__(16) __half kn[HD], vn[HD];
  __shared__ float ps[NW][HPW][64];
  __shared__ float wm[NW][HPW], wl[NW][HPW];
  __shared__ __align__(16) float wo[NW][HPW][RPI][HD];
  __shared__ float hinv[GRP + 1];
  // grid (nkv, nsplit): workgroups go to the 8 XCDs in turn, so with nkv a
  // multiple of 8 every split of KV head g runs on one XCD, where
  // attn_merge_kernel's blocks for g's query heads read the records
  const int split = blockIdx.y, g = blockIdx.x, nsplit = gridDim.y;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int hs = w % HS, kg = w / HS;
  const int kvdim = nkv * HD;
  const int rl = lane / LPR;            // row slot within an instruction's rows
  const int dd = (lane % LPR) * 8;      // this lane's 8 dims
  const uint32_t cache_bytes = (uint32_t)maxlen * (uint32_t)kvdim * 2u;
  const rsrc_t krs = make_rsrc(kc, cache_bytes), vrs = make_rsrc(vc, cache_bytes);
  // 8 binary16 values of row r at this lane's dims; rows past maxlen read as
  // zeros (offset out of range)
  auto row_off = [&](int r) -> uint32_t {
    return r < maxlen ? ((uint32_t)r * (uint32_t)kvdim + (uint32_t)(g * HD + dd)) * 2u
                      : kOutOfRange;
  };
  u32x4 kr[NI], vr[NI];
  auto load_chunk = [&](int cc, bool with_v) {
#pragma unroll
    for (int u = 0; u < NI; ++u) kr[u] = bload16(krs, row_off(cc * KC + u * RPI + rl));
    if (with_v) {
#pragma unroll
      for (int u = 0; u < NI; ++u) vr[u] = bload16(vrs, row_off(cc * KC + u * RPI + rl));
    }
  };
  // Prologue inputs, all issued ahead of the first chunk so that one wait
  // covers them: thread t's query pairs (d, half + d) of RoPE items
  // t + NT r, the new k pair (t < half) and v element (t < HD), the inverse
  // frequencies, the norm weights (zeros when absent) and the two halves of
  // the rows whose squares this wave sums for the per-head norms.
  constexpr int NQ = (GRP * half + NT - 1) / NT;   // RoPE items per thread
  constexpr int NR = (GRP + 1 + NW - 1) / NW;    // norm rows per wave
  const int t = threadIdx.x;
  const rsrc_t qrs = make_rsrc(q + (int64_t)g * GRP * HD, GRP * HD * 4);
  const rsrc_t knrs = make_rsrc(k + (int64_t)g * HD, HD * 4);
  const rsrc_t vnrs = make_rsrc(v + (int64_t)g * HD, HD * 4);
  const rsrc_t irs = make_rsrc(inv, half * 4);
  const rsrc_t qwrs = make_rsrc(qnw, qnw ? HD * 2 : 0), kwrs = make_rsrc(knw, knw ? HD * 2 : 0);
  float qa[NQ], qb[NQ], fq[NQ];
  uint32_t wqa[NQ], wqb[NQ];
#pragma unroll
  for (int r = 0; r < NQ; ++r) {
    const int idx = t + NT * r, hh = idx / half, d = idx % half;
    const bool ok = idx < GRP * half;
    qa[r] = bload4f(qrs, ok ? (uint32_t)(hh * HD + d) * 4u : kOutOfRange);
    qb[r] = bload4f(qrs, ok ? (uint32_t)(hh * HD + half + d) * 4u : kOutOfRange);
    fq[r] = bload4f(irs, (uint32_t)d * 4u);
    wqa[r] = bload2(qwrs, (uint32_t)d * 2u);
    wqb[r] = bload2(qwrs, (uint32_t)(half + d) * 2u);
  }
  const float ka = bload4f(knrs, t < half ? (uint32_t)t * 4u : kOutOfRange);
  const float kb = bload4f(knrs, t < half ? (uint32_t)(half + t) * 4u : kOutOfRange);
  const uint32_t wka = bload2(kwrs, t < half ? (uint32_t)t * 2u : kOutOfRange);
  const uint32_t wkb = bload2(kwrs, t < half ? (uint32_t)(half + t) * 2u : kOutOfRange);
  const float vv = bload4f(vnrs, t < HD ? (uint32_t)t * 4u : kOutOfRange);
  float na[NR], nb[NR];
#pragma unroll
  for (int x = 0; x < NR; ++x) {
    const int r = w + NW * x;          // q rows 0 .. GRP-1, then the k row
    const uint32_t o0 = (uint32_t)lane * 4u, o1 = (uint32_t)(64 + lane) * 4u;
    const float q0 = bload4f(qrs, r < GRP ? (uint32_t)(r * HD) * 4u + o0 : kOutOfRange);
    const float k0 = bload4f(knrs, r == GRP ? o0 : kOutOfRange);
    na[x] = r < GRP ? q0 : k0;
    nb[x] = 0.0f;
    if constexpr (HD == 128) {
      const float q1 = bload4f(qrs, r < GRP ? (uint32_t)(r * HD) * 4u + o1 : kOutOfRange);
      const float k1 = bload4f(knrs, r == GRP ? o1 : kOutOfRange);
      nb[x] = r < GRP ? q1 : k1;
    }
  }
  // The first chunk is loaded before the position is known, on the guess
  // that the block spans WPH chunks (true while chunks <= nsplit * WPH).
  const int c_guess = split * WPH + kg;
  load_chunk(c_guess, true);

  const int pos0 = posp ? *posp : pos0_host;
  const bool room = pos0 < maxlen;
  const int nctx = room ? pos0 + 1 : maxlen;
  const int chunks = (nctx + KC - 1) / KC;
  const int cpb = max(WPH, (chunks + nsplit - 1) / nsplit);
  const int active = (chunks + cpb - 1) / cpb;
  if (split >= active) return;
  const int c_end = min((split + 1) * cpb, chunks);
  int c = split * cpb + kg;
  if (c != c_guess && c < c_end) load_chunk(c, true);
  // row r as read, with rows past the context zeroed and row pos0 replaced
  // by this lane's 8 dims of the new row (selects, no branch)
  auto fix_row = [&](u32x4 raw, u32x4 fresh, int r) -> u32x4 {
    const bool keep = r < nctx, mine = r == pos0;
    u32x4 o;
    o.x = mine ? fresh.x : keep ? raw.x : 0u;
    o.y = mine ? fresh.y : keep ? raw.y : 0u;
    o.z = mine ? fresh.z : keep ? raw.z : 0u;
    o.w = mine ? fresh.w : keep ? raw.w : 0u;
    return o;
  };

  // per-head RMSNorm factors of q and the new k when norm weights are given
  // (k_rmsnorm2_w: one wave per row, the row's two 64-element halves summed
  // as block_sum256 sums them in q8_rmsnorm, so the normalised values are
  // the same bits), then RoPE of the group's query heads and the new k;
  // round k, v
  if (qnw || knw) {
#pragma unroll
    for (int x = 0; x < NR; ++x) {
      const int r = w + NW * x;
      if (r < GRP + 1) {
        float ss = wave_sum(na[x] * na[x]);
        if constexpr (HD == 128) ss = ss + wave_sum(nb[x] * nb[x]);
        if (lane == 0) hinv[r] = 1.0f / sqrtf(ss / (float)HD + eps);
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int r = 0; r < NQ; ++r) {
    const int idx = t + NT * r, hh = idx / half, d = idx % half;
    if (idx < GRP * half) {
      float cs, sn;
      rope_cs((float)pos0 * fq[r], cs, sn);
      const float x0 = qnw ? bf16_bits_to_f32(wqa[r]) * qa[r] * hinv[hh] : qa[r];
      const float x1 = qnw ? bf16_bits_to_f32(wqb[r]) * qb[r] * hinv[hh] : qb[r];
      rotate(x0, x1, cs, sn, qs[hh][d], qs[hh][half + d]);
    }
  }
  if (t < half) {                      // inv[t] is fq[0] here (item t < half)
    float cs, sn, r0, r1;
    rope_cs((float)pos0 * fq[0], cs, sn);
    const float x0 = knw ? bf16_bits_to_f32(wka) * ka * hinv[GRP] : ka;
    const float x1 = knw ? bf16_bits_to_f32(wkb) * kb * hinv[GRP] : kb;
    rotate(x0, x1, cs, sn, r0, r1);
    const __half y0 = __float2half_rn(r0), y1 = __float2half_rn(r1);
    kn[t] = y0;
    kn[half + t] = y1;
    if (room && split == 0) {
      kc[(int64_t)pos0 * kvdim + g * HD + t] = y0;
      kc[(int64_t)pos0 * kvdim + g * HD + half + t] = y1;
    }
  }
  if (t < HD) {
    const __half y = __float2half_rn(vv);
    vn[t] = y;
    if (room && split == 0) vc[(int64_t)pos0 * kvdim + g * HD + t] = y;
  }
  __syncthreads();

  const float rd = sqrtf((float)HD);
  const u32x4 kfresh = *reinterpret_cast<const u32x4 *>(kn + dd);
  const u32x4 vfresh = *reinterpret_cast<const u32x4 *>(vn + dd);
  float qv[HPW][8];
#pragma unroll
  for (int j = 0; j < HPW; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) qv[j][i] = qs[hs + HS * j][dd + i];
  float m_run[HPW], l_run[HPW], o_run[HPW][8];
#pragma unroll
  for (int j = 0; j < HPW; ++j) {
    m_run[j] = -INFINITY;
    l_run[j] = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) o_run[j][i] = 0.0f;
  }

  for (; c < c_end; c += WPH) {
    const int j0 = c * KC;
    // scores of the chunk's rows
#pragma unroll
    for (int u = 0; u < NI; ++u) {
      const u32x4 kw = fix_row(kr[u], kfresh, j0 + u * RPI + rl);
      const uint32_t rw[4] = {kw.x, kw.y, kw.z, kw.w};
#pragma unroll
      for (int j = 0; j < HPW; ++j) {
        float dot = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float2 kf = __half22float2(__builtin_bit_cast(__half2, rw[i]));
          dot = __builtin_fmaf(qv[j][2 * i], kf.x, dot);
          dot = __builtin_fmaf(qv[j][2 * i + 1], kf.y, dot);
        }
        // every lane of the row holds the same sum: all store it (one
        // address per row); the scale is applied below, one key per lane
        ps[w][j][u * RPI + rl] = lane_group_sum<LPR>(dot);
      }
    }
    const int cn = c + WPH;             // this wave's next chunk
    if (cn < c_end) load_chunk(cn, false);
    __builtin_amdgcn_wave_barrier();
    // softmax pieces: lane i < KC holds key j0 + i
    const bool key_ok = lane < KC && j0 + lane < nctx;
    float pnew[HPW], fa[HPW];
#pragma unroll
    for (int j = 0; j < HPW; ++j) {
      const float sc = key_ok ? ps[w][j][lane] / rd : -INFINITY;
      const float mx = wave_max(sc);
      const float p = key_ok ? expf(sc - mx) : 0.0f;
      const float l = wave_sum(p);
      const float mn = fmaxf(m_run[j], mx);
      fa[j] = expf(m_run[j] - mn);
      const float fb = expf(mx - mn);
      l_run[j] = __builtin_fmaf(l_run[j], fa[j], l * fb);
      m_run[j] = mn;
      pnew[j] = p * fb;
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int j = 0; j < HPW; ++j) ps[w][j][lane] = pnew[j];
    __builtin_amdgcn_wave_barrier();
    // P V: this lane's 8 dims over its rows of the chunk
#pragma unroll
    for (int j = 0; j < HPW; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) o_run[j][i] *= fa[j];
#pragma unroll
    for (int u = 0; u < NI; ++u) {
      const u32x4 vw = fix_row(vr[u], vfresh, j0 + u * RPI + rl);
      const uint32_t rw[4] = {vw.x, vw.y, vw.z, vw.w};
#pragma unroll
      for (int j = 0; j < HPW; ++j) {
        const float p = ps[w][j][u * RPI + rl];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float2 vf = __half22float2(__builtin_bit_cast(__half2, rw[i]));
          o_run[j][2 * i] = __builtin_fmaf(p, vf.x, o_run[j][2 * i]);
          o_run[j][2 * i + 1] = __builtin_fmaf(p, vf.y, o_run[j][2 * i + 1]);
        }
      }
    }
    if (cn < c_end) {
#pragma unroll
      for (int u = 0; u < NI; ++u) vr[u] = bload16(vrs, row_off(cn * KC + u * RPI + rl));
    }
    __builtin_amdgcn_wave_barrier();
  }
  // per wave: row-slot partial sums of o, and m, l (l = 0: no keys)
#pragma unroll
  for (int j = 0; j < HPW; ++j) {
    float4 *dst = reinterpret_cast<float4 *>(&wo[w][j][rl][dd]);
    dst[0] = make_float4(o_run[j][0], o_run[j][1], o_run[j][2], o_run[j][3]);
    dst[1] = make_float4(o_run[j][4], o_run[j][5], o_run[j][6], o_run[j][7]);
  }
  if (lane == 0) {
#pragma unroll
    for (int j = 0; j < HPW; ++j) {
      wm[w][j] = m_run[j];
      wl[w][j] = l_run[j];
    }
  }
  __syncthreads();
  // per head: the largest running max M of its waves and each wave's factor
  // exp(m_w - M) (0 for a wave without keys), one thread per (head, wave)
  __shared__ float wf[NW][HPW], hm[GRP];
  if (threadIdx.x < GRP * WPH) {
    const int hh = threadIdx.x / WPH, x0 = threadIdx.x % WPH;
    const int s0 = hh % HS, j = hh / HS;       // waves s0 + HS * x serve head hh
    float mx = -INFINITY;
#pragma unroll
    for (int x = 0; x < WPH; ++x) mx = fmaxf(mx, wm[s0 + HS * x][j]);
    const int wx = s0 + HS * x0;
    wf[wx][j] = wl[wx][j] != 0.0f ? expf(wm[wx][j] - mx) : 0.0f;
    if (x0 == 0) hm[hh] = mx;
  }
  __syncthreads();
  // the block's waves of each head -> one record per head: o = sum_w f_w o_w
  // and l = sum_w l_w f_w in wave order (a wave without keys adds l_w = 0
  // times f_w = 0, and its o_w is 0)
  float *rec = part + ((int64_t)g * nsplit + split) * (GRP * PR);
  for (int t = threadIdx.x; t < GRP * HD; t += NT) {
    const int hh = t / HD, d = t % HD;
    const int s0 = hh % HS, j = hh / HS;
    float o = 0.0f, l = 0.0f;
#pragma unroll
    for (int x = 0; x < WPH; ++x) {
      const int wx = s0 + HS * x;
      float os = 0.0f;
#pragma unroll
      for (int r = 0; r < RPI; ++r) os += wo[wx][j][r][d];
      o = __builtin_fmaf(os, wf[wx][j], o);
      l = __builtin_fmaf(wl[wx][j], wf[wx][j], l);
    }
    if (active == 1) {
      out[(g * GRP + hh) * HD + d] = o / l;
    } else {                             // merged by attn_merge_kernel
      rec[hh * PR + d] = o;
      if (d == 0) {
        rec[hh * PR + HD] = hm[hh];
        rec[hh * PR + HD + 1] = l;
      }
    }
  }
}

// Merge of the partial records of attn_decode_kernel: one block (HD threads)
// per head h, thread d its output dim d.  Every load is issued before
// the position is read: lane x takes split x's m and l, thread d split x's
// o[d] for every split (offsets past the records read as zeros).  Each wave
// then forms the active splits' factors exp(m_x - M) and l = sum_x l_x f_x
// itself (wave reductions, no LDS, no barrier), and thread d forms
// o[d] = sum_x f_x o_x[d] / l with f_x read from lane x.  Does nothing when
// one block per KV head was active (it wrote the output itself).
template <int HD, int GRP>
__global__ __launch_bounds__(HD) void attn_merge_kernel(const float *__restrict__ part,
                                                        float *__restrict__ out, int nsplit,
                                                        const int *posp, int pos0_host,
                                                        int maxlen) {
  constexpr int KC = decode_attn_chunk(HD, GRP), NW = decode_attn_waves(HD, GRP);
  constexpr int PR = HD + 2;
  constexpr int WPH = NW / decode_head_slots(HD, GRP);   // as attn_decode_kernel
  constexpr int NX = kDecodeAttnMaxSplit;
  static_assert(NX <= 64, "one lane per split");
  // block b serves head h = (b % nkv) GRP + b / nkv: with nkv a multiple of
  // 8 it runs on the XCD of the split blocks that wrote KV head h / GRP's
  // records, so they are read from that XCD's L2
  const int nkvb = (int)gridDim.x / GRP;
  const int h = ((int)blockIdx.x % nkvb) * GRP + (int)blockIdx.x / nkvb;
  const int g = h / GRP, hh = h % GRP;
  const int d = threadIdx.x, lane = threadIdx.x & 63;
  const rsrc_t prs = make_rsrc(part + (int64_t)g * nsplit * (GRP * PR),
                               (uint32_t)(nsplit * GRP * PR) * 4u);
  auto off = [&](int x, int e) -> uint32_t {
    return x < nsplit ? (uint32_t)(x * GRP * PR + hh * PR + e) * 4u : kOutOfRange;
  };
  const float m_lane = bload4f(prs, off(lane, HD));
  const float l_lane = bload4f(prs, off(lane, HD + 1));
  float ov[NX];
#pragma unroll
  for (int x = 0; x < NX; ++x) ov[x] = bload4f(prs, off(x, d));
  const int pos0 = posp ? *posp : pos0_host;
  const int nctx = pos0 < maxlen ? pos0 + 1 : maxlen;
  const int chunks = (nctx + KC - 1) / KC;
  const int cpb = max(WPH, (chunks + nsplit - 1) / nsplit);
  const int active = (chunks + cpb - 1) / cpb;
  if (active <= 1) return;
  const float mx = lane < active ? m_lane : -INFINITY;
  const float big = wave_max(mx);
  const float f = lane < active ? expf(mx - big) : 0.0f;
  const float l = wave_sum(lane < active ? l_lane * f : 0.0f);
  float o = 0.0f;
  for (int x = 0; x < active; ++x) {     // ov[x]: indexed register reads
    const float fx = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, f), x));
    o = __builtin_fmaf(ov[x], fx, o);
  }
  out[h * HD + d] = o / l;
}

// ---- elementwise (k_swiglu_mul, k_res_add, k_add) ----------------------------
__global__ __launch_bounds__(256) void swiglu_kernel(float *g, const float *u, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    const float v = g[i];
    g[i] = (v / (1.0f + expf(-v))) * u[i];
  }
}

__global__ __launch_bounds__(256) void res_add_kernel(const float *x, const float *o, float *y,
                                                      int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = x[i] + o[i];
}

__global__ __launch_bounds__(256) void add_kernel(const float *x, float *y, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] += x[i];
}

// ---- argmax (k_argmax) --------------------------------------------------------
// One 1024-thread block.  A value wins only if strictly greater (so a NaN
// never wins, and v[0] is the starting best as in the reference); among
// equal maxima the lowest index wins.
__global__ __launch_bounds__(1024) void argmax_kernel(const float *__restrict__ v, int64_t n,
                                                      int32_t *__restrict__ out) {
  __shared__ float bv[16];
  __shared__ int32_t bi[16];
  float best = v[0];
  int32_t bidx = 0;
  // 8 independent loads in flight per thread, then the scan in index order
  int64_t k = threadIdx.x;
  for (; k + 7 * 1024 < n; k += 8 * 1024) {
    float x[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) x[u] = v[k + u * 1024];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (x[u] > best) {
        best = x[u];
        bidx = (int32_t)(k + u * 1024);
      }
  }
  for (; k < n; k += 1024) {
    const float x = v[k];
    if (x > best) {
      best = x;
      bidx = (int32_t)k;
    }
  }
  // wave: compare (value desc, index asc) through lane shuffles
  for (int off = 32; off > 0; off >>= 1) {
    const float ob = __shfl_xor(best, off, 64);
    const int32_t oi = __shfl_xor(bidx, off, 64);
    if (ob > best || (ob == best && oi < bidx)) {
      best = ob;
      bidx = oi;
    }
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    bv[w] = best;
    bi[w] = bidx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float b = bv[0];
    int32_t id = bi[0];
    for (int t = 1; t < 16; ++t)
      if (bv[t] > b || (bv[t] == b && bi[t] < id)) {
        b = bv[t];
        id = bi[t];
      }
    out[0] = id;
  }
}

__global__ void pos_advance_kernel(int *pos, int s) {
  if (threadIdx.x == 0) pos[0] += s;
}

inline unsigned blocks_for(int64_t n, int t) { return (unsigned)((n + t - 1) / t); }

template <int HD, int GRP>
hipError_t launch_attn_t(const AttnArgs &a, hipStream_t st) {
  hipLaunchKernelGGL((attn_split_kernel<HD, GRP>), dim3((unsigned)a.nkv, (unsigned)a.nsplit, (unsigned)a.s),
                     dim3(64 * GRP), 0, st, a.q, a.kc, a.vc, a.part, a.nheads, a.nkv, a.posp,
                     a.pos0, a.nsplit, a.maxlen, a.ldq);
  hipLaunchKernelGGL((attn_combine_kernel<HD>), dim3((unsigned)a.nheads, (unsigned)a.s), dim3(64), 0,
                     st, a.part, a.out, a.nheads, a.posp, a.pos0, a.nsplit, a.maxlen);
  return hipGetLastError();
}

template <int HD, int GRP>
hipError_t launch_prefill_t(const AttnArgs &a, hipStream_t st) {
  constexpr int PB = 4 * (32 / GRP);
  hipLaunchKernelGGL((attn_prefill_kernel<HD, GRP>), dim3((unsigned)a.nkv, (unsigned)((a.s + PB - 1) / PB)),
                     dim3(256), 0, st, a.q, a.kc, a.vc, a.out, a.s, a.nheads, a.nkv, a.posp,
                     a.pos0, a.maxlen, a.ldq);
  return hipGetLastError();
}

template <int HD>
hipError_t launch_attn_hd(const AttnArgs &a, hipStream_t st) {
  const bool mfma = a.s >= kPrefillMinRows;
  switch (a.nheads / a.nkv) {
    case 1: return mfma ? launch_prefill_t<HD, 1>(a, st) : launch_attn_t<HD, 1>(a, st);
    case 2: return mfma ? launch_prefill_t<HD, 2>(a, st) : launch_attn_t<HD, 2>(a, st);
    case 4: return mfma ? launch_prefill_t<HD, 4>(a, st) : launch_attn_t<HD, 4>(a, st);
    case 8: return mfma ? launch_prefill_t<HD, 8>(a, st) : launch_attn_t<HD, 8>(a, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_rmsnorm(const uint16_t *wn, const float *x, const float *res, float *h_out,
                          float *y, int64_t rows, int64_t d, float eps, hipStream_t st,
                          int64_t per, int64_t ld) {
  if (rows == 0) return hipSuccess;
  if (per <= 0) {          // dense rows
    per = 1;
    ld = d;
  }
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)rows), dim3(256), 0, st, wn, x, res, h_out, y,
                     d, eps, per, ld);
  return hipGetLastError();
}

hipError_t launch_rope_kv(float *q, float *k, const float *v, __half *kc, __half *vc,
                          const float *inv, int s, const int *posp, int pos0, int nheads, int nkv,
                          int head_dim, int64_t maxlen, int64_t ldq, int64_t ldk,
                          hipStream_t st) {
  if (s == 0) return hipSuccess;
  const int64_t n = (int64_t)s * (nheads + nkv) * (head_dim / 2) + (int64_t)s * nkv * head_dim;
  hipLaunchKernelGGL(rope_kv_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, st, q, k, v, kc, vc,
                     inv, s, posp, pos0, nheads, nkv, head_dim, maxlen, ldq, ldk);
  return hipGetLastError();
}

hipError_t launch_attention(const AttnArgs &a, hipStream_t st) {
  if (a.s == 0) return hipSuccess;
  if (a.head_dim == 64) return launch_attn_hd<64>(a, st);
  if (a.head_dim == 128) return launch_attn_hd<128>(a, st);
  return hipErrorInvalidValue;
}

template <int HD, int GRP>
hipError_t launch_decode_attn_t(const DecodeAttnArgs &a, hipStream_t st) {
  hipLaunchKernelGGL((attn_decode_kernel<HD, GRP>), dim3((unsigned)a.nkv, (unsigned)a.nsplit),
                     dim3(64 * decode_attn_waves(HD, GRP)), 0, st, a.q, a.k, a.v, a.inv, a.kc, a.vc, a.part, a.out, a.nkv,
                     a.posp, a.pos0, a.maxlen, a.qnorm, a.knorm, a.eps);
  if (a.nsplit > 1)      // one split: its blocks wrote the output
    hipLaunchKernelGGL((attn_merge_kernel<HD, GRP>), dim3((unsigned)a.nheads), dim3(HD), 0, st,
                       a.part, a.out, a.nsplit, a.posp, a.pos0, a.maxlen);
  return hipGetLastError();
}

hipError_t launch_decode_attention(const DecodeAttnArgs &a, hipStream_t st) {
  const int grp = a.nheads / a.nkv;
  if (a.nsplit < 1 || a.nsplit > kDecodeAttnMaxSplit) return hipErrorInvalidValue;
  if (a.head_dim == 64) {
    if (grp == 1) return launch_decode_attn_t<64, 1>(a, st);
    if (grp == 2) return launch_decode_attn_t<64, 2>(a, st);
    if (grp == 4) return launch_decode_attn_t<64, 4>(a, st);
    if (grp == 8) return launch_decode_attn_t<64, 8>(a, st);
  } else if (a.head_dim == 128) {
    if (grp == 1) return launch_decode_attn_t<128, 1>(a, st);
    if (grp == 2) return launch_decode_attn_t<128, 2>(a, st);
    if (grp == 4) return launch_decode_attn_t<128, 4>(a, st);
    if (grp == 8) return launch_decode_attn_t<128, 8>(a, st);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_swiglu(float *g, const float *u, int64_t n, hipStream_t st) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(swiglu_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, st, g, u, n);
  return hipGetLastError();
}

hipError_t launch_res_add(const float *x, const float *o, float *y, int64_t n, hipStream_t st) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(res_add_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, st, x, o, y, n);
  return hipGetLastError();
}

hipError_t launch_add(const float *x, float *y, int64_t n, hipStream_t st) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(add_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, st, x, y, n);
  return hipGetLastError();
}

hipError_t launch_argmax(const float *v, int64_t n, int32_t *out, hipStream_t st) {
  hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, st, v, n, out);
  return hipGetLastError();
}

hipError_t launch_pos_advance(int *pos, int s, hipStream_t st) {
  hipLaunchKernelGGL(pos_advance_kernel, dim3(1), dim3(64), 0, st, pos, s);
  return hipGetLastError();
}

}  // namespace q8
