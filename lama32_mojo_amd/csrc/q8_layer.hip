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

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_mov<0xb1>(v));
  v = fmaxf(v, dpp_mov<0x4e>(v));
  v = fmaxf(v, dpp_mov<0x141>(v));
  v = fmaxf(v, dpp_mov<0x140>(v));
  const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

// Sum over a 256-thread block (4 waves); every thread gets the total.
__device__ __forceinline__ float block_sum256(float v, float *red) {
  v = wave_sum(v);
  const int wid = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wid] = v;
  __syncthreads();
  const float t = (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();
  return t;
}

// ---- RMSNorm (k_rmsnorm_w): y = bf16(w) * x * 1/sqrt(mean(x^2) + eps) -------
// One 256-thread block per row.  With res != null the row is h = x + res,
// stored to h_out, and normalised (k_res_add followed by k_rmsnorm_w).
__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t *__restrict__ wn,
                                                      const float *x, const float *res,
                                                      float *h_out, float *y, int64_t d,
                                                      float eps) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const float *xr = x + row * d;
  const float *rr = res ? res + row * d : nullptr;
  float ss = 0.0f;
  for (int64_t k = threadIdx.x; k < d; k += 256) {
    float v = xr[k];
    if (rr) {
      v += rr[k];
      h_out[row * d + k] = v;
    }
    ss = __builtin_fmaf(v, v, ss);
  }
  ss = block_sum256(ss, red);
  const float inv = 1.0f / sqrtf(ss / (float)d + eps);
  const float *src = rr ? h_out + row * d : xr;
  for (int64_t k = threadIdx.x; k < d; k += 256)
    y[row * d + k] = bf16_bits_to_f32(wn[k]) * src[k] * inv;
}

// ---- RoPE on q and k + KV append (k_rope_qk_copy2) ----------------------------
// HF rotate_half RoPE in place on q [s, qdim] and k [s, kvdim]; the rotated
// k and the unrotated v of row i are stored as binary16 at cache row
// pos0 + i (rows past maxlen are dropped).  One thread per rotated pair and
// one per v element.
__global__ __launch_bounds__(256) void rope_kv_kernel(float *q, float *k, const float *v,
                                                      __half *kc, __half *vc,
                                                      const float *inv, int s, const int *posp,
                                                      int pos0_host, int nheads, int nkv,
                                                      int head_dim, int64_t maxlen) {
  const int half = head_dim / 2;
  const int nall = nheads + nkv;
  const int64_t nrope = (int64_t)s * nall * half;
  const int qdim = nheads * head_dim, kvdim = nkv * head_dim;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int pos0 = posp ? *posp : pos0_host;
  if (idx < nrope) {
    const int i = (int)(idx / (nall * half));
    const int r = (int)(idx % (nall * half));
    const int h = r / half, d = r % half;
    const float freq = (float)(pos0 + i) * inv[d];
    const float c = cosf(freq), sn = sinf(freq);
    if (h < nheads) {
      float *base = q + (int64_t)i * qdim + h * head_dim;
      const float x0 = base[d], x1 = base[half + d];
      base[d] = x0 * c - x1 * sn;
      base[half + d] = x1 * c + x0 * sn;
    } else {
      const int hk = h - nheads;
      float *base = k + (int64_t)i * kvdim + hk * head_dim;
      const float x0 = base[d], x1 = base[half + d];
      const float y0 = x0 * c - x1 * sn, y1 = x1 * c + x0 * sn;
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
    if (row < maxlen) vc[row * kvdim + vi % kvdim] = __float2half_rn(v[vi]);
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
                                                              int maxlen) {
  constexpr int KC = 64;                       // keys per split
  constexpr int PW = HD + 2;                   // partial record: o[HD], m, l
  __shared__ float qs[GRP][HD];
  __shared__ float ps[GRP][KC];
  const int g = blockIdx.x, sp = blockIdx.y, i = blockIdx.z;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int h = g * GRP + w;
  const int qdim = nheads * HD, kvdim = nkv * HD;
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
  for (int d = lane; d < HD; d += 64) qs[w][d] = q[(int64_t)i * qdim + h * HD + d];
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
  for (int64_t k = threadIdx.x; k < n; k += 1024) {
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
                     a.pos0, a.nsplit, a.maxlen);
  hipLaunchKernelGGL((attn_combine_kernel<HD>), dim3((unsigned)a.nheads, (unsigned)a.s), dim3(64), 0,
                     st, a.part, a.out, a.nheads, a.posp, a.pos0, a.nsplit, a.maxlen);
  return hipGetLastError();
}

template <int HD>
hipError_t launch_attn_hd(const AttnArgs &a, hipStream_t st) {
  switch (a.nheads / a.nkv) {
    case 1: return launch_attn_t<HD, 1>(a, st);
    case 2: return launch_attn_t<HD, 2>(a, st);
    case 4: return launch_attn_t<HD, 4>(a, st);
    case 8: return launch_attn_t<HD, 8>(a, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_rmsnorm(const uint16_t *wn, const float *x, const float *res, float *h_out,
                          float *y, int64_t rows, int64_t d, float eps, hipStream_t st) {
  if (rows == 0) return hipSuccess;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)rows), dim3(256), 0, st, wn, x, res, h_out, y,
                     d, eps);
  return hipGetLastError();
}

hipError_t launch_rope_kv(float *q, float *k, const float *v, __half *kc, __half *vc,
                          const float *inv, int s, const int *posp, int pos0, int nheads, int nkv,
                          int head_dim, int64_t maxlen, hipStream_t st) {
  if (s == 0) return hipSuccess;
  const int64_t n = (int64_t)s * (nheads + nkv) * (head_dim / 2) + (int64_t)s * nkv * head_dim;
  hipLaunchKernelGGL(rope_kv_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, st, q, k, v, kc, vc,
                     inv, s, posp, pos0, nheads, nkv, head_dim, maxlen);
  return hipGetLastError();
}

hipError_t launch_attention(const AttnArgs &a, hipStream_t st) {
  if (a.s == 0) return hipSuccess;
  if (a.head_dim == 64) return launch_attn_hd<64>(a, st);
  if (a.head_dim == 128) return launch_attn_hd<128>(a, st);
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
