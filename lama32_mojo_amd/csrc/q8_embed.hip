// q8_embed.hip -- embedding gather from packed Q8 rows (gfx950).
//
// y[i, c] = f32(int8 q[id_i, c]) * f32(scale[id_i, c / G])
// (k_embed_gather_q8, src/llama_q8.mojo:96-109: one f32 multiply, so the
// result is bit-exact).  One thread per 4 outputs; ids outside [0, vocab)
// produce NaN rows instead of reading outside the table.
#include "q8_device.h"
#include "q8_launch.h"

namespace q8 {
namespace {

template <int G, int KIND>
__global__ __launch_bounds__(256) void embed_gather_kernel(
    const uint8_t *__restrict__ w, int64_t row_bytes,
    const int32_t *__restrict__ ids, float *__restrict__ y, int64_t s,
    int64_t d, int64_t vocab) {
  constexpr int SB = ScaleTraits<KIND>::bytes;
  const int64_t quads = d / 4;                 // d % 32 == 0
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= s * quads) return;
  const int64_t i = t / quads;
  const int64_t c = (t - i * quads) * 4;
  const int64_t id = ids[i];
  float *out = y + i * d + c;
  if (id < 0 || id >= vocab) {
    const float nan = __builtin_nanf("");
    out[0] = nan; out[1] = nan; out[2] = nan; out[3] = nan;
    return;
  }
  const uint8_t *row = w + id * row_bytes;
  const float sc = load_scale<KIND>(row, c / G);
  const int8_t *codes = reinterpret_cast<const int8_t *>(row + (d / G) * SB);
#pragma unroll
  for (int u = 0; u < 4; ++u) out[u] = (float)codes[c + u] * sc;
}

template <int G, int KIND>
hipError_t launch_g(const GatherArgs &a, hipStream_t st) {
  const int64_t threads = a.s * (a.d / 4);
  dim3 grid((unsigned)((threads + 255) / 256)), block(256);
  hipLaunchKernelGGL((embed_gather_kernel<G, KIND>), grid, block, 0, st, a.w,
                     a.row_bytes, a.ids, a.y, a.s, a.d, a.vocab);
  return hipGetLastError();
}

// The token step's last launch: the argmax over the GEMV's per-workgroup
// partials (value desc, row asc; k_argmax's result: index 0 when logits[0]
// is NaN or no value exceeds it), written to ids[0]; the device position
// advanced; and, with emb, the embedding row of that id gathered into xnext
// exactly as embed_gather_kernel gathers it.  One 1024-thread workgroup.
template <int G, int KIND>
__global__ __launch_bounds__(1024) void argmax_finish_kernel(
    const float *__restrict__ part, int nblocks, const float *__restrict__ logits,
    int32_t *__restrict__ ids, int *pos, int pos_step, const uint8_t *__restrict__ emb,
    int64_t row_bytes, int64_t vocab, float *__restrict__ xnext, int64_t d) {
  constexpr int SB = ScaleTraits<KIND>::bytes;
  __shared__ float bv[16];
  __shared__ int bi[16];
  __shared__ int sid;
  const int *pidx = reinterpret_cast<const int *>(part + nblocks);
  float best = -INFINITY;
  int bidx = INT32_MAX;
  // the partials in batches of 8 independent loads per thread, then the
  // compares (in index order within the thread)
  for (int t0 = threadIdx.x; t0 < nblocks; t0 += 8 * 1024) {
    float v[8];
    int i[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int t = t0 + 1024 * u;
      v[u] = t < nblocks ? part[t] : -INFINITY;
      i[u] = t < nblocks ? pidx[t] : INT32_MAX;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (v[u] > best || (v[u] == best && i[u] < bidx)) {
        best = v[u];
        bidx = i[u];
      }
  }
  for (int off = 32; off > 0; off >>= 1) {
    const float ob = __shfl_xor(best, off, 64);
    const int oi = __shfl_xor(bidx, off, 64);
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
    int id = bi[0];
    for (int t = 1; t < 16; ++t)
      if (bv[t] > b || (bv[t] == b && bi[t] < id)) {
        b = bv[t];
        id = bi[t];
      }
    const float v0 = logits[0];
    if (id == INT32_MAX || v0 != v0) id = 0;
    ids[0] = id;
    if (pos) pos[0] += pos_step;
    sid = id;
  }
  if (!emb) return;
  __syncthreads();
  // (ids are logit rows, below vocab by construction; the clamp keeps the
  // gather inside the table whatever the partials hold)
  const int64_t id = sid < vocab ? sid : 0;
  const uint8_t *row = emb + id * row_bytes;
  const int8_t *codes = reinterpret_cast<const int8_t *>(row + (d / G) * SB);
  for (int64_t c = 4 * (int64_t)threadIdx.x; c < d; c += 4 * 1024) {
    const float sc = load_scale<KIND>(row, c / G);
#pragma unroll
    for (int u = 0; u < 4; ++u) xnext[c + u] = (float)codes[c + u] * sc;
  }
}

template <int G, int KIND>
hipError_t launch_finish_g(const ArgmaxFinishArgs &a, hipStream_t st) {
  hipLaunchKernelGGL((argmax_finish_kernel<G, KIND>), dim3(1), dim3(1024), 0, st, a.part,
                     a.nblocks, a.logits, a.ids, a.pos, a.pos_step, a.emb, a.row_bytes, a.vocab,
                     a.xnext, a.d);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_argmax_finish(const ArgmaxFinishArgs &a, hipStream_t st) {
  if (a.nblocks < 1 || a.nblocks > kArgmaxMaxBlocks) return hipErrorInvalidValue;
  if (!a.emb || (a.G == 64 && a.kind == SCALE_F16)) return launch_finish_g<64, SCALE_F16>(a, st);
  if (a.G == 64 && a.kind == SCALE_F32) return launch_finish_g<64, SCALE_F32>(a, st);
  if (a.G == 32 && a.kind == SCALE_F16) return launch_finish_g<32, SCALE_F16>(a, st);
  if (a.G == 32 && a.kind == SCALE_F32) return launch_finish_g<32, SCALE_F32>(a, st);
  return hipErrorInvalidValue;
}

hipError_t launch_embed_gather(const GatherArgs &a, hipStream_t st) {
  if (a.s == 0) return hipSuccess;
  if (a.G == 64 && a.kind == SCALE_F16) return launch_g<64, SCALE_F16>(a, st);
  if (a.G == 64 && a.kind == SCALE_F32) return launch_g<64, SCALE_F32>(a, st);
  if (a.G == 32 && a.kind == SCALE_F16) return launch_g<32, SCALE_F16>(a, st);
  if (a.G == 32 && a.kind == SCALE_F32) return launch_g<32, SCALE_F32>(a, st);
  return hipErrorInvalidValue;
}

}  // namespace q8
