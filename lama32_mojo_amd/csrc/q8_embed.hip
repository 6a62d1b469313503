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

}  // namespace

hipError_t launch_embed_gather(const GatherArgs &a, hipStream_t st) {
  if (a.s == 0) return hipSuccess;
  if (a.G == 64 && a.kind == SCALE_F16) return launch_g<64, SCALE_F16>(a, st);
  if (a.G == 64 && a.kind == SCALE_F32) return launch_g<64, SCALE_F32>(a, st);
  if (a.G == 32 && a.kind == SCALE_F16) return launch_g<32, SCALE_F16>(a, st);
  if (a.G == 32 && a.kind == SCALE_F32) return launch_g<32, SCALE_F32>(a, st);
  return hipErrorInvalidValue;
}

}  // namespace q8
