// q8_pack.hip -- quantize + pack kernel for gfx950.
//
// Bit-exact restatement of pack_q8 (qwen3_mojo/scripts/quantize.py:31-43):
//   per group of G weights along the input dim
//     scale = max|w| / 127             f32, correctly rounded division (:36)
//     scale = max(scale, 1e-8f)        f32; NaN stays NaN (:37)
//     scale16 = RNE f16(scale)         binary16 with denormals (:37)
//     q = rint(w / f32(scale16))       correctly rounded division, ties-even (:38)
//     q = clip(q, -127, 127) -> int8   NaN (0/0 for scale16 == 0) -> 0 (:39)
//   packed row: [scale16 x m/G | int8 x m] (:41-42)
// With SCALE_F32 the f16 rounding is skipped and each scale is an f32.
//
// Mapping: one thread per 8 consecutive weights, so a group of G weights is
// G/8 adjacent lanes of one wavefront (aligned, never straddling a wave).
// The group's |max| is reduced across those lanes with DPP quad/half-row
// moves; each lane then writes its 8 codes, and the group's first lane
// writes the scale.  Loads are 16-byte vectors when the source allows.
//
// This file must be compiled without fast-math and with correctly rounded
// f32 division (-fhip-fp32-correctly-rounded-divide-sqrt, hipcc's default).
#include "q8_device.h"
#include "q8_launch.h"

namespace q8 {
namespace {

template <int CTRL>
__device__ __forceinline__ float dpp_max_step(float v) {
  float o = __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                         0xf, 0xf, false));
  return nanmax(v, o);
}

template <bool SRC_F32, bool VEC_LOAD>
__device__ __forceinline__ void load8(const void *src, int64_t e, float v[8]) {
  if constexpr (SRC_F32) {
    const float *p = reinterpret_cast<const float *>(src) + e;
    if constexpr (VEC_LOAD) {
      f32x4 a = *reinterpret_cast<const f32x4 *>(p);
      f32x4 b = *reinterpret_cast<const f32x4 *>(p + 4);
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
      v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = p[i];
    }
  } else {
    const uint16_t *p = reinterpret_cast<const uint16_t *>(src) + e;
    if constexpr (VEC_LOAD) {
      u32x4 a = *reinterpret_cast<const u32x4 *>(p);
      uint32_t d[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[2 * i] = __builtin_bit_cast(float, d[i] << 16);
        v[2 * i + 1] = __builtin_bit_cast(float, d[i] & 0xffff0000u);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = bf16_bits_to_f32(p[i]);
    }
  }
}

__device__ __forceinline__ int32_t quant1(float w, float sf) {
  float r = w / sf;                 // correctly rounded f32 division
  float q = __builtin_rintf(r);     // round half to even
  if (q != q) return 0;             // NaN -> 0 (numpy's float->int8 cast)
  q = q > 127.0f ? 127.0f : q;
  q = q < -127.0f ? -127.0f : q;
  return (int32_t)q;
}

template <int G, int KIND, bool SRC_F32, bool VEC_LOAD>
__global__ __launch_bounds__(256) void pack_kernel(
    const void *__restrict__ src, int64_t n, int64_t m,
    uint8_t *__restrict__ dst, int64_t dst_row_bytes) {
  constexpr int LPG = G / 8;                       // lanes per group
  constexpr int SB = ScaleTraits<KIND>::bytes;
  const int64_t chunks_per_row = m / 8;
  const int64_t total = n * chunks_per_row;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const bool live = t < total;
  const int64_t j = live ? t / chunks_per_row : 0;
  const int64_t c = live ? t - j * chunks_per_row : 0;   // chunk within row

  float v[8];
  if (live) {
    load8<SRC_F32, VEC_LOAD>(src, j * m + c * 8, v);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = 0.0f;
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = nanmax(amax, __builtin_fabsf(v[i]));
  // Reduce over the LPG lanes of this group (all lanes take part).
  if constexpr (LPG >= 2) amax = dpp_max_step<0xb1>(amax);   // quad_perm [1,0,3,2]
  if constexpr (LPG >= 4) amax = dpp_max_step<0x4e>(amax);   // quad_perm [2,3,0,1]
  if constexpr (LPG >= 8) amax = dpp_max_step<0x141>(amax);  // row_half_mirror
  static_assert(LPG == 4 || LPG == 8, "G must be 32 or 64");

  float sc = amax / 127.0f;
  if (!(sc >= 1e-8f)) sc = (sc != sc) ? sc : 1e-8f;
  float sf;
  uint32_t sbits;
  if constexpr (KIND == SCALE_F16) {
    uint16_t h = f32_to_f16_bits(sc);
    sbits = h;
    sf = f16_bits_to_f32(h);
  } else {
    sf = sc;
    sbits = __builtin_bit_cast(uint32_t, sc);
  }
  if (!live) return;

  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) lo |= ((uint32_t)quant1(v[i], sf) & 0xffu) << (8 * i);
#pragma unroll
  for (int i = 0; i < 4; ++i) hi |= ((uint32_t)quant1(v[4 + i], sf) & 0xffu) << (8 * i);

  uint8_t *row = dst + j * dst_row_bytes;
  const int64_t g = c / LPG;
  // Codes section starts after (m/G) scales; it is 2-byte aligned.
  uint16_t *cp = reinterpret_cast<uint16_t *>(row + (m / G) * SB + c * 8);
  cp[0] = (uint16_t)lo;
  cp[1] = (uint16_t)(lo >> 16);
  cp[2] = (uint16_t)hi;
  cp[3] = (uint16_t)(hi >> 16);
  if (c % LPG == 0) {
    uint16_t *sp = reinterpret_cast<uint16_t *>(row + g * SB);
    sp[0] = (uint16_t)sbits;
    if constexpr (SB == 4) sp[1] = (uint16_t)(sbits >> 16);
  }
}

template <int G, int KIND>
hipError_t launch_pack_g(const PackArgs &a, hipStream_t st) {
  const int64_t total = a.n * (a.m / 8);
  const int64_t blocks = (total + 255) / 256;
  const uintptr_t base = reinterpret_cast<uintptr_t>(a.src);
  const bool vec = (base % 16 == 0);   // m % 8 == 0 keeps every row aligned
  dim3 grid((unsigned)blocks), block(256);
  if (a.src_is_f32) {
    if (vec)
      hipLaunchKernelGGL((pack_kernel<G, KIND, true, true>), grid, block, 0, st,
                         a.src, a.n, a.m, a.dst, a.dst_row_bytes);
    else
      hipLaunchKernelGGL((pack_kernel<G, KIND, true, false>), grid, block, 0, st,
                         a.src, a.n, a.m, a.dst, a.dst_row_bytes);
  } else {
    if (vec)
      hipLaunchKernelGGL((pack_kernel<G, KIND, false, true>), grid, block, 0, st,
                         a.src, a.n, a.m, a.dst, a.dst_row_bytes);
    else
      hipLaunchKernelGGL((pack_kernel<G, KIND, false, false>), grid, block, 0, st,
                         a.src, a.n, a.m, a.dst, a.dst_row_bytes);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_pack(const PackArgs &a, hipStream_t st) {
  if (a.n == 0) return hipSuccess;
  if (a.G == 64 && a.kind == SCALE_F16) return launch_pack_g<64, SCALE_F16>(a, st);
  if (a.G == 64 && a.kind == SCALE_F32) return launch_pack_g<64, SCALE_F32>(a, st);
  if (a.G == 32 && a.kind == SCALE_F16) return launch_pack_g<32, SCALE_F16>(a, st);
  if (a.G == 32 && a.kind == SCALE_F32) return launch_pack_g<32, SCALE_F32>(a, st);
  return hipErrorInvalidValue;
}

}  // namespace q8
