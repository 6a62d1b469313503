// q8_device.h -- device-side helpers shared by the gfx950 kernels.
//
// Packed rows (qwen3_mojo/scripts/quantize.py:4-12): [ (m/G) scales | m int8 ]
// with each scale a binary16 (SCALE_F16, the reference layout) or an f32
// (SCALE_F32).  All kernels address a row by its byte base and take the
// scale section's size in bytes, so both layouts share one code path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace q8 {

enum ScaleKind { SCALE_F16 = 1, SCALE_F32 = 2 };

template <int KIND> struct ScaleTraits;
template <> struct ScaleTraits<SCALE_F16> { static constexpr int bytes = 2; };
template <> struct ScaleTraits<SCALE_F32> { static constexpr int bytes = 4; };

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

// f32 -> binary16 with the hardware conversion (round to nearest even in the
// default float mode; binary16 denormals are kept on gfx9).
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) {
  return __builtin_bit_cast(float, b << 16);
}

// Scale g of a packed row starting at byte pointer `row`.
template <int KIND>
__device__ __forceinline__ float load_scale(const uint8_t *row, int64_t g) {
  if constexpr (KIND == SCALE_F16) {
    return f16_bits_to_f32(*reinterpret_cast<const uint16_t *>(row + 2 * g));
  } else {
    // f32 scales sit at 2-byte alignment in general: assemble from halves.
    const uint16_t *p = reinterpret_cast<const uint16_t *>(row + 4 * g);
    return __builtin_bit_cast(float, (uint32_t)p[0] | ((uint32_t)p[1] << 16));
  }
}

// Signed byte `i` (0..3) of a dword, converted to f32 exactly.
template <int I>
__device__ __forceinline__ float sbyte_to_f32(uint32_t w) {
  return (float)(int32_t)((int32_t)(w << (24 - 8 * I)) >> 24);
}

// Unscaled dot product of 16 signed codes (one dwordx4) with 16 f32 values.
__device__ __forceinline__ float dot16(u32x4 q, f32x4 xa, f32x4 xb, f32x4 xc, f32x4 xd) {
  float p = xa.x * sbyte_to_f32<0>(q.x);
  p = __builtin_fmaf(xa.y, sbyte_to_f32<1>(q.x), p);
  p = __builtin_fmaf(xa.z, sbyte_to_f32<2>(q.x), p);
  p = __builtin_fmaf(xa.w, sbyte_to_f32<3>(q.x), p);
  p = __builtin_fmaf(xb.x, sbyte_to_f32<0>(q.y), p);
  p = __builtin_fmaf(xb.y, sbyte_to_f32<1>(q.y), p);
  p = __builtin_fmaf(xb.z, sbyte_to_f32<2>(q.y), p);
  p = __builtin_fmaf(xb.w, sbyte_to_f32<3>(q.y), p);
  p = __builtin_fmaf(xc.x, sbyte_to_f32<0>(q.z), p);
  p = __builtin_fmaf(xc.y, sbyte_to_f32<1>(q.z), p);
  p = __builtin_fmaf(xc.z, sbyte_to_f32<2>(q.z), p);
  p = __builtin_fmaf(xc.w, sbyte_to_f32<3>(q.z), p);
  p = __builtin_fmaf(xd.x, sbyte_to_f32<0>(q.w), p);
  p = __builtin_fmaf(xd.y, sbyte_to_f32<1>(q.w), p);
  p = __builtin_fmaf(xd.z, sbyte_to_f32<2>(q.w), p);
  p = __builtin_fmaf(xd.w, sbyte_to_f32<3>(q.w), p);
  return p;
}

// ---- buffer loads and bf16 packing (MFMA kernels) -----------------------

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;

// Raw buffer resource (stride 0, 32-bit data format).  Loads whose VGPR
// offset lies at or past `bytes` return zeros, so every read of a ragged
// edge is either inside the tensor or zero-filled.
__device__ __forceinline__ rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes,
                                           0x00020000);
}
__device__ __forceinline__ u32x4 bload16(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ float bload4f(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__device__ __forceinline__ uint32_t bload2(rsrc_t r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}
constexpr uint32_t kOutOfRange = 0x80000000u;   // an offset past every tensor here

__device__ __forceinline__ uint32_t pk_hi16(float lo, float hi) {
  // Upper halves of two f32 whose values are exact in bf16.
  return __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, hi), __builtin_bit_cast(uint32_t, lo),
                               0x07060302u);
}

// 8 signed codes (two dwords) -> 8 bf16, exact.
__device__ __forceinline__ bf16x8_t codes_to_bf16(uint32_t d0, uint32_t d1) {
  u32x4 o = {pk_hi16(sbyte_to_f32<0>(d0), sbyte_to_f32<1>(d0)),
             pk_hi16(sbyte_to_f32<2>(d0), sbyte_to_f32<3>(d0)),
             pk_hi16(sbyte_to_f32<0>(d1), sbyte_to_f32<1>(d1)),
             pk_hi16(sbyte_to_f32<2>(d1), sbyte_to_f32<3>(d1))};
  return __builtin_bit_cast(bf16x8_t, o);
}

__device__ __forceinline__ uint32_t bf16_rne(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

// ---- wavefront reductions (wave64) --------------------------------------
// DPP row operations reduce within each row of 16 lanes; the four row sums
// are then combined with readlane.  Every lane returns the full sum.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                         0xf, 0xf, false));
}

__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_mov<0xb1>(v);   // quad_perm [1,0,3,2]
  v += dpp_mov<0x4e>(v);   // quad_perm [2,3,0,1]
  v += dpp_mov<0x141>(v);  // row_half_mirror
  v += dpp_mov<0x140>(v);  // row_mirror
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return (a + b) + (c + d);
}

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

// Sum over a 256-thread block (4 waves), the same value in every thread:
// wave sums, then (w0 + w1) + (w2 + w3).  red: 4 floats of LDS.
__device__ __forceinline__ float block_sum256(float v, float *red) {
  v = wave_sum(v);
  const int wid = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wid] = v;
  __syncthreads();
  const float t = (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();
  return t;
}

// Max of |.| with NaN propagation (numpy's max propagates NaN).
__device__ __forceinline__ float nanmax(float a, float b) {
  if (a != a) return a;
  if (b != b) return b;
  return a > b ? a : b;
}

}  // namespace q8
