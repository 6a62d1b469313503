// q8_gemm.hip -- prefill-path Q8 GEMM on gfx950 bf16 MFMA.
//
// y[i, j] = sum_g scale[j, g] * sum_{k in g} x[i, k] * q[j, k]
// (k_mm_q8's arithmetic, src/llama_q8.mojo:73-84: unscaled dot per group,
// one scale multiply per group) computed as a tiled GEMM:
//   * int8 codes are converted to bf16 once per workgroup while staging the
//     weight tile into LDS; |q| <= 127 is exact in bf16, and a bf16 x bf16
//     product is exact in the f32 MFMA accumulator, so the per-group partial
//     dot is computed exactly up to f32 accumulation;
//   * each group's partial lives in its own MFMA accumulator (started at 0)
//     and is folded into the running f32 result with one v_fma per output
//     and group, using the per-column scale held in LDS;
//   * f32 activations (the W8A32 path with large s) are split into
//     hi = bf16(x) and lo = bf16(x - hi) and run as two MFMAs; the residual
//     error is below 2^-17 |x|.
// Tiles: 128 x 128 outputs per 256-thread workgroup, K step 64, four waves
// in a 2 x 2 arrangement each owning 64 x 64 = 2 x 2 v_mfma_f32_32x32x16_bf16
// tiles.
#include "q8_device.h"
#include "q8_launch.h"

namespace q8 {
namespace {

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int LDA = BK + 8;     // bf16 elements per LDS row (16 B pad)

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

__device__ __forceinline__ uint32_t pack_bf16_pair_from_f32(float lo, float hi) {
  // Upper halves of two f32 whose values are exact in bf16.
  return __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, hi),
                               __builtin_bit_cast(uint32_t, lo), 0x07060302u);
}

__device__ __forceinline__ uint16_t bf16_rne_bits(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

template <int G, int KIND, bool XF32>
__global__ __launch_bounds__(256) void gemm_kernel(
    const uint8_t *__restrict__ w, int64_t row_bytes, const void *__restrict__ xv,
    float *__restrict__ y, int64_t s, int64_t m, int64_t n) {
  constexpr int SB = ScaleTraits<KIND>::bytes;
  constexpr int GPB = BK / G;   // groups per K step (1 or 2)
  __shared__ __attribute__((aligned(16))) uint16_t As[BM * LDA];
  __shared__ __attribute__((aligned(16))) uint16_t Al[XF32 ? BM * LDA : 8];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[BN * LDA];
  __shared__ float Ss[BN * GPB];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = tid >> 6;
  const int wm = wid >> 1, wn = wid & 1;
  const int64_t m0 = (int64_t)blockIdx.y * BM;
  const int64_t n0 = (int64_t)blockIdx.x * BN;
  const int64_t scale_bytes = (m / G) * SB;

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  for (int64_t k0 = 0; k0 < m; k0 += BK) {
    // ---- stage A (activations) --------------------------------------------
    if constexpr (!XF32) {
      const uint16_t *x = reinterpret_cast<const uint16_t *>(xv);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int c = tid + 256 * u;          // 1024 chunks of 8 bf16
        const int row = c >> 3, kc = (c & 7) * 8;
        u32x4 v = {0u, 0u, 0u, 0u};
        if (m0 + row < s && k0 + kc < m)
          v = *reinterpret_cast<const u32x4 *>(x + (m0 + row) * m + k0 + kc);
        *reinterpret_cast<u32x4 *>(&As[row * LDA + kc]) = v;
      }
    } else {
      const float *x = reinterpret_cast<const float *>(xv);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int c = tid + 256 * u;
        const int row = c >> 3, kc = (c & 7) * 8;
        f32x4 a = {0.f, 0.f, 0.f, 0.f}, b = {0.f, 0.f, 0.f, 0.f};
        if (m0 + row < s && k0 + kc < m) {
          const f32x4 *p = reinterpret_cast<const f32x4 *>(x + (m0 + row) * m + k0 + kc);
          a = p[0];
          b = p[1];
        }
        float f[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        uint16_t hi[8], lo[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          hi[e] = bf16_rne_bits(f[e]);
          lo[e] = bf16_rne_bits(f[e] - bf16_bits_to_f32(hi[e]));
        }
        u32x4 vh, vl;
        vh.x = hi[0] | ((uint32_t)hi[1] << 16); vh.y = hi[2] | ((uint32_t)hi[3] << 16);
        vh.z = hi[4] | ((uint32_t)hi[5] << 16); vh.w = hi[6] | ((uint32_t)hi[7] << 16);
        vl.x = lo[0] | ((uint32_t)lo[1] << 16); vl.y = lo[2] | ((uint32_t)lo[3] << 16);
        vl.z = lo[4] | ((uint32_t)lo[5] << 16); vl.w = lo[6] | ((uint32_t)lo[7] << 16);
        *reinterpret_cast<u32x4 *>(&As[row * LDA + kc]) = vh;
        *reinterpret_cast<u32x4 *>(&Al[row * LDA + kc]) = vl;
      }
    }
    // ---- stage B (codes -> bf16) -----------------------------------------------
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int c = tid + 256 * u;            // 512 chunks of 16 codes
      const int row = c >> 2, kc = (c & 3) * 16;
      u32x4 q = {0u, 0u, 0u, 0u};
      if (n0 + row < n && k0 + kc < m)
        q = *reinterpret_cast<const u32x4 *>(w + (n0 + row) * row_bytes + scale_bytes + k0 + kc);
      uint32_t d[4] = {q.x, q.y, q.z, q.w};
      u32x4 o0, o1;
      uint32_t o[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        o[2 * e] = pack_bf16_pair_from_f32(sbyte_to_f32<0>(d[e]), sbyte_to_f32<1>(d[e]));
        o[2 * e + 1] = pack_bf16_pair_from_f32(sbyte_to_f32<2>(d[e]), sbyte_to_f32<3>(d[e]));
      }
      o0.x = o[0]; o0.y = o[1]; o0.z = o[2]; o0.w = o[3];
      o1.x = o[4]; o1.y = o[5]; o1.z = o[6]; o1.w = o[7];
      *reinterpret_cast<u32x4 *>(&Bs[row * LDA + kc]) = o0;
      *reinterpret_cast<u32x4 *>(&Bs[row * LDA + kc + 8]) = o1;
    }
    if (tid < BN * GPB) {
      const int row = tid / GPB, gi = tid % GPB;
      const int64_t g = k0 / G + gi;
      float sc = 0.0f;
      if (n0 + row < n && g < m / G) sc = load_scale<KIND>(w + (n0 + row) * row_bytes, g);
      Ss[row * GPB + gi] = sc;
    }
    __syncthreads();

    // ---- MFMA --------------------------------------------------------------------
    const int lr = lane & 31;
    const int lk = (lane >> 5) * 8;
#pragma unroll
    for (int gi = 0; gi < GPB; ++gi) {
      f32x16 tmp[2][2];
#pragma unroll
      for (int ks = 0; ks < G / 16; ++ks) {
        const int kk = gi * G + ks * 16 + lk;
        bf16x8_t a[2], al[2], b[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          a[i] = *reinterpret_cast<const bf16x8_t *>(&As[(wm * 64 + i * 32 + lr) * LDA + kk]);
          if constexpr (XF32)
            al[i] = *reinterpret_cast<const bf16x8_t *>(&Al[(wm * 64 + i * 32 + lr) * LDA + kk]);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j)
          b[j] = *reinterpret_cast<const bf16x8_t *>(&Bs[(wn * 64 + j * 32 + lr) * LDA + kk]);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            if (ks == 0) {
              const f32x16 z = {};
              tmp[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], z, 0, 0, 0);
            } else {
              tmp[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], tmp[i][j], 0, 0, 0);
            }
            if constexpr (XF32)
              tmp[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[i], b[j], tmp[i][j], 0, 0, 0);
          }
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float sc = Ss[(wn * 64 + j * 32 + lr) * GPB + gi];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int v = 0; v < 16; ++v) acc[i][j][v] = __builtin_fmaf(sc, tmp[i][j][v], acc[i][j][v]);
      }
    }
    __syncthreads();
  }

  // ---- epilogue: D layout of v_mfma_f32_32x32x16: lane -> column lane % 32,
  // element v -> row 8 (v / 4) + 4 (lane / 32) + v % 4.
  const int lr = lane & 31;
  const int lh = lane >> 5;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t col = n0 + wn * 64 + j * 32 + lr;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t row = m0 + wm * 64 + i * 32 + (v >> 2) * 8 + lh * 4 + (v & 3);
        if (row < s && col < n) y[row * n + col] = acc[i][j][v];
      }
    }
}

template <int G, int KIND>
hipError_t launch_g(const LinearArgs &a, hipStream_t st) {
  dim3 grid((unsigned)((a.n + BN - 1) / BN), (unsigned)((a.s + BM - 1) / BM)), block(256);
  if (a.x_is_bf16)
    hipLaunchKernelGGL((gemm_kernel<G, KIND, false>), grid, block, 0, st, a.w,
                       a.row_bytes, a.x, a.y, a.s, a.m, a.n);
  else
    hipLaunchKernelGGL((gemm_kernel<G, KIND, true>), grid, block, 0, st, a.w,
                       a.row_bytes, a.x, a.y, a.s, a.m, a.n);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm(const LinearArgs &a, hipStream_t st) {
  if (a.s == 0 || a.n == 0) return hipSuccess;
  if (a.G == 64 && a.kind == SCALE_F16) return launch_g<64, SCALE_F16>(a, st);
  if (a.G == 64 && a.kind == SCALE_F32) return launch_g<64, SCALE_F32>(a, st);
  if (a.G == 32 && a.kind == SCALE_F16) return launch_g<32, SCALE_F16>(a, st);
  if (a.G == 32 && a.kind == SCALE_F32) return launch_g<32, SCALE_F32>(a, st);
  return hipErrorInvalidValue;
}

}  // namespace q8
