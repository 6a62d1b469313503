// q8_gemv.hip -- decode-path Q8 GEMV for gfx950 (f32 activations, s <= 4 per pass).
//
// y[b, j] = sum_g scale[j, g] * sum_{k in g} x[b, k] * q[j, k]
// (k_mm_q8, src/llama_q8.mojo:54-93: unscaled dot per group, then one scale
// multiply per group).
//
// The kernel is HBM-bound: every weight byte is read exactly once.  Layout
// and mapping:
//   * a wavefront owns R whole rows at a time (or, for rows longer than 4096
//     codes, one K quarter of R rows shared by the workgroup's 4 waves); lane
//     l owns the 16-byte code slices k = 16 l + 1024 i, so each load
//     instruction is one 1 KiB fully coalesced run per row
//     (global_load_dwordx4, non-temporal);
//   * the R rows' loads are issued together, so a wave keeps R KiB in flight
//     per step and many waves per CU cover HBM latency;
//   * the lane's 16 codes lie inside one quantization group (16 | G), so one
//     scale per row per step is applied after the unscaled 16-term dot;
//   * x (S rows of m f32) is staged once per workgroup in LDS and read with
//     ds_read_b128;
//   * each (row, batch) partial is reduced across the wave with DPP row
//     moves plus readlane; lane 0 stores.
// Rows are distributed over a grid sized to fill all 256 CUs; workgroups
// stride over row tiles, so a large matrix (lm_head) is one launch.
//
// A generic fallback handles packed rows or x that are not 16-byte aligned.
#include "q8_device.h"
#include "q8_launch.h"

namespace q8 {
namespace {

constexpr int kWaves = 4;               // wavefronts per workgroup
constexpr int kLdsFloats = 16384;       // x staged in LDS up to 64 KiB

template <int G, int KIND, int S, int R, int SPLITK, bool XLDS>
__global__ __launch_bounds__(256) void gemv_kernel(
    const uint8_t *__restrict__ w, int64_t row_bytes, int64_t n,
    const float *__restrict__ x, int64_t m, float *__restrict__ y) {
  extern __shared__ float xs[];
  __shared__ float part[SPLITK > 1 ? SPLITK : 1][R][S];
  constexpr int SB = ScaleTraits<KIND>::bytes;
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int64_t scale_bytes = (m / G) * SB;
  // SPLITK == 1: each wave owns R rows over the whole K range.
  // SPLITK == 4: the 4 waves of a workgroup share R rows, wave w owning the
  // K range [w m/4, (w+1) m/4); partial sums meet in LDS.
  const int64_t k_lo = SPLITK > 1 ? wid * (m / SPLITK) : 0;
  const int64_t k_hi = SPLITK > 1 ? k_lo + m / SPLITK : m;

  const float *xp = x;
  if constexpr (XLDS) {
    const int64_t tot = S * m;   // multiple of 4 (m % 32 == 0)
    for (int64_t i = 4 * threadIdx.x; i < tot; i += 4 * blockDim.x)
      *reinterpret_cast<f32x4 *>(xs + i) = *reinterpret_cast<const f32x4 *>(x + i);
    __syncthreads();
    xp = xs;
  }

  const int64_t rows_per_group = SPLITK > 1 ? R : (int64_t)kWaves * R;
  const int64_t stride_rows = (int64_t)gridDim.x * rows_per_group;
  int64_t r0 = (int64_t)blockIdx.x * rows_per_group + (SPLITK > 1 ? 0 : wid * R);
  for (; r0 < n; r0 += stride_rows) {
    float acc[R][S];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int b = 0; b < S; ++b) acc[r][b] = 0.0f;

    const uint8_t *rowp[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      int64_t j = r0 + r < n ? r0 + r : n - 1;   // clamp: tail rows recompute row n-1
      rowp[r] = w + j * row_bytes;
    }

    for (int64_t k = k_lo + 16 * lane; k < k_hi; k += 1024) {
      u32x4 q[R];
      float sc[R];
#pragma unroll
      for (int r = 0; r < R; ++r)
        q[r] = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4 *>(rowp[r] + scale_bytes + k));
#pragma unroll
      for (int r = 0; r < R; ++r) sc[r] = load_scale<KIND>(rowp[r], k / G);
#pragma unroll
      for (int b = 0; b < S; ++b) {
        const f32x4 *xv4 = reinterpret_cast<const f32x4 *>(xp + b * m + k);
        f32x4 xa = xv4[0], xb = xv4[1], xc = xv4[2], xd = xv4[3];
#pragma unroll
        for (int r = 0; r < R; ++r)
          acc[r][b] = __builtin_fmaf(sc[r], dot16(q[r], xa, xb, xc, xd), acc[r][b]);
      }
    }

    if constexpr (SPLITK == 1) {
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int b = 0; b < S; ++b) {
          float v = wave_sum(acc[r][b]);
          if (lane == 0 && r0 + r < n) y[b * n + r0 + r] = v;
        }
    } else {
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int b = 0; b < S; ++b) {
          float v = wave_sum(acc[r][b]);
          if (lane == 0) part[wid][r][b] = v;
        }
      __syncthreads();
      if (threadIdx.x < R * S) {
        const int r = threadIdx.x / S, b = threadIdx.x % S;
        float v = part[0][r][b];
#pragma unroll
        for (int u = 1; u < SPLITK; ++u) v += part[u][r][b];
        if (r0 + r < n) y[b * n + r0 + r] = v;
      }
      __syncthreads();
    }
  }
}

// Any alignment and either activation dtype: one wavefront per output,
// one code per lane per step.
template <int G, int KIND, bool XBF16>
__global__ __launch_bounds__(256) void gemv_generic_kernel(
    const uint8_t *__restrict__ w, int64_t row_bytes, int64_t n,
    const void *__restrict__ xv, int64_t s, int64_t m, float *__restrict__ y) {
  constexpr int SB = ScaleTraits<KIND>::bytes;
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  const int64_t nw = (int64_t)gridDim.x * kWaves;
  const int64_t scale_bytes = (m / G) * SB;
  for (int64_t task = wave; task < s * n; task += nw) {
    const int64_t b = task / n, j = task - b * n;
    const uint8_t *row = w + j * row_bytes;
    const int8_t *codes = reinterpret_cast<const int8_t *>(row + scale_bytes);
    float acc = 0.0f;
    for (int64_t g = 0; g < m / G; ++g) {
      float p = 0.0f;
      for (int64_t k = g * G + lane; k < (g + 1) * G; k += 64)
      {
        float xk;
        if constexpr (XBF16)
          xk = bf16_bits_to_f32(reinterpret_cast<const uint16_t *>(xv)[b * m + k]);
        else
          xk = reinterpret_cast<const float *>(xv)[b * m + k];
        p = __builtin_fmaf(xk, (float)codes[k], p);
      }
      acc = __builtin_fmaf(load_scale<KIND>(row, g), p, acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) y[b * n + j] = acc;
  }
}

int grid_for(int64_t tiles, int64_t cap) {
  return (int)(tiles < cap ? (tiles > 0 ? tiles : 1) : cap);
}

template <int G, int KIND, int S, int R, int SPLITK>
hipError_t launch_fast(const LinearArgs &a, const float *x, float *y, int64_t cap,
                       hipStream_t st) {
  const int64_t rows_per_group = SPLITK > 1 ? R : kWaves * R;
  const int64_t tiles = (a.n + rows_per_group - 1) / rows_per_group;
  dim3 grid(grid_for(tiles, cap)), block(256);
  if (S * a.m <= kLdsFloats) {
    size_t lds = (size_t)S * a.m * sizeof(float);
    hipLaunchKernelGGL((gemv_kernel<G, KIND, S, R, SPLITK, true>), grid, block, lds, st,
                       a.w, a.row_bytes, a.n, x, a.m, y);
  } else {
    hipLaunchKernelGGL((gemv_kernel<G, KIND, S, R, SPLITK, false>), grid, block, 0, st,
                       a.w, a.row_bytes, a.n, x, a.m, y);
  }
  return hipGetLastError();
}

// Shape classes (tuned on MI355X, decode shapes of Llama-3.2-1B / Qwen3-8B):
//   long rows (m > 4096):         K split over the 4 waves, 4 rows per workgroup
//   vocabulary heads (n >= 64K):  2 rows per wave, up to 8192 workgroups
//   wide (n >= 8192):             4 rows per wave, up to 1024 workgroups
//   small:                        1 row per wave
template <int G, int KIND, int S>
hipError_t launch_rows(const LinearArgs &a, const float *x, float *y, hipStream_t st) {
  if (a.m > 4096 && a.m % 64 == 0) return launch_fast<G, KIND, S, 4, 4>(a, x, y, 1024, st);
  if (a.n >= 65536) return launch_fast<G, KIND, S, 2, 1>(a, x, y, 8192, st);
  if (a.n >= 8192) return launch_fast<G, KIND, S, 4, 1>(a, x, y, 1024, st);
  return launch_fast<G, KIND, S, 1, 1>(a, x, y, 4096, st);
}

template <int G, int KIND>
hipError_t launch_g(const LinearArgs &a, hipStream_t st) {
  const float *x = reinterpret_cast<const float *>(a.x);
  const bool aligned = !a.x_is_bf16 && reinterpret_cast<uintptr_t>(a.w) % 16 == 0 &&
                       a.row_bytes % 16 == 0 &&
                       ((a.m / G) * ScaleTraits<KIND>::bytes) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(x) % 16 == 0;
  if (!aligned) {
    const int64_t tasks = a.s * a.n;
    dim3 grid(grid_for((tasks + kWaves - 1) / kWaves, 4096)), block(256);
    if (a.x_is_bf16)
      hipLaunchKernelGGL((gemv_generic_kernel<G, KIND, true>), grid, block, 0, st,
                         a.w, a.row_bytes, a.n, a.x, a.s, a.m, a.y);
    else
      hipLaunchKernelGGL((gemv_generic_kernel<G, KIND, false>), grid, block, 0, st,
                         a.w, a.row_bytes, a.n, a.x, a.s, a.m, a.y);
    return hipGetLastError();
  }
  // Batches of up to 4 activation rows per pass over the weights.
  for (int64_t b0 = 0; b0 < a.s; b0 += 4) {
    const int64_t sb = a.s - b0 < 4 ? a.s - b0 : 4;
    const float *xb = x + b0 * a.m;
    float *yb = a.y + b0 * a.n;
    hipError_t e;
    switch (sb) {
      case 1: e = launch_rows<G, KIND, 1>(a, xb, yb, st); break;
      case 2: e = launch_rows<G, KIND, 2>(a, xb, yb, st); break;
      case 3: e = launch_rows<G, KIND, 3>(a, xb, yb, st); break;
      default: e = launch_rows<G, KIND, 4>(a, xb, yb, st); break;
    }
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace

hipError_t launch_gemv(const LinearArgs &a, hipStream_t st) {
  if (a.s == 0 || a.n == 0) return hipSuccess;
  if (a.G == 64 && a.kind == SCALE_F16) return launch_g<64, SCALE_F16>(a, st);
  if (a.G == 64 && a.kind == SCALE_F32) return launch_g<64, SCALE_F32>(a, st);
  if (a.G == 32 && a.kind == SCALE_F16) return launch_g<32, SCALE_F16>(a, st);
  if (a.G == 32 && a.kind == SCALE_F32) return launch_g<32, SCALE_F32>(a, st);
  return hipErrorInvalidValue;
}

}  // namespace q8
