// q8_gemv.hip -- decode-path Q8 GEMV for gfx950 (f32 activations, s <= 4 per pass).
//
// y[b, j] = sum_g scale[j, g] * sum_{k in g} x[b, k] * q[j, k]
// (k_mm_q8, src/llama_q8.mojo:54-93: unscaled dot per group, then one scale
// multiply per group).
//
// The kernel is HBM-bound: every weight byte is read exactly once.  Layout
// and mapping:
//   * a wavefront owns R whole rows at a time (or, for rows longer than 4096
//     codes, one K quarter of R rows shared by a group of 4 waves); lane l
//     owns the 16-byte code slices k = 16 l + 1024 i, so each load
//     instruction is one 1 KiB fully coalesced run per row
//     (global_load_dwordx4, non-temporal);
//   * a wave issues a whole chunk of NPF steps of its R rows at once, so it
//     keeps NPF R KiB in flight and waits for each step's loads alone: the
//     dot products of the chunk's early steps overlap the later steps'
//     arrival (the loop over a chunk has no branch, see compute_chunk);
//   * the lane's 16 codes lie inside one quantization group (16 | G), so one
//     scale per row per step is applied after the unscaled 16-term dot;
//   * x (S rows of m f32) is staged once per workgroup in LDS and read with
//     ds_read_b128, or held in registers (a wave K range of at most 2
//     steps); either way its loads are issued before the weights;
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
constexpr int kLdsFloats = 16384;       // fused prologues stage up to 16384 floats of x (80 KiB padded)
// Plain x is staged only up to 32 KiB: a larger stage caps the workgroups
// per CU (160 KiB of LDS) below what the grid needs for one round, and the
// waves read x from L2 just as well.
constexpr int kLdsStageFloats = 8192;
// The fused launches (a prologue or an epilogue) stage x in LDS with 4
// floats of padding after every 16: the 16-float slices that lanes read 64
// bytes apart then start 80 bytes apart, so 8 (or 16) neighbouring lanes'
// 16-byte reads fall on distinct banks (LDS bank-conflict cycles of the 1B
// fused gate|up launch 1.18 M -> 0.39 M; Llama-3.1-8B step 1.958-1.962 ->
// 1.947-1.952 ms, the same bits).  Plain launches keep x dense: there the
// larger stage cost more than the conflicts (Qwen3-8B decode linears
// 1.755 -> 1.777 ms padded, fewer workgroups per CU).
__host__ __device__ constexpr int64_t xs_index(int64_t i) { return (i >> 4) * 20 + (i & 15); }
__host__ __device__ constexpr int64_t xs_floats(int64_t n) { return (n + 15) / 16 * 20; }
constexpr bool x_padded(int pre, int post) { return !(pre == PRE_NONE && post == POST_STORE); }

template <int G, int KIND, int S, int R, int SPLITK, bool XLDS, int PRE = PRE_NONE,
          int POST = POST_STORE, int NPF = 1, int NW = kWaves>
__global__ __launch_bounds__(64 * NW) void gemv_kernel(
    const uint8_t *__restrict__ w, int64_t row_bytes, int64_t n,
    const float *__restrict__ x, int64_t m, float *y, const uint16_t *__restrict__ wn,
    float eps, const float *res, float *__restrict__ amax) {
  extern __shared__ float xs[];
  __shared__ float part[SPLITK > 1 ? NW : 1][R][S];
  __shared__ float red[4];
  static_assert(NW == kWaves || (SPLITK > 1 && NW % SPLITK == 0 && PRE != PRE_RMSNORM),
                "workgroups of more than 4 waves are K-split row groups (no rmsnorm prologue)");
  static_assert(PRE == PRE_NONE || (XLDS && S == 1), "fused prologues stage one x row in LDS");
  static_assert(POST != POST_SWIGLU || (SPLITK == 1 && R % 2 == 0 && S == 1),
                "the swiglu epilogue pairs gate and up rows within a wave");
  static_assert(POST != POST_ARGMAX || (SPLITK == 1 && S == 1),
                "the argmax epilogue keeps whole rows per wave");
  constexpr int SB = ScaleTraits<KIND>::bytes;
  constexpr int NT = 64 * NW;                   // threads
  constexpr bool XPAD = XLDS && x_padded(PRE, POST);   // stage layout: xs_index
  const int lane = threadIdx.x & 63;
  // wave-uniform by construction, so row pointers and K ranges live in
  // scalar registers
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t scale_bytes = (m / G) * SB;
  // SPLITK == 1: each wave owns R rows over the whole K range.
  // SPLITK == 4: each group of 4 waves of a workgroup (NW / 4 groups, one
  // after another) shares R rows, wave w of a group owning the K range
  // [w m/4, (w+1) m/4); partial sums meet in LDS.
  // POST_SWIGLU: a wave's R rows are R/2 gate rows j.. and the matching up
  // rows n/2 + j..; it stores the R/2 outputs silu(gate) * up.
  constexpr int RO = POST == POST_SWIGLU ? R / 2 : R;   // outputs per wave tile
  const int64_t nout = POST == POST_SWIGLU ? n / 2 : n;
  constexpr int RG = SPLITK > 1 ? NW / SPLITK : 1;   // row groups of a K split
  const int rgw = SPLITK > 1 ? wid / SPLITK : 0;      // this wave's row group
  const int64_t rows_per_group = SPLITK > 1 ? (int64_t)RG * RO : (int64_t)NW * RO;
  const int64_t stride_rows = (int64_t)gridDim.x * rows_per_group;
  int64_t r0 = (int64_t)blockIdx.x * rows_per_group + (SPLITK > 1 ? rgw * RO : wid * RO);
  const int64_t k_lo = SPLITK > 1 ? (wid % SPLITK) * (m / SPLITK) : 0;
  const int64_t k_hi = SPLITK > 1 ? k_lo + m / SPLITK : m;
  const int64_t k_first = k_lo + 16 * lane;
  // weight row of slot r for output tile r0 (clamped: tail slots recompute
  // the last row)
  auto row_of = [&](int64_t t0, int r) -> int64_t {
    if constexpr (POST == POST_SWIGLU) {
      const int64_t o = t0 + (r % RO) < nout ? t0 + (r % RO) : nout - 1;
      return r < RO ? o : nout + o;
    } else {
      return t0 + r < n ? t0 + r : n - 1;
    }
  };

  // A wave loads up to NPF steps (1 KiB per row each) of its R rows at once,
  // then computes; NPF covers the wave's whole K range up to 4 steps, so a
  // tile with m / SPLITK <= 4096 waits on memory once.  Steps past the range
  // reload the current step instead of sitting in a branch, so the loads
  // are unconditional and the compiler can wait on each group alone.
  u32x4 q[NPF][R];
  float sc[NPF][R];
  // (kc itself lies past the range only for lanes beyond a row shorter than
  // 1024 codes: those reload the range's first slice, k_lo, which every row
  // has)
  auto load_chunk = [&](const uint8_t *const *rowp, int64_t kc) {
    const int64_t base = kc < k_hi ? kc : k_lo;
#pragma unroll
    for (int p = 0; p < NPF; ++p) {
      const int64_t k = kc + 1024 * p < k_hi ? kc + 1024 * p : base;
#pragma unroll
      for (int r = 0; r < R; ++r)
        q[p][r] = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4 *>(rowp[r] + scale_bytes + k));
#pragma unroll
      for (int r = 0; r < R; ++r) sc[p][r] = load_scale<KIND>(rowp[r], k / G);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  const uint8_t *rowp[R];
#pragma unroll
  for (int r = 0; r < R; ++r) rowp[r] = w + row_of(r0, r) * row_bytes;

  // Load order at the start: loads return in issue order, so x goes first
  // (its first staging batch, or with x read from L2 and one activation row
  // this lane's x slices of the first NPF <= 2 steps, held in registers),
  // then every weight step of the first tile.  Staging x then waits for x
  // alone while the weights are still arriving.
  constexpr int XB = 4;                          // staging batch: 16-byte loads per thread
  constexpr bool XREG = !XLDS && S == 1 && NPF <= 2;
  f32x4 xv[XB], uv[XB];
  uint2 wb[XB];
  f32x4 xr[XREG ? NPF : 1][4];
  const int64_t tot = S * m;                     // multiple of 4 (m % 32 == 0)
  auto load_x = [&](int64_t i0) {
#pragma unroll
    for (int u = 0; u < XB; ++u) {
      const int64_t i = i0 + 4 * NT * u;
      if (i < tot) {
        xv[u] = *reinterpret_cast<const f32x4 *>(x + i);
        if constexpr (PRE == PRE_SWIGLU) uv[u] = *reinterpret_cast<const f32x4 *>(x + m + i);
        if constexpr (PRE == PRE_RMSNORM) wb[u] = *reinterpret_cast<const uint2 *>(wn + i);
      }
    }
  };
  if constexpr (XLDS) load_x(4 * threadIdx.x);
  if constexpr (XREG) {
    const int64_t base = k_first < k_hi ? k_first : k_lo;
#pragma unroll
    for (int p = 0; p < NPF; ++p) {
      const int64_t k = k_first + 1024 * p < k_hi ? k_first + 1024 * p : base;
      const f32x4 *xv4 = reinterpret_cast<const f32x4 *>(x + k);
#pragma unroll
      for (int c = 0; c < 4; ++c) xr[p][c] = xv4[c];
    }
  }
  load_chunk(rowp, k_first);
  // POST_RESIDUAL: the first tile's residual values, loaded after the
  // weights (the store at the end would otherwise wait on one more round
  // trip).  Without a K split lane 0 stores the wave's outputs, so every
  // lane holds them all; with one, thread t < R S stores output (t / S,
  // t % S).  Indices past the outputs are clamped (their stores are
  // skipped).  A residual that is y itself is read before this kernel
  // writes any of it.
  constexpr int RR = POST == POST_RESIDUAL ? (SPLITK > 1 ? 1 : RO * S) : 1;
  float resv[RR] = {};
  if constexpr (POST == POST_RESIDUAL) {
    if constexpr (SPLITK > 1) {
      // thread t < RG R S: row group t / (R S), row (t / S) % R, batch t % S
      const int t = threadIdx.x < RG * R * S ? threadIdx.x : 0;
      const int64_t tr = r0 - rgw * RO + (t / (R * S)) * RO + (t / S) % R;
      const int64_t o = tr < nout ? tr : nout - 1;
      resv[0] = res[(t % S) * n + o];
    } else {
#pragma unroll
      for (int r = 0; r < RO; ++r)
#pragma unroll
        for (int b = 0; b < S; ++b) {
          const int64_t o = r0 + r < nout ? r0 + r : nout - 1;
          resv[r * S + b] = res[b * n + o];
        }
    }
  }
  // Every load above stays ahead of the first use: without this the
  // scheduler sinks weight loads of later steps below the dot products of
  // earlier ones, and fewer bytes are in flight while the first arrive.
  __builtin_amdgcn_sched_barrier(0);

  // PRE_RMSNORM: x is staged as bf16(wn) * x and every output is scaled by
  // 1 / sqrt(mean(x^2) + eps) at the end (W (wn x inv) = inv W (wn x)); the
  // squares are summed from the loaded values, so the norm adds no pass.
  float inv = 1.0f;
  const float *xp = x;
  if constexpr (XLDS) {
    float ss = 0.0f;
    // batches of XB independent 16-byte loads per thread, then the LDS
    // stores (a load-store-load chain would wait on L2 once per step)
    for (int64_t i0 = 4 * threadIdx.x; i0 < tot; i0 += 4 * NT * XB) {
      if (i0 != 4 * threadIdx.x) load_x(i0);     // the first batch is in flight already
#pragma unroll
      for (int u = 0; u < XB; ++u) {
        const int64_t i = i0 + 4 * NT * u;
        if (i >= tot) continue;
        f32x4 o = xv[u];
        if constexpr (PRE == PRE_SWIGLU) {
          // x holds [gate | up]: 2m floats
          const f32x4 gv = xv[u];
          o.x = (gv.x / (1.0f + expf(-gv.x))) * uv[u].x;
          o.y = (gv.y / (1.0f + expf(-gv.y))) * uv[u].y;
          o.z = (gv.z / (1.0f + expf(-gv.z))) * uv[u].z;
          o.w = (gv.w / (1.0f + expf(-gv.w))) * uv[u].w;
        } else if constexpr (PRE == PRE_RMSNORM) {
          const f32x4 v4 = xv[u];
          ss = __builtin_fmaf(v4.x, v4.x, ss);
          ss = __builtin_fmaf(v4.y, v4.y, ss);
          ss = __builtin_fmaf(v4.z, v4.z, ss);
          ss = __builtin_fmaf(v4.w, v4.w, ss);
          o.x = bf16_bits_to_f32(wb[u].x & 0xffffu) * v4.x;
          o.y = bf16_bits_to_f32(wb[u].x >> 16) * v4.y;
          o.z = bf16_bits_to_f32(wb[u].y & 0xffffu) * v4.z;
          o.w = bf16_bits_to_f32(wb[u].y >> 16) * v4.w;
        }
        *reinterpret_cast<f32x4 *>(xs + (XPAD ? xs_index(i) : i)) = o;
      }
    }
    if constexpr (PRE == PRE_RMSNORM) {
      ss = wave_sum(ss);
      if (lane == 0) red[wid] = ss;
    }
    __syncthreads();
    if constexpr (PRE == PRE_RMSNORM)
      inv = 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)m + eps);
    xp = xs;
  }

  // one finished output (value v of tile slot r) -> memory
  // (rv: the prefetched residual, used for the first tile)
  auto store = [&](int64_t t0, int r, int b, float v, float v_up, float rv, bool first_tile) {
    const int64_t o = t0 + r;
    if (o >= nout) return;
    if constexpr (POST == POST_SWIGLU) {
      const float g = inv * v, u = inv * v_up;
      y[o] = (g / (1.0f + expf(-g))) * u;
    } else {
      v = inv * v;
      if constexpr (POST == POST_RESIDUAL) v = (first_tile ? rv : res[b * n + o]) + v;
      y[b * n + o] = v;
    }
  };

  float best_v = -INFINITY;              // POST_ARGMAX: lane 0's best row so far
  int best_i = INT32_MAX;

  // The dot products of one chunk of NPF steps starting at the
  // wave-uniform kw (each lane adds its own offset), from the loads in q
  // and sc.  No step sits in a branch: a lane whose step lies past the
  // range reads a valid x slice and keeps its sum (a select), so the
  // compiler waits for each step's loads alone and the dot products of
  // early steps overlap the loads still in flight (a branch here made
  // every wave wait for all of its loads, and with x read from L2 inside
  // it, for one more round trip per step).
  const int64_t kx_safe = k_first < k_hi ? k_first : k_lo;
  auto compute_chunk = [&](int64_t kw, float (&acc)[R][S]) {
    const int64_t kc = kw + 16 * lane;
#pragma unroll
    for (int p = 0; p < NPF; ++p) {
      const int64_t k = kc + 1024 * p;
      const bool live = k < k_hi;
      const int64_t kx = live ? k : kx_safe;
#pragma unroll
      for (int b = 0; b < S; ++b) {
        f32x4 xa, xb, xc, xd;
        if (XREG && kw == k_lo) {
          xa = xr[XREG ? p : 0][0];
          xb = xr[XREG ? p : 0][1];
          xc = xr[XREG ? p : 0][2];
          xd = xr[XREG ? p : 0][3];
        } else {
          const f32x4 *xv4 = reinterpret_cast<const f32x4 *>(
              xp + (XPAD ? xs_index(b * m + kx) : b * m + kx));
          xa = xv4[0];
          xb = xv4[1];
          xc = xv4[2];
          xd = xv4[3];
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const float t = __builtin_fmaf(sc[p][r], dot16(q[p][r], xa, xb, xc, xd), acc[r][b]);
          acc[r][b] = live ? t : acc[r][b];
        }
      }
    }
  };

  // A finished tile: wave sums, the K split's partials met in LDS, the
  // epilogue.
  auto finish_tile = [&](int64_t t0, const float (&acc)[R][S], bool first_tile) {
    if constexpr (SPLITK == 1) {
      float v[R][S];
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int b = 0; b < S; ++b) v[r][b] = wave_sum(acc[r][b]);
      if (lane == 0) {
#pragma unroll
        for (int r = 0; r < RO; ++r)
#pragma unroll
          for (int b = 0; b < S; ++b)
            store(t0, r, b, v[r][b], POST == POST_SWIGLU ? v[(r + RO) % R][b] : 0.0f,
                  resv[POST == POST_RESIDUAL ? r * S + b : 0], first_tile);
        if constexpr (POST == POST_ARGMAX) {
          // rows in increasing order, strict >: the lowest row among equal
          // values; NaN never wins
#pragma unroll
          for (int r = 0; r < R; ++r) {
            const float yv = inv * v[r][0];
            if (t0 + r < n && yv > best_v) {
              best_v = yv;
              best_i = (int)(t0 + r);
            }
          }
        }
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
      if (threadIdx.x < RG * R * S) {
        const int g = threadIdx.x / (R * S), r = (threadIdx.x / S) % R, b = threadIdx.x % S;
        float v = part[g * SPLITK][r][b];
#pragma unroll
        for (int u = 1; u < SPLITK; ++u) v += part[g * SPLITK + u][r][b];
        store(t0 - rgw * RO + g * RO, r, b, v, 0.0f, resv[0], first_tile);
      }
      __syncthreads();
    }
  };

  // The first tile's first chunk was loaded before x was staged; it is
  // consumed in straight-line code, with no branch between those loads and
  // their use (a wave whose first tile lies past the outputs computes on
  // the clamped rows it loaded and stores nothing), and every wave reaches
  // the barriers of finish_tile.
  {
    float acc[R][S];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int b = 0; b < S; ++b) acc[r][b] = 0.0f;
    compute_chunk(k_lo, acc);
    for (int64_t kw = k_lo + 1024 * NPF; kw < k_hi; kw += 1024 * NPF) {
      load_chunk(rowp, kw + 16 * lane);
      compute_chunk(kw, acc);
    }
    finish_tile(r0, acc, true);
  }
  for (r0 += stride_rows; r0 < nout; r0 += stride_rows) {
#pragma unroll
    for (int r = 0; r < R; ++r) rowp[r] = w + row_of(r0, r) * row_bytes;
    float acc[R][S];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int b = 0; b < S; ++b) acc[r][b] = 0.0f;
    for (int64_t kw = k_lo; kw < k_hi; kw += 1024 * NPF) {
      load_chunk(rowp, kw + 16 * lane);
      compute_chunk(kw, acc);
    }
    finish_tile(r0, acc, false);
  }
  if constexpr (POST == POST_ARGMAX) {
    __shared__ float bv[kWaves];
    __shared__ int bi[kWaves];
    if (lane == 0) {
      bv[wid] = best_v;
      bi[wid] = best_i;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      float b = bv[0];
      int i = bi[0];
      for (int u = 1; u < kWaves; ++u)
        if (bv[u] > b || (bv[u] == b && bi[u] < i)) {
          b = bv[u];
          i = bi[u];
        }
      amax[blockIdx.x] = b;
      reinterpret_cast<int *>(amax)[gridDim.x + blockIdx.x] = i;
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

// NPF: K steps in flight per wave.  Batches of 2-4 rows (the unaligned
// fallback) keep one step for waves of 2+ rows (registers against
// occupancy).  One activation row puts the wave's whole K range in flight,
// up to 4 steps (2 or 4, by the range): every wave waits on memory once, so
// the weights stream at full rate from the start instead of in two waves of
// requests (gate|up 2048 -> 16384: first step's data in 3.4 us per wave,
// then the second step's round trip).
template <int R, int S> constexpr int npf_for() { return R * S >= 4 ? 1 : 4; }

inline bool two_steps(int64_t m, int splitk) { return m / splitk <= 2048; }

template <int G, int KIND, int S, int R, int SPLITK, int NPF, int NW = kWaves>
hipError_t launch_fast_t(const LinearArgs &a, const float *x, float *y, int64_t cap,
                         hipStream_t st) {
  const int64_t rows_per_group = SPLITK > 1 ? (int64_t)(NW / SPLITK) * R : (int64_t)NW * R;
  const int64_t tiles = (a.n + rows_per_group - 1) / rows_per_group;
  dim3 grid(grid_for(tiles, cap)), block(64 * NW);
  // x staged in LDS for rows up to the stage limit (and always in the
  // workgroups of K-split row groups), except when each lane's x slices fit
  // in registers (one activation row, a wave K range of at most 2 steps):
  // those are loaded before the weights and need no stage or barrier (the
  // 8192 x 2048 linear: 6.40 -> 5.82 us)
  const bool xreg = NW == kWaves && S == 1 && NPF <= 2 && a.m / SPLITK <= 1024 * NPF;
  if ((NW > kWaves || S * a.m <= kLdsStageFloats) && !xreg) {
    size_t lds = (size_t)S * a.m * sizeof(float);
    hipLaunchKernelGGL((gemv_kernel<G, KIND, S, R, SPLITK, true, PRE_NONE, POST_STORE, NPF, NW>),
                       grid, block, lds, st, a.w, a.row_bytes, a.n, x, a.m, y, nullptr, 0.0f,
                       nullptr, nullptr);
  } else if constexpr (NW == kWaves) {
    hipLaunchKernelGGL((gemv_kernel<G, KIND, S, R, SPLITK, false, PRE_NONE, POST_STORE, NPF>),
                       grid, block, 0, st, a.w, a.row_bytes, a.n, x, a.m, y, nullptr, 0.0f,
                       nullptr, nullptr);
  }
  return hipGetLastError();
}

template <int G, int KIND, int S, int R, int SPLITK>
hipError_t launch_fast(const LinearArgs &a, const float *x, float *y, int64_t cap,
                       hipStream_t st) {
  if constexpr (S == 1) {
    if (two_steps(a.m, SPLITK)) return launch_fast_t<G, KIND, S, R, SPLITK, 2>(a, x, y, cap, st);
    return launch_fast_t<G, KIND, S, R, SPLITK, 4>(a, x, y, cap, st);
  } else {
    return launch_fast_t<G, KIND, S, R, SPLITK, npf_for<R, S>()>(a, x, y, cap, st);
  }
}

// Long rows at one activation row and at least 4096 outputs: the K split
// over 4 waves, in workgroups of 4 row groups (16 waves, 16 rows, one
// workgroup per CU at 4096 rows) that stage x once in LDS with one batch of
// loads issued ahead of the weights, so x is read from LDS independently of
// the weights' arrival and fetched once per 16 rows instead of once per 4
// from L2.  Each wave streams its K range in chunks of 2 steps: the second
// chunk's loads go out while the first chunk's dot products run (the
// Llama-3.1-8B down projection 14336 -> 4096: 16.0 us with 4 rows per
// workgroup and x from L2, 17.2 with 16 waves and 4-step chunks, 13.5 with
// 2-step chunks; Qwen3-8B 12288 -> 4096 14.8 -> 13.3 us).  Fewer outputs
// keep the 4-wave workgroups (with 8 waves the 1B down projection ran 6.0
// against 5.9 us).  The stage holds m floats.
inline bool long_row_groups(const LinearArgs &a) {
  return a.s == 1 && a.m <= kLdsFloats && a.n >= 4096;
}

// Shape classes (tuned on MI355X, decode shapes of Llama-3.2-1B / Qwen3-8B):
//   long rows (m > 4096):         K split over the 4 waves, 4 rows per workgroup
//   vocabulary heads (n >= 64K):  2 rows per wave, up to 8192 workgroups
//   one row, n >= 16384:          2 rows per wave, up to 2048 workgroups
//   wide (n >= 8192):             4 rows per wave, up to 1024 workgroups
//   one row, n >= 4096:           2 rows per wave
//   small:                        1 row per wave
template <int G, int KIND, int S>
hipError_t launch_rows(const LinearArgs &a, const float *x, float *y, hipStream_t st) {
  if (a.m > 4096 && a.m % 64 == 0) {
    if constexpr (S == 1) {
      if (long_row_groups(a)) return launch_fast_t<G, KIND, S, 4, 4, 2, 16>(a, x, y, 256, st);
    }
    return launch_fast<G, KIND, S, 4, 4>(a, x, y, 1024, st);
  }
  // vocabulary heads: one K step in flight per wave (more waves per CU; the
  // 8192 workgroups walk about two row tiles each, so occupancy, not one
  // round of loads, covers the latency: 2 steps made the 1B lm_head 42 ->
  // 47 us)
  if (a.n >= 65536) return launch_fast_t<G, KIND, S, 2, 1, 1>(a, x, y, 8192, st);
  // one row, 16384 .. 65535 outputs: 2 rows per wave, up to 2048 workgroups
  // (Qwen3-8B gate|up 4096 -> 24576: its decode-linears step 1.762 -> 1.750
  // ms; the 8192 x 2048 linear keeps 4 rows, 2 were 0.4-1.1 % slower)
  if (S == 1 && a.n >= 16384) return launch_fast<G, KIND, S, 2, 1>(a, x, y, 2048, st);
  if (a.n >= 8192) return launch_fast<G, KIND, S, 4, 1>(a, x, y, 1024, st);
  // one row, 4096 .. 8191 outputs: 2 rows per wave (Qwen3-8B o and q|k|v)
  if (S == 1 && a.n >= 4096) return launch_fast<G, KIND, S, 2, 1>(a, x, y, 2048, st);
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

template <int G, int KIND, int R, int SPLITK, int PRE, int POST, int NPF, int NW = kWaves>
hipError_t launch_fused_npf(const FusedLinearArgs &f, int64_t cap, hipStream_t st) {
  const LinearArgs &a = f.lin;
  constexpr int RO = POST == POST_SWIGLU ? R / 2 : R;
  const int64_t nout = POST == POST_SWIGLU ? a.n / 2 : a.n;
  const int64_t rows_per_group = SPLITK > 1 ? (int64_t)(NW / SPLITK) * RO : (int64_t)NW * RO;
  const int64_t tiles = (nout + rows_per_group - 1) / rows_per_group;
  dim3 grid(grid_for(tiles, cap)), block(64 * NW);
  const float *x = reinterpret_cast<const float *>(a.x);
  // x read from L2 by every wave past the stage limit, and held in
  // registers (loaded before the weights) when a wave's K range is at most
  // 2 steps: the stage and its barrier cost more than they save (Qwen3-0.6B
  // o projection: step 0.741 -> 0.737 ms).  The fused prologues keep the
  // LDS stage: whole rows in every wave's registers (m <= 2048) made the
  // 1B gate|up 8.57 -> 11.0 us (registers past one round of workgroups,
  // and x and the norm weights fetched per wave instead of per workgroup).
  if (f.grid_out) *f.grid_out = (int)grid.x;
  if constexpr (PRE == PRE_NONE && NW == kWaves) {
    if (a.m > kLdsStageFloats || (NPF <= 2 && a.m / SPLITK <= 1024 * NPF)) {
      hipLaunchKernelGGL((gemv_kernel<G, KIND, 1, R, SPLITK, false, PRE, POST, NPF>), grid, block,
                         0, st, a.w, a.row_bytes, a.n, x, a.m, a.y, f.wn, f.eps, f.res, f.part);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((gemv_kernel<G, KIND, 1, R, SPLITK, true, PRE, POST, NPF, NW>), grid, block,
                     (size_t)(x_padded(PRE, POST) ? xs_floats(a.m) : a.m) * sizeof(float), st,
                     a.w, a.row_bytes, a.n, x, a.m, a.y, f.wn,
                     f.eps, f.res, f.part);
  return hipGetLastError();
}

template <int G, int KIND, int R, int SPLITK, int PRE, int POST>
hipError_t launch_fused_t(const FusedLinearArgs &f, int64_t cap, hipStream_t st) {
  if (two_steps(f.lin.m, SPLITK)) return launch_fused_npf<G, KIND, R, SPLITK, PRE, POST, 2>(f, cap, st);
  return launch_fused_npf<G, KIND, R, SPLITK, PRE, POST, 4>(f, cap, st);
}

// Shape classes as launch_rows; the swiglu epilogue keeps whole rows per
// wave (gate and up rows of one output in the same wave).
template <int G, int KIND, int PRE, int POST>
hipError_t launch_fused_rows(const FusedLinearArgs &f, hipStream_t st) {
  const LinearArgs &a = f.lin;
  if constexpr (POST == POST_SWIGLU) {
    // one gate and one up row per wave (the 1B gate|up: step 0.5309 ->
    // 0.5276 ms against 2 + 2 rows per wave, with every K step in flight)
    if (a.n >= 8192) return launch_fused_t<G, KIND, 2, 1, PRE, POST>(f, 2048, st);
    return launch_fused_t<G, KIND, 2, 1, PRE, POST>(f, 4096, st);
  } else if constexpr (POST == POST_ARGMAX) {
    // whole rows per wave; the grid stays within kArgmaxMaxBlocks partials
    if (a.n >= 65536) return launch_fused_npf<G, KIND, 2, 1, PRE, POST, 1>(f, 8192, st);
    return launch_fused_t<G, KIND, 1, 1, PRE, POST>(f, 4096, st);
  } else {
    if (a.m > 4096 && a.m % 64 == 0) {
      // (a swiglu prologue stages [gate | up]: its registers do not fit the
      // 16-wave workgroups, and the decode step never uses it on long rows)
      if constexpr (PRE == PRE_NONE) {
        if (long_row_groups(a)) return launch_fused_npf<G, KIND, 4, 4, PRE, POST, 2, 16>(f, 256, st);
      }
      return launch_fused_t<G, KIND, 4, 4, PRE, POST>(f, 1024, st);
    }
    if (a.n >= 65536) return launch_fused_npf<G, KIND, 2, 1, PRE, POST, 1>(f, 8192, st);
    if (a.n >= 8192) return launch_fused_t<G, KIND, 4, 1, PRE, POST>(f, 1024, st);
    // 2 rows per wave from 4096 rows (Llama-3.1-8B q|k|v and o: step
    // 2.308 -> 2.238 ms)
    if (a.n >= 4096) return launch_fused_t<G, KIND, 2, 1, PRE, POST>(f, 2048, st);
    return launch_fused_t<G, KIND, 1, 1, PRE, POST>(f, 4096, st);
  }
}

template <int G, int KIND, int PRE>
hipError_t launch_fused_pre(const FusedLinearArgs &f, hipStream_t st) {
  if (f.post == POST_STORE) return launch_fused_rows<G, KIND, PRE, POST_STORE>(f, st);
  if (f.post == POST_RESIDUAL) return launch_fused_rows<G, KIND, PRE, POST_RESIDUAL>(f, st);
  if (f.post == POST_SWIGLU) return launch_fused_rows<G, KIND, PRE, POST_SWIGLU>(f, st);
  if (f.post == POST_ARGMAX) return launch_fused_rows<G, KIND, PRE, POST_ARGMAX>(f, st);
  return hipErrorInvalidValue;
}

template <int G, int KIND>
hipError_t launch_fused_g(const FusedLinearArgs &f, hipStream_t st) {
  if (f.pre == PRE_NONE) return launch_fused_pre<G, KIND, PRE_NONE>(f, st);
  if (f.pre == PRE_RMSNORM) return launch_fused_pre<G, KIND, PRE_RMSNORM>(f, st);
  if (f.pre == PRE_SWIGLU) return launch_fused_pre<G, KIND, PRE_SWIGLU>(f, st);
  return hipErrorInvalidValue;
}

}  // namespace

bool gemv_fused_supported(const FusedLinearArgs &f) {
  const LinearArgs &a = f.lin;
  const int pre = f.pre, post = f.post;
  const int sb = a.kind == SCALE_F16 ? 2 : 4;
  if (pre == PRE_RMSNORM && reinterpret_cast<uintptr_t>(f.wn) % 8 != 0) return false;
  return a.s == 1 && !a.x_is_bf16 && (pre == PRE_NONE || a.m <= kLdsFloats) && a.m % 32 == 0 &&
         (a.G == 32 || a.G == 64) && reinterpret_cast<uintptr_t>(a.w) % 16 == 0 &&
         a.row_bytes % 16 == 0 && ((a.m / a.G) * sb) % 16 == 0 &&
         reinterpret_cast<uintptr_t>(a.x) % 16 == 0 && pre >= PRE_NONE && pre <= PRE_SWIGLU &&
         post >= POST_STORE && post <= POST_ARGMAX && (post != POST_SWIGLU || a.n % 2 == 0) &&
         (post != POST_ARGMAX || a.n <= INT32_MAX);
}

hipError_t launch_gemv_fused(const FusedLinearArgs &f, hipStream_t st) {
  const LinearArgs &a = f.lin;
  if (!gemv_fused_supported(f) || (f.post == POST_ARGMAX && !f.part)) return hipErrorInvalidValue;
  if (a.n == 0) return hipSuccess;
  if (a.G == 64 && a.kind == SCALE_F16) return launch_fused_g<64, SCALE_F16>(f, st);
  if (a.G == 64 && a.kind == SCALE_F32) return launch_fused_g<64, SCALE_F32>(f, st);
  if (a.G == 32 && a.kind == SCALE_F16) return launch_fused_g<32, SCALE_F16>(f, st);
  if (a.G == 32 && a.kind == SCALE_F32) return launch_fused_g<32, SCALE_F32>(f, st);
  return hipErrorInvalidValue;
}

hipError_t launch_gemv(const LinearArgs &a, hipStream_t st) {
  if (a.s == 0 || a.n == 0) return hipSuccess;
  if (a.G == 64 && a.kind == SCALE_F16) return launch_g<64, SCALE_F16>(a, st);
  if (a.G == 64 && a.kind == SCALE_F32) return launch_g<64, SCALE_F32>(a, st);
  if (a.G == 32 && a.kind == SCALE_F16) return launch_g<32, SCALE_F16>(a, st);
  if (a.G == 32 && a.kind == SCALE_F32) return launch_g<32, SCALE_F32>(a, st);
  return hipErrorInvalidValue;
}

}  // namespace q8
