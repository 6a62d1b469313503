// q8_gemm.hip -- prefill-path Q8 GEMM on gfx950 bf16 MFMA.
//
// y[i, j] = sum_g scale[j, g] * sum_{k in g} x[i, k] * q[j, k]
// (k_mm_q8's arithmetic, src/llama_q8.mojo:73-84: unscaled dot per group,
// one scale multiply per group) computed as a tiled GEMM on
// v_mfma_f32_32x32x16_bf16:
//   * |q| <= 127 is exact in bf16 and a bf16 x bf16 product is exact in the
//     f32 accumulator, so each group's partial dot is exact up to f32
//     accumulation; every group's partial starts from 0 in its own MFMA
//     accumulator and is folded into the result with one v_fma per output;
//   * f32 activations (the W8A32 path with many rows) are split into
//     hi = bf16(x) and lo = bf16(x - hi) and run as two MFMAs; the residual
//     error is below 2^-17 |x|.
//
// Work decomposition (one 512-thread workgroup per BM x 128 output tile):
//   * the 8 waves form 4 column slices of 32 outputs x 2 K-parities; wave
//     (p, h) accumulates columns p*32.. over the 64-code K slots of parity h,
//     so each SIMD runs two independent instruction streams whose MFMA and
//     VALU work co-issue; the two parities meet in LDS at the end;
//   * a wave's weight codes never touch LDS: lane l owns output column
//     l % 32 and loads its 32 codes of a slot straight from HBM into
//     registers (two dwordx4), converted to bf16 in registers.  The MFMA K
//     order inside a slot is permuted so each lane's codes come in two
//     16-byte chunks and no k-step straddles a quantization group; the
//     activation fragments read from LDS use the same permutation;
//   * activations are staged through double-buffered LDS, 128 k per step;
//   * both the weight and activation loads run in register rings several
//     K steps ahead, with the loop unrolled so ring slots are compile-time
//     registers (a runtime slot index would force the loads to complete
//     immediately).
#include "q8_device.h"
#include "q8_launch.h"

namespace q8 {
namespace {

constexpr int NT = 512;        // 8 waves
constexpr int BN = 128;        // 4 column slices of 32
constexpr int KT = 128;        // k per iteration = 2 slots of 64 codes
constexpr int LDA = KT + 8;    // bf16 per LDS row (16-byte pad)

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

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

// Raw scale bits of one 64-code slot: G=64 -> 1 scale, G=32 -> 2 scales.
template <int G, int KIND> struct SlotScale;
template <> struct SlotScale<64, SCALE_F16> {
  typedef uint16_t raw;
  static __device__ __forceinline__ raw load(const uint8_t *row, int64_t slot) {
    return *reinterpret_cast<const uint16_t *>(row + 2 * slot);
  }
  static __device__ __forceinline__ float get(raw r, int) { return f16_bits_to_f32(r); }
};
template <> struct SlotScale<64, SCALE_F32> {
  typedef uint32_t raw;
  static __device__ __forceinline__ raw load(const uint8_t *row, int64_t slot) {
    const uint16_t *p = reinterpret_cast<const uint16_t *>(row + 4 * slot);
    return (uint32_t)p[0] | ((uint32_t)p[1] << 16);
  }
  static __device__ __forceinline__ float get(raw r, int) { return __builtin_bit_cast(float, r); }
};
template <> struct SlotScale<32, SCALE_F16> {
  typedef uint32_t raw;   // two binary16, 2-byte aligned
  static __device__ __forceinline__ raw load(const uint8_t *row, int64_t slot) {
    const uint16_t *p = reinterpret_cast<const uint16_t *>(row + 4 * slot);
    return (uint32_t)p[0] | ((uint32_t)p[1] << 16);
  }
  static __device__ __forceinline__ float get(raw r, int gi) {
    return f16_bits_to_f32((uint16_t)(gi ? r >> 16 : r));
  }
};
template <> struct SlotScale<32, SCALE_F32> {
  typedef u32x2 raw;      // two f32, 2-byte aligned
  static __device__ __forceinline__ raw load(const uint8_t *row, int64_t slot) {
    const uint16_t *p = reinterpret_cast<const uint16_t *>(row + 8 * slot);
    return u32x2{(uint32_t)p[0] | ((uint32_t)p[1] << 16), (uint32_t)p[2] | ((uint32_t)p[3] << 16)};
  }
  static __device__ __forceinline__ float get(raw r, int gi) {
    return __builtin_bit_cast(float, gi ? r.y : r.x);
  }
};

template <int G, int KIND, bool XF32, int BM, int PB, int PA>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(2, 2)))
void gemm_kernel(const uint8_t *__restrict__ w, int64_t row_bytes, const void *__restrict__ xv,
                 float *__restrict__ y, int64_t s, int64_t m, int64_t n, int nit,
                 float *__restrict__ ws) {
  // blockIdx.z selects a K range of nit iterations (split-K): with
  // gridDim.z == 1 y is written directly, otherwise split z writes its
  // partial sums to ws[z] and splitk_reduce_kernel adds them up.
  const int it0 = (int)blockIdx.z * nit;
  constexpr int SB = ScaleTraits<KIND>::bytes;
  constexpr int TM = BM / 32;                 // 32-row MFMA tiles per wave
  constexpr int AU = BM * KT / 8 / NT;        // activation chunks (8 elements) per thread
  constexpr int P = PB > PA ? PB : PA;        // unroll period
  static_assert(P % PB == 0 && P % PA == 0, "ring depths must divide the period");
  typedef SlotScale<G, KIND> SS;
  constexpr int NLDS = XF32 ? 2 : 1;
  __shared__ __attribute__((aligned(16))) uint16_t As[2][NLDS][BM * LDA];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int p = wid & 3, h = wid >> 2;
  const int lr = lane & 31, lh = lane >> 5;
  const int64_t m0 = (int64_t)blockIdx.y * BM;
  const int64_t col = (int64_t)blockIdx.x * BN + p * 32 + lr;
  const uint8_t *wrow0 = w + (col < n ? col : n - 1) * row_bytes;   // clamped: loads stay in bounds
  // Everything below is relative to this split's first K slot: codes and
  // scales are addressed from shifted row pointers, activations from a
  // shifted column, and mk / nslot / ngroups count what is left of the row.
  const int64_t kbase = (int64_t)it0 * KT;
  const uint8_t *codes = wrow0 + (m / G) * SB + kbase;
  const uint8_t *wrow = wrow0 + (2 * (int64_t)it0) * (64 / G) * SB;
  const int64_t mk = m - kbase;
  const int64_t nslot = (mk + 63) / 64;
  const int64_t ngroups = m / G - 2 * (int64_t)it0 * (64 / G);

  // activation chunk coordinates (iteration-independent rows)
  int64_t arow[AU];
  bool arow_ok[AU];
  int akc[AU];
#pragma unroll
  for (int u = 0; u < AU; ++u) {
    const int c = tid + NT * u;
    const int row = c / (KT / 8);
    akc[u] = (c % (KT / 8)) * 8;
    arow_ok[u] = m0 + row < s;
    arow[u] = m0 + row < s ? m0 + row : s - 1;
  }

  f32x16 acc[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[i][v] = 0.0f;

  u32x4 qb[PB][2];
  typename SS::raw sr[PB];
  u32x4 ra[PA][XF32 ? 2 * AU : AU];

  // Codes of one 64-code slot held by a lane, as two 16-code chunks.  The
  // MFMA K order inside a slot is chosen so each k-step of 16 stays inside
  // one quantization group: k-step t of lane half lh reads codes
  //   G=64: [32 lh + 8 t, +8)                       (chunks at 32 lh, 32 lh + 16)
  //   G=32: [32 (t / 2) + 16 lh + 8 (t % 2), +8)     (chunks at 16 lh, 32 + 16 lh)
  // so t = 0..1 covers the slot's first group of 32 and t = 2..3 its second.
  const int chunk0 = G == 64 ? 32 * lh : 16 * lh;
  const int chunk1 = G == 64 ? 32 * lh + 16 : 32 + 16 * lh;
  auto load_b = [&](u32x4 (&q)[2], typename SS::raw &r, int it) {
    int slot = 2 * it + h;
    slot = slot < nslot ? slot : (int)nslot - 1;
    // the last slot of a G=32 row may hold only 32 codes: never read past the row
    int o0 = slot * 64 + chunk0, o1 = slot * 64 + chunk1;
    o0 = o0 + 16 <= mk ? o0 : (int)mk - 16;
    o1 = o1 + 16 <= mk ? o1 : (int)mk - 16;
    q[0] = *reinterpret_cast<const u32x4 *>(codes + o0);
    q[1] = *reinterpret_cast<const u32x4 *>(codes + o1);
    // reads the slot's scale(s); a missing second G=32 scale reads the first
    // code bytes of the row (in bounds) and is replaced by 0 below
    r = SS::load(wrow, slot);
  };
  auto load_a = [&](u32x4 *dst, int it) {
#pragma unroll
    for (int u = 0; u < AU; ++u) {
      int k = it * KT + akc[u];
      k = k < mk ? k : (int)mk - 8;
      if constexpr (!XF32) {
        const uint16_t *x = reinterpret_cast<const uint16_t *>(xv) + kbase;
        dst[u] = *reinterpret_cast<const u32x4 *>(x + arow[u] * m + k);
      } else {
        const float *x = reinterpret_cast<const float *>(xv) + kbase;
        const u32x4 *pp = reinterpret_cast<const u32x4 *>(x + arow[u] * m + k);
        dst[2 * u] = pp[0];
        dst[2 * u + 1] = pp[1];
      }
    }
  };
  auto store_a = [&](const u32x4 *src, int buf, int it) {
#pragma unroll
    for (int u = 0; u < AU; ++u) {
      const int c = tid + NT * u;
      const int row = c / (KT / 8);
      const bool ok = arow_ok[u] && it * KT + akc[u] < mk;
      if constexpr (!XF32) {
        const u32x4 v = ok ? src[u] : u32x4{0u, 0u, 0u, 0u};
        *reinterpret_cast<u32x4 *>(&As[buf][0][row * LDA + akc[u]]) = v;
      } else {
        const uint32_t d[8] = {src[2 * u].x, src[2 * u].y, src[2 * u].z, src[2 * u].w,
                               src[2 * u + 1].x, src[2 * u + 1].y, src[2 * u + 1].z,
                               src[2 * u + 1].w};
        uint32_t hi[4], lo[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float f0 = ok ? __builtin_bit_cast(float, d[2 * e]) : 0.0f;
          const float f1 = ok ? __builtin_bit_cast(float, d[2 * e + 1]) : 0.0f;
          const uint32_t h0 = bf16_rne(f0), h1 = bf16_rne(f1);
          const uint32_t l0 = bf16_rne(f0 - __builtin_bit_cast(float, h0 << 16));
          const uint32_t l1 = bf16_rne(f1 - __builtin_bit_cast(float, h1 << 16));
          hi[e] = h0 | (h1 << 16);
          lo[e] = l0 | (l1 << 16);
        }
        *reinterpret_cast<u32x4 *>(&As[buf][0][row * LDA + akc[u]]) = u32x4{hi[0], hi[1], hi[2], hi[3]};
        *reinterpret_cast<u32x4 *>(&As[buf][1][row * LDA + akc[u]]) = u32x4{lo[0], lo[1], lo[2], lo[3]};
      }
    }
  };

#pragma unroll
  for (int q = 0; q < PB; ++q) load_b(qb[q], sr[q], q < nit ? q : nit - 1);
  // Activation tile t lives in ring slot t % PA: tile 0 is staged first,
  // then the ring is primed with tiles 1 .. PA.
  load_a(ra[0], 0);
  store_a(ra[0], 0, 0);
#pragma unroll
  for (int q = 1; q <= PA; ++q) load_a(ra[q % PA], q < nit ? q : nit - 1);
  __syncthreads();

  for (int i0 = 0; i0 < nit; i0 += P) {
#pragma unroll
    for (int j = 0; j < P; ++j) {
      const int it = i0 + j;
      const int buf = it & 1;
      const int bs = j % PB;
      bf16x8_t bf[4];
      bf[0] = codes_to_bf16(qb[bs][0].x, qb[bs][0].y);
      bf[1] = codes_to_bf16(qb[bs][0].z, qb[bs][0].w);
      bf[2] = codes_to_bf16(qb[bs][1].x, qb[bs][1].y);
      bf[3] = codes_to_bf16(qb[bs][1].z, qb[bs][1].w);
      // a slot beyond the last real one carries zero activations; its scale
      // is forced to 0 as well (its codes are a clamped re-read)
      const int slot = 2 * it + h;
      const bool live = slot < nslot;
      const float sc0 = live ? SS::get(sr[bs], 0) : 0.0f;
      const float sc1 = (G == 32 && 2 * slot + 1 < ngroups) ? SS::get(sr[bs], 1) : 0.0f;
      load_b(qb[bs], sr[bs], it + PB < nit ? it + PB : nit - 1);

      const uint16_t *A0 = As[buf][0];
      // activation column of k-step t (same permutation as the codes)
      auto acol = [&](int t) {
        return 64 * h + (G == 64 ? 32 * lh + 8 * t : 32 * (t >> 1) + 16 * lh + 8 * (t & 1));
      };
      // The TM row tiles of a group run as TM / TH passes of TH independent
      // MFMA chains: TH = 2 keeps the per-group temporaries at 32 VGPRs so
      // 128-row tiles fit the 256-VGPR budget of two waves per SIMD.
      constexpr int TH = TM < 2 ? TM : 2;
#pragma unroll
      for (int i0 = 0; i0 < TM; i0 += TH) {
        f32x16 tmp[TH];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          bf16x8_t af[TH], al[TH];
#pragma unroll
          for (int ii = 0; ii < TH; ++ii) {
            af[ii] = *reinterpret_cast<const bf16x8_t *>(&A0[((i0 + ii) * 32 + lr) * LDA + acol(t)]);
            if constexpr (XF32)
              al[ii] = *reinterpret_cast<const bf16x8_t *>(
                  &As[buf][XF32 ? 1 : 0][((i0 + ii) * 32 + lr) * LDA + acol(t)]);
          }
          // G=64: one group over t = 0..3; G=32: groups t = 0..1 and 2..3
          const bool fresh = (t == 0) || (G == 32 && t == 2);
#pragma unroll
          for (int ii = 0; ii < TH; ++ii) {
            if (fresh) {
              const f32x16 z = {};
              tmp[ii] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[ii], bf[t], z, 0, 0, 0);
            } else {
              tmp[ii] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[ii], bf[t], tmp[ii], 0, 0, 0);
            }
            if constexpr (XF32)
              tmp[ii] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[ii], bf[t], tmp[ii], 0, 0, 0);
          }
          if ((G == 32 && t == 1) || t == 3) {
            const float sc = (G == 32 && t == 1) ? sc0 : (G == 32 ? sc1 : sc0);
#pragma unroll
            for (int ii = 0; ii < TH; ++ii)
#pragma unroll
              for (int v = 0; v < 16; ++v)
                acc[i0 + ii][v] = __builtin_fmaf(sc, tmp[ii][v], acc[i0 + ii][v]);
          }
        }
      }
      store_a(ra[(j + 1) % PA], buf ^ 1, it + 1);
      __syncthreads();
      load_a(ra[(j + 1) % PA], it + 1 + PA < nit ? it + 1 + PA : nit - 1);
    }
  }

  // The two K parities of each column slice meet in LDS (reusing As).
  float *red = reinterpret_cast<float *>(&As[0][0][0]);   // 4 * TM * 16 * 64 floats
  static_assert(4 * TM * 16 * 64 * 4 <= (int)sizeof(As), "reduction buffer too small");
  __syncthreads();
  if (h == 1) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) red[((p * TM + i) * 16 + v) * 64 + lane] = acc[i][v];
  }
  __syncthreads();
  const int splits = (int)gridDim.z;
  if (h == 0 && col < n) {
    // D layout of v_mfma_f32_32x32x16: lane -> column lane % 32,
    // element v -> row 8 (v / 4) + 4 (lane / 32) + v % 4.
    float *out = (splits == 1 ? y : ws + (int64_t)blockIdx.z * s * n) + (m0 + lh * 4) * n + col;
    const int rows_left = (int)(s - m0 - lh * 4);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int r = i * 32 + (v >> 2) * 8 + (v & 3);
        if (r < rows_left)
          out[(int64_t)r * n] = acc[i][v] + red[((p * TM + i) * 16 + v) * 64 + lane];
      }
  }
}

// y[i] = sum over splits z (in order) of ws[z][i]; four outputs per thread.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float *__restrict__ ws,
                                                            float *__restrict__ y, int64_t count,
                                                            int splits) {
  const int64_t i = 4 * ((int64_t)blockIdx.x * blockDim.x + threadIdx.x);
  if (i >= count) return;
  if (i + 4 <= count && (count & 3) == 0) {
    f32x4 v = *reinterpret_cast<const f32x4 *>(ws + i);
    for (int z = 1; z < splits; ++z) v += *reinterpret_cast<const f32x4 *>(ws + z * count + i);
    *reinterpret_cast<f32x4 *>(y + i) = v;
  } else {
    for (int64_t e = i; e < i + 4 && e < count; ++e) {
      float v = ws[e];
      for (int z = 1; z < splits; ++z) v += ws[z * count + e];
      y[e] = v;
    }
  }
}

template <int G, int KIND, bool XF32, int BM>
hipError_t launch_bm(const LinearArgs &a, hipStream_t st) {
  constexpr int PB = 2, PA = 2, P = 2;
  const int64_t nslot = (a.m + 63) / 64;
  const int64_t nit_all = (nslot + 1) / 2;
  const int64_t gx = (a.n + BN - 1) / BN, gy = (a.s + BM - 1) / BM;
  // Split K when the output tiles alone leave CUs idle (256 CUs, one 8-wave
  // workgroup each); every split keeps at least 2 periods of iterations.
  int64_t splits = 1;
  if (a.ws) {
    while (gx * gy * splits * 2 <= 256 && (nit_all + 2 * splits - 1) / (2 * splits) >= 2 * P &&
           2 * splits * a.s * a.n <= a.ws_floats)
      splits *= 2;
  }
  int64_t nit = (nit_all + splits - 1) / splits;
  nit = (nit + P - 1) / P * P;
  dim3 grid((unsigned)gx, (unsigned)gy, (unsigned)splits), block(NT);
  hipLaunchKernelGGL((gemm_kernel<G, KIND, XF32, BM, PB, PA>), grid, block, 0, st, a.w,
                     a.row_bytes, a.x, a.y, a.s, a.m, a.n, (int)nit, a.ws);
  if (splits > 1) {
    const int64_t count = a.s * a.n;
    const int64_t threads = (count + 3) / 4;
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                       st, a.ws, a.y, count, (int)splits);
  }
  return hipGetLastError();
}

template <int G, int KIND, bool XF32>
hipError_t launch_x(const LinearArgs &a, hipStream_t st) {
  // 64-row tiles: the largest that run two waves per SIMD without register
  // spills; grids with few tiles are widened by splitting K.
  return launch_bm<G, KIND, XF32, 64>(a, st);
}

template <int G, int KIND>
hipError_t launch_g(const LinearArgs &a, hipStream_t st) {
  if (a.x_is_bf16) return launch_x<G, KIND, false>(a, st);
  return launch_x<G, KIND, true>(a, st);
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
