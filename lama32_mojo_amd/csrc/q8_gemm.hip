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
// Cost model.  The per-group fold is one non-packed f32 FMA per output and
// group, i.e. MACs / G FMAs: at G = 32 the VALU needs as many cycles for the
// fold as the MFMA pipe needs for the products (16 FMA lanes vs 512 MACs per
// clock and SIMD).  Everything else on the VALU is kept small: the codes of a
// weight fragment are converted once and reused by all row tiles of a wave,
// and all addressing is 32-bit buffer offsets whose range check also zero-fills
// the ragged edges (no clamps in the loop).
//
// Work decomposition (one 512-thread workgroup per BM x 128 output tile):
//   * the 8 waves form 4 column slices of 32 outputs x 2 K-parities; wave
//     (p, h) accumulates columns p*32.. over the 64-code K slots of parity h,
//     so each SIMD runs two independent instruction streams whose MFMA and
//     VALU work co-issue; the two parities meet in LDS at the end;
//   * a wave's weight codes never touch LDS: lane l owns output column
//     l % 32 and loads its 32 codes of a slot straight from memory into
//     registers (two dwordx4), converted to bf16 in registers.  The MFMA K
//     order inside a slot is permuted so each lane's codes come in two
//     16-byte chunks and no k-step straddles a quantization group; the
//     activation fragments read from LDS use the same permutation;
//   * activations are staged through double-buffered LDS, 128 k per step,
//     loaded one step ahead; the weight codes run in a register ring PB
//     slots ahead, with the loop unrolled so ring slots are compile-time
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

// Raw scale bits of 4 consecutive 64-code slots (one load period), and the
// scales of slot j of a period.  A slot holds 64 / G scales, so a period is
// 8 (G=64, f16), 16 (G=64 f32 or G=32 f16) or 32 (G=32, f32) bytes, loaded
// with naturally aligned loads: the scale section of a row is 16-byte
// aligned (checked by the host) and periods start at multiples of 4 slots.
template <int G, int KIND> struct ScalePeriod {
  static constexpr int slot_bytes = (64 / G) * ScaleTraits<KIND>::bytes;
  static constexpr int bytes = 4 * slot_bytes;
  static constexpr int words = bytes / 4;
  uint32_t wd[words];
  __device__ __forceinline__ void load(rsrc_t r, uint32_t off) {
    if constexpr (bytes == 8) {
      const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
      wd[0] = v.x; wd[1] = v.y;
    } else {
#pragma unroll
      for (int i = 0; i < words / 4; ++i) {
        const u32x4 v = bload16(r, off + 16 * i);
        wd[4 * i] = v.x; wd[4 * i + 1] = v.y; wd[4 * i + 2] = v.z; wd[4 * i + 3] = v.w;
      }
    }
  }
  // scale gi (0 .. 64/G - 1) of slot j (0..3) of the period
  __device__ __forceinline__ float get(int j, int gi) const {
    if constexpr (G == 64 && KIND == SCALE_F16)
      return f16_bits_to_f32((uint16_t)(wd[j / 2] >> (16 * (j % 2))));
    else if constexpr (G == 64)
      return __builtin_bit_cast(float, wd[j]);
    else if constexpr (KIND == SCALE_F16)
      return f16_bits_to_f32((uint16_t)(wd[j] >> (16 * gi)));
    else
      return __builtin_bit_cast(float, wd[2 * j + gi]);
  }
};

template <int G, int KIND, bool XF32, int BM, int PB>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(2, 2)))
void gemm_kernel(const uint8_t *__restrict__ w, int64_t row_bytes, const void *__restrict__ xv,
                 float *__restrict__ y, int64_t s, int64_t m, int64_t n, int nit,
                 float *__restrict__ ws) {
  // blockIdx.z selects a K range of nit iterations (split-K): with
  // gridDim.z == 1 y is written directly, otherwise split z writes its
  // partial sums to ws[z] and splitk_reduce_kernel adds them up.
  constexpr int SB = ScaleTraits<KIND>::bytes;
  constexpr int TM = BM / 32;                 // 32-row MFMA tiles per wave
  constexpr int XB = XF32 ? 4 : 2;            // bytes per activation
  constexpr int AU = BM * KT / 8 / NT;        // 8-activation chunks per thread
  constexpr int NLDS = XF32 ? 2 : 1;
  typedef ScalePeriod<G, KIND> SP;
  static_assert(PB == 4, "scale loads cover periods of 4 slots");
  __shared__ __attribute__((aligned(16))) uint16_t As[2][NLDS][BM * LDA];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int p = wid & 3, h = wid >> 2;
  const int lr = lane & 31, lh = lane >> 5;
  const int64_t n0 = (int64_t)blockIdx.x * BN, m0 = (int64_t)blockIdx.y * BM;
  // This split covers codes [kbase, kbase + nit * KT).  Wave parity h takes
  // K half h of it, starting at khalf; iteration it of the wave covers the
  // 64-code slot at khalf + 64 it (and the LDS tile of an iteration holds
  // half 0's 64 columns, then half 1's).
  const int64_t kbase = (int64_t)blockIdx.z * nit * KT;
  const int64_t khalf = kbase + (int64_t)h * nit * 64;
  const int64_t mh = m - khalf;                       // codes of the row from khalf on

  // Weights: this block's (at most) 128 packed rows.  Lane offsets are
  // relative to the block's first row; a row past n lies past the resource.
  const int64_t nrows = n - n0 < BN ? n - n0 : BN;
  const rsrc_t wr = make_rsrc(w + n0 * row_bytes, (uint32_t)(nrows * row_bytes));
  const uint32_t wrow = (uint32_t)((p * 32 + lr) * row_bytes);
  // Codes of one 64-code slot held by a lane, as two 16-code chunks.  The
  // MFMA K order inside a slot is chosen so each k-step of 16 stays inside
  // one quantization group: k-step t of lane half lh reads codes
  //   G=64: [32 lh + 8 t, +8)                       (chunks at 32 lh, 32 lh + 16)
  //   G=32: [32 (t / 2) + 16 lh + 8 (t % 2), +8)     (chunks at 16 lh, 32 + 16 lh)
  // so t = 0..1 covers the slot's first group of 32 and t = 2..3 its second.
  const int chunk0 = G == 64 ? 32 * lh : 16 * lh;
  const int chunk1 = G == 64 ? 32 * lh + 16 : 32 + 16 * lh;
  const uint32_t vcodes = wrow + (uint32_t)((m / G) * SB + khalf);
  const uint32_t vscale = wrow + (uint32_t)(khalf / G * SB);
  // Codes past the row end read the next row (finite codes that meet zero
  // activations) or lie past the resource; scales past the last group are
  // replaced by 0 below.
  auto load_b = [&](u32x4 (&q)[2], int it) {
    q[0] = bload16(wr, vcodes + it * 64 + chunk0);
    q[1] = bload16(wr, vcodes + it * 64 + chunk1);
  };

  // Activations: this block's (at most) BM rows.  Chunk u of a thread is
  // row c / 16, LDS columns 8 (c % 16) .. +8 (c = tid + NT u); LDS columns
  // [0, 64) come from K half 0 and [64, 128) from K half 1.  A row past s
  // lies past the resource, a column past m is sent past it explicitly.
  const int64_t arows = s - m0 < BM ? s - m0 : BM;
  const rsrc_t xr = make_rsrc(reinterpret_cast<const uint8_t *>(xv) + m0 * m * XB,
                              (uint32_t)(arows * m * XB));
  const int64_t mk = m - kbase;
  uint32_t vx[AU];
  int akc[AU], akk[AU];
#pragma unroll
  for (int u = 0; u < AU; ++u) {
    const int c = tid + NT * u;
    akc[u] = (c % (KT / 8)) * 8;
    akk[u] = akc[u] < 64 ? akc[u] : nit * 64 + akc[u] - 64;   // code offset within the split
    vx[u] = (uint32_t)(((c / (KT / 8)) * m + kbase + akk[u]) * XB);
  }
  auto load_a = [&](u32x4 *dst, int it) {
#pragma unroll
    for (int u = 0; u < AU; ++u) {
      const uint32_t off = it * 64 + akk[u] < mk ? vx[u] + it * 64 * XB : kOutOfRange;
      if constexpr (!XF32) {
        dst[u] = bload16(xr, off);
      } else {
        dst[2 * u] = bload16(xr, off);
        dst[2 * u + 1] = bload16(xr, off + 16);
      }
    }
  };
  auto store_a = [&](const u32x4 *src, int buf) {
#pragma unroll
    for (int u = 0; u < AU; ++u) {
      const int row = (tid + NT * u) / (KT / 8);
      if constexpr (!XF32) {
        *reinterpret_cast<u32x4 *>(&As[buf][0][row * LDA + akc[u]]) = src[u];
      } else {
        const uint32_t d[8] = {src[2 * u].x, src[2 * u].y, src[2 * u].z, src[2 * u].w,
                               src[2 * u + 1].x, src[2 * u + 1].y, src[2 * u + 1].z,
                               src[2 * u + 1].w};
        uint32_t hi[4], lo[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float f0 = __builtin_bit_cast(float, d[2 * e]);
          const float f1 = __builtin_bit_cast(float, d[2 * e + 1]);
          const uint32_t h0 = bf16_rne(f0), h1 = bf16_rne(f1);
          const uint32_t l0 = bf16_rne(f0 - __builtin_bit_cast(float, h0 << 16));
          const uint32_t l1 = bf16_rne(f1 - __builtin_bit_cast(float, h1 << 16));
          hi[e] = h0 | (h1 << 16);
          lo[e] = l0 | (l1 << 16);
        }
        *reinterpret_cast<u32x4 *>(&As[buf][0][row * LDA + akc[u]]) = u32x4{hi[0], hi[1], hi[2], hi[3]};
        *reinterpret_cast<u32x4 *>(&As[buf][NLDS - 1][row * LDA + akc[u]]) =
            u32x4{lo[0], lo[1], lo[2], lo[3]};
      }
    }
  };

  f32x16 acc[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[i][v] = 0.0f;

  // units of work per slot: TH row tiles x one group of NG = 64 / G; a
  // group is KS = G / 16 k-steps
  constexpr int TH = TM < 2 ? TM : 2;
  constexpr int NG = 64 / G, KS = G / 16;
  constexpr int FPER = 16 / KS;               // fold FMAs after each MFMA
  f32x16 pq[TH];                              // partials of the unit awaiting its fold
#pragma unroll
  for (int i = 0; i < TH; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) pq[i][v] = 0.0f;
  float psc = 0.0f;

  u32x4 qb[PB][2];
  SP sp;                                      // scales of the current period
  u32x4 ra[XF32 ? 2 * AU : AU];

#pragma unroll
  for (int q = 0; q < PB; ++q) load_b(qb[q], q);
  sp.load(wr, vscale);
  load_a(ra, 0);
  store_a(ra, 0);
  load_a(ra, 1);
  __syncthreads();

  for (int i0 = 0; i0 < nit; i0 += PB) {
    // this period's scales, and the next period's in flight
    SP spc = sp;
    sp.load(wr, vscale + (i0 + PB) * SP::slot_bytes);
#pragma unroll
    for (int j = 0; j < PB; ++j) {
      const int it = i0 + j;
      const int buf = it & 1;
      bf16x8_t bf[4];
      bf[0] = codes_to_bf16(qb[j][0].x, qb[j][0].y);
      bf[1] = codes_to_bf16(qb[j][0].z, qb[j][0].w);
      bf[2] = codes_to_bf16(qb[j][1].x, qb[j][1].y);
      bf[3] = codes_to_bf16(qb[j][1].z, qb[j][1].w);
      // a slot (or its second G=32 group) past the row end meets zero
      // activations; its scales (whatever bytes were read) are forced to 0
      const float sc0 = it * 64 < mh ? spc.get(j, 0) : 0.0f;
      const float sc1 = (G == 32 && it * 64 + 32 < mh) ? spc.get(j, 1) : 0.0f;
      load_b(qb[j], it + PB);

      // activation column of k-step t (same permutation as the codes)
      auto acol = [&](int t) {
        return 64 * h + (G == 64 ? 32 * lh + 8 * t : 32 * (t >> 1) + 16 * lh + 8 * (t & 1));
      };
      // Work of a slot comes in units (TH row tiles x one quantization
      // group): the unit's MFMAs fill fresh partials tq, and the f32 fold of
      // the previous unit's partials pq (acc += scale * pq) is interleaved
      // between them, so the fold never waits on an MFMA that has just been
      // issued and the MFMA pipe never waits on the fold.  The last unit of
      // a slot is folded during the first unit of the next slot.
#pragma unroll
      for (int u = 0; u < (TM / TH) * NG; ++u) {
        const int ib = (u / NG) * TH, g = u % NG;
        const int pib = u == 0 ? TM - TH : ((u - 1) / NG) * TH;   // rows of pq
        f32x16 tq[TH];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const int t = g * KS + ks;
          bf16x8_t af[TH], al[TH];
#pragma unroll
          for (int ii = 0; ii < TH; ++ii) {
            const int ao = ((ib + ii) * 32 + lr) * LDA + acol(t);
            af[ii] = *reinterpret_cast<const bf16x8_t *>(&As[buf][0][ao]);
            if constexpr (XF32) al[ii] = *reinterpret_cast<const bf16x8_t *>(&As[buf][NLDS - 1][ao]);
          }
#pragma unroll
          for (int ii = 0; ii < TH; ++ii) {
            if (ks == 0) {
              const f32x16 z = {};
              tq[ii] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[ii], bf[t], z, 0, 0, 0);
            } else {
              tq[ii] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[ii], bf[t], tq[ii], 0, 0, 0);
            }
            if constexpr (XF32)
              tq[ii] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[ii], bf[t], tq[ii], 0, 0, 0);
            const int e0 = (ks * TH + ii) * FPER;
#pragma unroll
            for (int e = e0; e < e0 + FPER; ++e)
              acc[pib + e / 16][e % 16] = __builtin_fmaf(psc, pq[e / 16][e % 16], acc[pib + e / 16][e % 16]);
          }
        }
#pragma unroll
        for (int ii = 0; ii < TH; ++ii) pq[ii] = tq[ii];
        psc = g == 0 ? sc0 : sc1;
      }
      store_a(ra, buf ^ 1);
      __syncthreads();
      load_a(ra, it + 2);
    }
  }

  // fold of the last unit
#pragma unroll
  for (int ii = 0; ii < TH; ++ii)
#pragma unroll
    for (int v = 0; v < 16; ++v)
      acc[TM - TH + ii][v] = __builtin_fmaf(psc, pq[ii][v], acc[TM - TH + ii][v]);

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
  const int64_t col = n0 + p * 32 + lr;
  if (h == 0 && col < n) {
    // D layout of v_mfma_f32_32x32x16: lane -> column lane % 32,
    // element v -> row 8 (v / 4) + 4 (lane / 32) + v % 4.
    float *out = (gridDim.z == 1 ? y : ws + (int64_t)blockIdx.z * s * n) + (m0 + lh * 4) * n + col;
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
  constexpr int PB = 4;
  const int64_t nit_all = (a.m + KT - 1) / KT;
  const int64_t gx = (a.n + BN - 1) / BN, gy = (a.s + BM - 1) / BM;
  // Split K when the output tiles alone leave CUs idle (256 CUs, one 8-wave
  // workgroup each); every split keeps at least 2 ring periods of iterations.
  int64_t splits = 1;
  if (a.ws) {
    while (gx * gy * splits * 2 <= 256 && (nit_all + 2 * splits - 1) / (2 * splits) >= 2 * PB &&
           2 * splits * a.s * a.n <= a.ws_floats)
      splits *= 2;
  }
  int64_t nit = (nit_all + splits - 1) / splits;
  nit = (nit + PB - 1) / PB * PB;
  dim3 grid((unsigned)gx, (unsigned)gy, (unsigned)splits), block(NT);
  hipLaunchKernelGGL((gemm_kernel<G, KIND, XF32, BM, PB>), grid, block, 0, st, a.w, a.row_bytes,
                     a.x, a.y, a.s, a.m, a.n, (int)nit, a.ws);
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
  // bf16 activations: 128-row tiles once the rows fill them (each converted
  // weight fragment then feeds four row tiles); f32 activations carry a hi
  // and a lo LDS copy and run 64-row tiles.
  if constexpr (!XF32) {
    if (a.s > 64) return launch_bm<G, KIND, XF32, 128>(a, st);
  }
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
