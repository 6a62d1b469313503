// q8_gemm.hip -- prefill-path Q8 GEMM on gfx950 f16 MFMA, weights
// dequantized in registers.
//
// y[i, j] = sum_k x[i, k] * (q[j, k] * scale[j, k / G])
// (k_mm_q8's product, src/llama_q8.mojo:73-84) as a dequant-GEMM on
// v_mfma_f32_32x32x16_f16, in two launches:
//   1. act16_kernel: each activation row is scaled by a power of two 2^-e_i
//      so that its largest |x| lies in [2^14, 2^15), rounded to binary16
//      (exact for bf16 input: binary16 has three more mantissa bits and the
//      scaled row sits inside its normal range), and written with e_i.  With
//      f32 scales the same launch gives every weight row j an exponent f_j
//      that puts its largest scale in [2^7, 2^8) (binary16 scales need none:
//      f_j = 0);
//   2. gemm_kernel: each lane turns its column's int8 codes into binary16
//      weights q * s 2^-f_j in registers and feeds them to the MFMA as the B
//      operand; the activations come through LDS as the A operand; the f32
//      accumulators need no per-group rescale, and each output is scaled
//      once by 2^(e_i + f_j).
// Rounding: the binary16 weight carries one rounding of q * s (two with f32
// scales: s 2^-f_j is rounded to binary16 first), i.e. a relative error
// below 2^-11 each; products and sums are f32.  Without the row exponent
// an f32 scale below 2^-14 (a group absmax under about 7.75e-3) would land
// in binary16's subnormal range and lose relative precision; with it only
// groups 2^21 times smaller than their row's largest group do, and their
// share of any output is that much smaller.
//
// Cost model (per SIMD: 512 MFMA MACs or 16 VALU lanes per clock).  A weight
// costs 1.75 VALU operations (one xor per 4 codes, then per 2 codes a v_perm
// that builds binary16 1024 + (q + 128), a packed subtract of 1152 and a
// packed multiply by the scale) and is used by BM rows; the activations
// cost no VALU work in the loop.  At BM = 128 the VALU needs ~0.44 clocks
// per MFMA clock.
//
// Work decomposition (one workgroup of 8 waves per BM x BN output tile,
// BN = 128 * TN): the waves form 4 column groups of 32 * TN outputs x 2
// K-parities; wave (p, h) owns TN column tiles of 32 and all BM rows and
// takes the second 64-code slot of each 128-code iteration when h = 1; the
// two parities meet in LDS at the end.  Per iteration the workgroup stages
// three tiles through registers into double-buffered LDS, each loaded with
// whole 128-byte lines: activations (BM x 128 binary16), codes (BN rows x
// 128 bytes, 16-byte chunks XOR-swizzled by row) and, every other
// iteration, the scales of the next two.  A lane then reads its column's
// codes and scales from LDS and dequantizes them in registers as the MFMA
// B operand; the MFMA K order inside a slot is permuted so each lane's
// codes come in two 16-byte chunks and no k-step straddles a quantization
// group (the A fragments read from LDS use the same permutation).
#include "q8_device.h"
#include "q8_launch.h"

namespace q8 {
namespace {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int KT = 128;        // k per iteration = two 64-code slots
constexpr int kWaves = 8;      // waves per workgroup: 8 (two K parities) or 4
constexpr int LDA = KT + 8;    // halves per LDS row (16-byte pad)

// ---- 1. activation rows to binary16 ----------------------------------------
// Exponent f that puts a weight row's largest f32 scale mx in [2^7, 2^8):
// then |q| * s 2^-f <= 127 * 2^8 stays far inside binary16's range and
// every scale above 2^-21 mx is a normal binary16 number.  Zero, inf and
// NaN maxima keep f = 0.
__device__ __forceinline__ int weight_row_exponent(float mx) {
  if (!(mx > 0.0f) || !(mx <= 3.4028235e38f)) return 0;
  int bias = 0;
  if (mx < 1.17549435e-38f) {              // subnormal: scale up exactly first
    mx *= 18446744073709551616.0f;         // 2^64
    bias = 64;
  }
  return (int)((__builtin_bit_cast(uint32_t, mx) >> 23) & 255u) - 127 - 7 - bias;
}

// Blocks [0, s): one 256-thread block per activation row.  With CH > 0 the
// row (m <= 2048 CH) stays in registers between the max and the conversion
// (one pass over memory); CH = 0 reads it twice.  Blocks [s, s + nwb): one
// wave per weight row, the row exponent of its f32 scales (ew), f32 scales
// only (nwb = 0 otherwise).
template <bool XF32, int CH, int G>
__global__ __launch_bounds__(256) void act16_kernel(const void *__restrict__ xv, int64_t s,
                                                    int64_t m, uint16_t *__restrict__ x16,
                                                    int *__restrict__ ex,
                                                    const uint8_t *__restrict__ w,
                                                    int64_t row_bytes, int64_t n,
                                                    int *__restrict__ ew) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x;
  if (r >= s) {
    // the whole block takes this branch (no barrier in it)
    const int64_t j = (r - s) * 4 + (tid >> 6);
    if (j >= n) return;
    const float *sc = reinterpret_cast<const float *>(w + j * row_bytes);
    float mx = 0.0f;
    for (int64_t g = tid & 63; g < m / G; g += 64) mx = fmaxf(mx, fabsf(sc[g]));
    mx = wave_max(mx);
    if ((tid & 63) == 0) ew[j] = weight_row_exponent(mx);
    return;
  }
  // 8 consecutive values per step (m is a multiple of 8)
  auto load8 = [&](int64_t k, float (&v)[8]) {
    if constexpr (XF32) {
      const f32x4 *p = reinterpret_cast<const f32x4 *>(static_cast<const float *>(xv) + r * m + k);
      const f32x4 a = p[0], b = p[1];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        v[c] = a[c];
        v[4 + c] = b[c];
      }
    } else {
      const u32x4 d = *reinterpret_cast<const u32x4 *>(static_cast<const uint16_t *>(xv) + r * m + k);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        v[2 * c] = __builtin_bit_cast(float, d[c] << 16);
        v[2 * c + 1] = __builtin_bit_cast(float, d[c] & 0xffff0000u);
      }
    }
  };
  auto store8 = [&](int64_t k, const float (&v)[8], int e) {
    u32x4 o;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const f16x2 hv = {(_Float16)__builtin_ldexpf(v[2 * c], -e),
                        (_Float16)__builtin_ldexpf(v[2 * c + 1], -e)};
      o[c] = __builtin_bit_cast(uint32_t, hv);
    }
    *reinterpret_cast<u32x4 *>(x16 + r * m + k) = o;
  };
  auto exponent = [&](float mx) {
    mx = wave_max(mx);
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    // largest |x| * 2^-e in [2^14, 2^15); rows of zeros, inf or NaN keep e = 0
    int e = 0;
    if (mx > 0.0f && mx <= 3.4028235e38f) {
      e = (int)((__builtin_bit_cast(uint32_t, mx) >> 23) & 255u) - 127 - 14;
      if (mx < 1.17549435e-38f) e = -126;     // subnormal maximum: as far as 2^126 goes
      e = e < -126 ? -126 : e;
    }
    return e;
  };
  float mx = 0.0f;
  int e;
  if constexpr (CH > 0) {
    float v[CH][8];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int64_t k = 8 * tid + 2048 * c;
      if (k < m) {
        load8(k, v[c]);
#pragma unroll
        for (int j = 0; j < 8; ++j) mx = fmaxf(mx, fabsf(v[c][j]));
      }
    }
    e = exponent(mx);
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int64_t k = 8 * tid + 2048 * c;
      if (k < m) store8(k, v[c], e);
    }
  } else {
    for (int64_t k = 8 * tid; k < m; k += 2048) {
      float v[8];
      load8(k, v);
#pragma unroll
      for (int j = 0; j < 8; ++j) mx = fmaxf(mx, fabsf(v[j]));
    }
    e = exponent(mx);
    for (int64_t k = 8 * tid; k < m; k += 2048) {
      float v[8];
      load8(k, v);
      store8(k, v, e);
    }
  }
  if (tid == 0) ex[r] = e;
}

// nw weight rows get their exponents (0 for none).
template <bool XF32, int G>
void launch_act16(const LinearArgs &a, uint16_t *x16, int *ex, int *ew, int64_t nw,
                  hipStream_t st) {
  const dim3 grid((unsigned)(a.s + (nw + 3) / 4)), block(256);
#define Q8_ACT16(CH)                                                                         \
  hipLaunchKernelGGL((act16_kernel<XF32, CH, G>), grid, block, 0, st, a.x, a.s, a.m, x16, ex, \
                     a.w, a.row_bytes, nw, ew)
  if (a.m <= 2048)
    Q8_ACT16(1);
  else if (a.m <= 4096)
    Q8_ACT16(2);
  else if (a.m <= 8192)
    Q8_ACT16(4);
  else if (a.m <= 16384)
    Q8_ACT16(8);
  else
    Q8_ACT16(0);
#undef Q8_ACT16
}

// ---- 2. the GEMM --------------------------------------------------------------
// Eight codes (two dwords, k order) times one binary16 scale pair.
__device__ __forceinline__ f16x8 dequant8(uint32_t d0, uint32_t d1, f16x2 s2) {
  const f16x2 off = {(_Float16)1152.0f, (_Float16)1152.0f};
  const uint32_t x0 = d0 ^ 0x80808080u, x1 = d1 ^ 0x80808080u;   // q + 128 per byte
  // binary16 0x64hh = 1024 + hh exactly; minus 1152 gives q exactly
  const f16x2 a = (__builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, x0, 0x04010400u)) - off) * s2;
  const f16x2 b = (__builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, x0, 0x04030402u)) - off) * s2;
  const f16x2 c = (__builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, x1, 0x04010400u)) - off) * s2;
  const f16x2 d = (__builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, x1, 0x04030402u)) - off) * s2;
  return f16x8{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
}

template <int G, int KIND, int BM, int TN, int NW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(NW / 4, NW / 4)))
void gemm_kernel(const uint8_t *__restrict__ w, int64_t row_bytes,
                   const uint16_t *__restrict__ x16, const int *__restrict__ ex,
                   const int *__restrict__ ew, float *__restrict__ y, int64_t s, int64_t m,
                   int64_t n, int nit, float *__restrict__ ws) {
  // blockIdx.z selects a K range of nit iterations (split-K): with
  // gridDim.z == 1 y is written directly, otherwise split z writes its
  // partial sums to ws[z] and splitk_reduce_kernel adds them up.
  constexpr int NT = 64 * NW;                 // threads
  constexpr int NP = NW / 4;                  // K parities among the waves (1 or 2)
  constexpr int SB = ScaleTraits<KIND>::bytes;
  constexpr int TM = BM / 32;                 // 32-row MFMA tiles per wave
  constexpr int BN = 128 * TN;
  constexpr int AU = BM * KT / 8 / NT;        // 8-half A chunks per thread
  constexpr int NG = 64 / G;                  // groups per 64-code slot
  constexpr int SPB = (KT / G) * SB;          // scale bytes of a row per iteration
  constexpr int SDW = BN * SPB / 4;           // ... as dwords per block
  constexpr int SU = (SDW + NT - 1) / NT;     // ... per thread
  constexpr int CU = BN * KT / 16 / NT;       // 16-byte code chunks per thread
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * LDA];
  __shared__ __attribute__((aligned(16))) uint8_t Bs[2][BN * KT];    // codes, swizzled rows
  __shared__ __attribute__((aligned(16))) uint8_t Ss[2][BN * SPB];   // scales
  __shared__ int exs[BM];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int p = wid & 3, h0 = wid >> 2;
  const int lr = lane & 31, lh = lane >> 5;
  const int64_t n0 = (int64_t)blockIdx.x * BN, m0 = (int64_t)blockIdx.y * BM;
  // This split covers codes [kbase, kbase + nit * KT); iteration it covers
  // the 128 codes from kbase + KT it: with 8 waves parity h0 takes the
  // 64-code slot at 64 h0, with 4 waves each wave takes both slots.
  const int64_t kbase = (int64_t)blockIdx.z * nit * KT;

  // Weights: this block's (at most) BN packed rows; a row past n lies past
  // the resource (its loads read zeros).
  const int64_t nrows = n - n0 < BN ? n - n0 : BN;
  const rsrc_t wr = make_rsrc(w + n0 * row_bytes, (uint32_t)(nrows * row_bytes));
  // Code tiles: BN rows x 128 codes per iteration, 8 threads per 128-byte
  // row (coalesced), staged through registers.  The 16-byte chunk c of row
  // r sits at LDS chunk c ^ ((r >> 1) & 7): the 16 rows one ds_read_b128
  // pass reads then fall on 16 different bank groups.
  auto load_codes = [&](u32x4 *dst, int it) {
#pragma unroll
    for (int u = 0; u < CU; ++u) {
      const int c = tid + NT * u, r = c >> 3;
      dst[u] = bload16(wr, (uint32_t)(r * row_bytes + (m / G) * SB + kbase + KT * it + 16 * (c & 7)));
    }
  };
  auto store_codes = [&](const u32x4 *src, int buf) {
#pragma unroll
    for (int u = 0; u < CU; ++u) {
      const int c = tid + NT * u, r = c >> 3;
      *reinterpret_cast<u32x4 *>(&Bs[buf][r * KT + 16 * ((c & 7) ^ ((r >> 1) & 7))]) = src[u];
    }
  };
  // Scale tiles: BN rows x SPB bytes per iteration, as dwords (thread t
  // takes dwords t, t + NT, ... of the [BN][SPB / 4] tile; a thread past the
  // tile loads a duplicate it does not store, so no load sits in a branch).
  auto load_scales = [&](uint32_t *dst, int it) {
#pragma unroll
    for (int u = 0; u < SU; ++u) {
      const int i = (tid + NT * u) % SDW;
      dst[u] = __builtin_amdgcn_raw_buffer_load_b32(
          wr, (uint32_t)((i / (SPB / 4)) * row_bytes + (kbase + KT * it) / G * SB +
                         4 * (i % (SPB / 4))), 0, 0);
    }
  };
  auto store_scales = [&](const uint32_t *src, int buf) {
#pragma unroll
    for (int u = 0; u < SU; ++u) {
      const int i = tid + NT * u;
      if (i < SDW) *reinterpret_cast<uint32_t *>(&Ss[buf][4 * i]) = src[u];
    }
  };
  // This lane's column within the block for tile t
  auto bcol = [&](int t) { return p * 32 * TN + 32 * t + lr; };
  // k-step ks of lane half lh reads codes (offsets within the slot)
  //   G=64: [32 lh + 8 ks, +8)                      (chunks at 32 lh, 32 lh + 16)
  //   G=32: [32 (ks / 2) + 16 lh + 8 (ks % 2), +8)   (chunks at 16 lh, 32 + 16 lh)
  // so for G = 32 k-steps 0..1 are the slot's first group and 2..3 its second.
  const int chunk0 = G == 64 ? 32 * lh : 16 * lh;
  const int chunk1 = G == 64 ? 32 * lh + 16 : 32 + 16 * lh;

  // Activations (binary16 rows from act16_kernel): this block's (at most)
  // BM rows, 128 k per iteration; chunk u of a thread is row c / 16, k
  // 8 (c % 16) .. +8 (c = tid + NT u).  A row past s lies past the
  // resource, a column past m is sent past it explicitly.
  const int64_t arows = s - m0 < BM ? s - m0 : BM;
  const rsrc_t xr = make_rsrc(x16 + m0 * m, (uint32_t)(arows * m * 2));
  const int64_t mk = m - kbase;
  uint32_t vx[AU];
  int akc[AU];
#pragma unroll
  for (int u = 0; u < AU; ++u) {
    const int c = tid + NT * u;
    akc[u] = (c % (KT / 8)) * 8;
    vx[u] = (uint32_t)(((c / (KT / 8)) * m + kbase + akc[u]) * 2);
  }
  auto load_a = [&](u32x4 *dst, int it) {
#pragma unroll
    for (int u = 0; u < AU; ++u) {
      const uint32_t off = KT * it + akc[u] < mk ? vx[u] + KT * it * 2 : kOutOfRange;
      dst[u] = bload16(xr, off);
    }
  };
  auto store_a = [&](const u32x4 *src, int buf) {
#pragma unroll
    for (int u = 0; u < AU; ++u) {
      const int row = (tid + NT * u) / (KT / 8);
      *reinterpret_cast<u32x4 *>(&As[buf][row * LDA + akc[u]]) = src[u];
    }
  };
  // activation column of k-step ks (same permutation as the codes)
  auto acol = [&](int h, int ks) {
    return 64 * h + (G == 64 ? 32 * lh + 8 * ks : 32 * (ks >> 1) + 16 * lh + 8 * (ks & 1));
  };

  if (tid < BM) exs[tid] = tid < arows ? ex[m0 + tid] : 0;
  // this lane's weight-row exponents (f32 scales) per column tile
  int ewc[TN];
#pragma unroll
  for (int t = 0; t < TN; ++t)
    ewc[t] = KIND == SCALE_F32 && n0 + bcol(t) < n ? ew[n0 + bcol(t)] : 0;

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int t = 0; t < TN; ++t)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][t][v] = 0.0f;

  // Every iteration stages the tiles of the next one; loads past the split's
  // K range read zeros or bytes that are never used, so none of them sits in
  // a branch (a load in a branch makes the wave wait for all its loads).
  u32x4 ra[AU], rc[CU];
  uint32_t rs[SU];
  load_scales(rs, 0);
  load_codes(rc, 0);
  load_a(ra, 0);
  store_scales(rs, 0);
  store_codes(rc, 0);
  store_a(ra, 0);
  load_scales(rs, 1);
  load_codes(rc, 1);
  load_a(ra, 1);
  __syncthreads();

  const f16x2 zero2 = {(_Float16)0.0f, (_Float16)0.0f};
  for (int it = 0; it < nit; ++it) {
    const uint8_t *bt = Bs[it & 1];
    const uint8_t *st = Ss[it & 1];
    const uint16_t *at = As[it & 1];
#pragma unroll
    for (int hh = 0; hh < 2 / NP; ++hh) {
      const int h = h0 + hh;
      // the slot's codes and scales for each column tile; a slot (or its
      // second G=32 group) past the row end meets zero activations and its
      // scales (whatever bytes were read) are forced to 0
      const int64_t k0 = kbase + KT * it + 64 * h;
      u32x4 cq[TN][2];
      f16x2 s2[TN][NG];
#pragma unroll
      for (int t = 0; t < TN; ++t) {
        const int r = bcol(t);
        const int sw = (r >> 1) & 7;
        cq[t][0] = *reinterpret_cast<const u32x4 *>(bt + r * KT + 16 * ((4 * h + (chunk0 >> 4)) ^ sw));
        cq[t][1] = *reinterpret_cast<const u32x4 *>(bt + r * KT + 16 * ((4 * h + (chunk1 >> 4)) ^ sw));
        const uint8_t *sp = st + r * SPB + h * NG * SB;
#pragma unroll
        for (int g = 0; g < NG; ++g) {
          _Float16 hs;
          if constexpr (KIND == SCALE_F16)
            hs = *reinterpret_cast<const _Float16 *>(sp + 2 * g);
          else
            hs = (_Float16)__builtin_ldexpf(*reinterpret_cast<const float *>(sp + 4 * g), -ewc[t]);
          s2[t][g] = k0 + g * G < m ? f16x2{hs, hs} : zero2;
        }
      }
      // The slot's MFMA work runs at raised wave priority: of the SIMD's two
      // waves the one in its MFMA phase issues first, the other stages and
      // dequantizes meanwhile.
      __builtin_amdgcn_s_setprio(1);
      // A fragments of k-step ks + 1 are read while k-step ks runs
      f16x8 af[2][TM];
#pragma unroll
      for (int ii = 0; ii < TM; ++ii)
        af[0][ii] = *reinterpret_cast<const f16x8 *>(&at[(ii * 32 + lr) * LDA + acol(h, 0)]);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        if (ks < 3) {
#pragma unroll
          for (int ii = 0; ii < TM; ++ii)
            af[(ks + 1) & 1][ii] =
                *reinterpret_cast<const f16x8 *>(&at[(ii * 32 + lr) * LDA + acol(h, ks + 1)]);
        }
        const int g = G == 64 ? 0 : ks >> 1;
        f16x8 bq[TN];
#pragma unroll
        for (int t = 0; t < TN; ++t) {
          const u32x4 &c = cq[t][ks >> 1];
          bq[t] = (ks & 1) ? dequant8(c.z, c.w, s2[t][g]) : dequant8(c.x, c.y, s2[t][g]);
        }
#pragma unroll
        for (int ii = 0; ii < TM; ++ii)
#pragma unroll
          for (int t = 0; t < TN; ++t)
            acc[ii][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[ks & 1][ii], bq[t], acc[ii][t], 0, 0, 0);
      }
      __builtin_amdgcn_s_setprio(0);
    }
    // stage the tiles of iteration it + 1, then load those of it + 2
    store_scales(rs, (it + 1) & 1);
    store_codes(rc, (it + 1) & 1);
    store_a(ra, (it + 1) & 1);
    __syncthreads();
    load_scales(rs, it + 2);
    load_codes(rc, it + 2);
    load_a(ra, it + 2);
  }

  // With two K parities, each column tile's parities meet in LDS (reusing
  // As), one column tile at a time; each output is scaled by 2^(e_i + f_j).
  float *red = reinterpret_cast<float *>(&As[0][0]);   // 4 * TM * 16 * 64 floats
  static_assert(4 * TM * 16 * 64 * 4 <= (int)sizeof(As), "reduction buffer too small");
  const int rows_left = (int)(s - m0 - lh * 4);
#pragma unroll
  for (int t = 0; t < TN; ++t) {
    if constexpr (NP == 2) {
      __syncthreads();
      if (h0 == 1) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int v = 0; v < 16; ++v) red[((p * TM + i) * 16 + v) * 64 + lane] = acc[i][t][v];
      }
      __syncthreads();
    }
    const int64_t col = n0 + bcol(t);
    if (h0 == 0 && col < n) {
      // D layout of v_mfma_f32_32x32x16: lane -> column lane % 32,
      // element v -> row 8 (v / 4) + 4 (lane / 32) + v % 4.
      float *out = (gridDim.z == 1 ? y : ws + (int64_t)blockIdx.z * s * n) + (m0 + lh * 4) * n + col;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int r = i * 32 + (v >> 2) * 8 + (v & 3);
          float o = acc[i][t][v];
          if constexpr (NP == 2) o += red[((p * TM + i) * 16 + v) * 64 + lane];
          if (r < rows_left) out[(int64_t)r * n] = __builtin_ldexpf(o, exs[r + lh * 4] + ewc[t]);
        }
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

template <int G, int KIND, int BM, int TN, int NW>
hipError_t launch_t(const LinearArgs &a, const uint16_t *x16, const int *ex, const int *ew,
                    hipStream_t st) {
  constexpr int BN = 128 * TN;
  const int64_t nit_all = (a.m + KT - 1) / KT;
  const int64_t gx = (a.n + BN - 1) / BN, gy = (a.s + BM - 1) / BM;
  // Split K when the output tiles alone leave CUs idle (256 CUs, one 8-wave
  // workgroup each); every split keeps at least 4 iterations.
  int64_t splits = 1;
  if (a.ws) {
    while (gx * gy * splits * 2 <= 256 && (nit_all + 2 * splits - 1) / (2 * splits) >= 4 &&
           2 * splits * a.s * a.n <= a.ws_floats)
      splits *= 2;
  }
  int64_t nit = (nit_all + splits - 1) / splits;
  dim3 grid((unsigned)gx, (unsigned)gy, (unsigned)splits), block(64 * NW);
  hipLaunchKernelGGL((gemm_kernel<G, KIND, BM, TN, NW>), grid, block, 0, st, a.w, a.row_bytes, x16,
                     ex, ew, a.y, a.s, a.m, a.n, (int)nit, a.ws);
  if (splits > 1) return launch_splitk_reduce(a.ws, a.y, a.s * a.n, (int)splits, st);
  return hipGetLastError();
}

template <int G, int KIND>
hipError_t launch_g(const LinearArgs &a, uint16_t *x16, int *ex, int *ew, bool weights,
                    hipStream_t st) {
  // weight-row exponents only for f32 scales, and only when asked (a call
  // split into row chunks computes them with its first chunk)
  const int64_t nw = KIND == SCALE_F32 && weights ? a.n : 0;
  if (a.x_is_bf16)
    launch_act16<false, G>(a, x16, ex, ew, nw, st);
  else
    launch_act16<true, G>(a, x16, ex, ew, nw, st);
  // 128-row tiles once the rows fill them; two column tiles per wave when
  // the 256-column tiles still give every CU a workgroup.
  if (a.s > 64) {
    const int64_t tiles256 = (a.n + 255) / 256 * ((a.s + 127) / 128);
    if (tiles256 >= 256) return launch_t<G, KIND, 128, 2, kWaves>(a, x16, ex, ew, st);
    return launch_t<G, KIND, 128, 1, kWaves>(a, x16, ex, ew, st);
  }
  return launch_t<G, KIND, 64, 1, kWaves>(a, x16, ex, ew, st);
}

}  // namespace

hipError_t launch_splitk_reduce(const float *ws, float *y, int64_t count, int splits,
                                hipStream_t st) {
  const int64_t threads = (count + 3) / 4;
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     st, ws, y, count, splits);
  return hipGetLastError();
}

hipError_t launch_gemm(const LinearArgs &a, uint16_t *x16, int *ex, int *ew, bool weights,
                       hipStream_t st) {
  if (a.s == 0 || a.n == 0) return hipSuccess;
  if (a.G == 64 && a.kind == SCALE_F16) return launch_g<64, SCALE_F16>(a, x16, ex, ew, weights, st);
  if (a.G == 64 && a.kind == SCALE_F32) return launch_g<64, SCALE_F32>(a, x16, ex, ew, weights, st);
  if (a.G == 32 && a.kind == SCALE_F16) return launch_g<32, SCALE_F16>(a, x16, ex, ew, weights, st);
  if (a.G == 32 && a.kind == SCALE_F32) return launch_g<32, SCALE_F32>(a, x16, ex, ew, weights, st);
  return hipErrorInvalidValue;
}

}  // namespace q8
