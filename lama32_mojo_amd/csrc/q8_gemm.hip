// q8_gemm.hip -- prefill-path Q8 GEMM on gfx950 f16 MFMA, weights
// dequantized once per workgroup into LDS.
//
// y[i, j] = sum_k x[i, k] * (q[j, k] * scale[j, k / G])
// (k_mm_q8's product, src/llama_q8.mojo:73-84) as a dequant-GEMM on
// v_mfma_f32_32x32x16_f16, in two launches (a third, splitk_reduce_kernel,
// adds the partial sums when a grid with few output tiles splits K):
//   1. act16_kernel (or norm16_kernel, which first forms the row's RMSNorm
//      exactly as rmsnorm_kernel does): each activation row is scaled by a
//      power of two 2^-e_i
//      so that its largest |x| lies in [2^14, 2^15), rounded to binary16
//      (exact for bf16 input: binary16 has three more mantissa bits and the
//      scaled row sits inside its normal range), and written with e_i.  With
//      f32 scales the same launch gives every weight row j an exponent f_j
//      that puts its largest scale in [2^7, 2^8) (binary16 scales need none:
//      f_j = 0);
//   2. gemm_kernel: producer waves turn int8 codes into binary16 weights
//      q * s 2^-f_j and stage them, with the binary16 activations, in LDS;
//      consumer waves run the MFMAs on both (A = activations, B = weights);
//      the f32 accumulators need no per-group rescale, and each output is
//      scaled once by 2^(e_i + f_j).
// Rounding: the binary16 weight carries one rounding of q * s (two with f32
// scales: s 2^-f_j is rounded to binary16 first), i.e. a relative error
// below 2^-11 each; products and sums are f32.  Without the row exponent
// an f32 scale below 2^-14 (a group absmax under about 7.75e-3) would land
// in binary16's subnormal range and lose relative precision; with it only
// groups 2^21 times smaller than their row's largest group do, and their
// share of any output is that much smaller.
//
// Cost per weight (dequantized once per workgroup, used by BM rows): 1.75
// VALU operations (one xor per 4 codes, then per 2 codes a v_perm that
// builds binary16 1024 + (q + 128), a packed subtract of 1152 and a packed
// multiply by the scale) and one 2-byte LDS write, read back by the one
// consumer wave that owns its column (two when the consumers sit 2 x 2).
#include "q8_device.h"
#include "q8_launch.h"

namespace q8 {
namespace {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));


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

// Exponent e of an activation row whose largest |value| (over the block)
// is mx: the row is stored as binary16 x 2^-e, largest |x| 2^-e in
// [2^14, 2^15); rows of zeros, inf or NaN keep e = 0.  Block-wide (256
// threads; red holds 4 floats).
__device__ __forceinline__ int act_row_exponent(float mx, float *red) {
  const int tid = threadIdx.x;
  mx = wave_max(mx);
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  int e = 0;
  if (mx > 0.0f && mx <= 3.4028235e38f) {
    e = (int)((__builtin_bit_cast(uint32_t, mx) >> 23) & 255u) - 127 - 14;
    if (mx < 1.17549435e-38f) e = -126;     // subnormal maximum: as far as 2^126 goes
    e = e < -126 ? -126 : e;
  }
  return e;
}

// Block b of the weight-row part of a pre-pass: one wave per weight row
// j = 4 b + wave, the exponent of its f32 scales.
template <int G>
__device__ __forceinline__ void weight_exponents(int64_t b, const uint8_t *__restrict__ w,
                                                 int64_t row_bytes, int64_t m, int64_t n,
                                                 int *__restrict__ ew) {
  const int tid = threadIdx.x;
  const int64_t j = b * 4 + (tid >> 6);
  if (j >= n) return;
  const float *sc = reinterpret_cast<const float *>(w + j * row_bytes);
  float mx = 0.0f;
  for (int64_t g = tid & 63; g < m / G; g += 64) mx = fmaxf(mx, fabsf(sc[g]));
  mx = wave_max(mx);
  if ((tid & 63) == 0) ew[j] = weight_row_exponent(mx);
}

// Blocks [0, s): one 256-thread block per activation row.  With CH > 0 the
// row (m <= 2048 CH) stays in registers between the max and the conversion
// (one pass over memory); CH = 0 reads it twice.  Blocks [s, s + nwb): one
// wave per weight row, the row exponent of its f32 scales (ew), f32 scales
// only (nwb = 0 otherwise).
// SWIGLU (f32 x): x holds gate rows and up the matching up rows; the values
// converted are silu(gate) * up, computed as swiglu_kernel computes them.
// Row r of x (and of up) starts ldx elements after row r-1.
template <bool XF32, int CH, int G, bool SWIGLU = false>
__global__ __launch_bounds__(256) void act16_kernel(const void *__restrict__ xv, int64_t s,
                                                    int64_t m, uint16_t *__restrict__ x16,
                                                    int *__restrict__ ex,
                                                    const uint8_t *__restrict__ w,
                                                    int64_t row_bytes, int64_t n,
                                                    int *__restrict__ ew,
                                                    const float *__restrict__ up, int64_t ldx) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x;
  if (r >= s) {
    // the whole block takes this branch (no barrier in it)
    weight_exponents<G>(r - s, w, row_bytes, m, n, ew);
    return;
  }
  // 8 consecutive values per step (m is a multiple of 8)
  auto load8 = [&](int64_t k, float (&v)[8]) {
    if constexpr (XF32) {
      const f32x4 *p = reinterpret_cast<const f32x4 *>(static_cast<const float *>(xv) + r * ldx + k);
      const f32x4 a = p[0], b = p[1];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        v[c] = a[c];
        v[4 + c] = b[c];
      }
      if constexpr (SWIGLU) {
        const f32x4 *pu = reinterpret_cast<const f32x4 *>(up + r * ldx + k);
        const f32x4 ua = pu[0], ub = pu[1];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          v[c] = (v[c] / (1.0f + expf(-v[c]))) * ua[c];
          v[4 + c] = (v[4 + c] / (1.0f + expf(-v[4 + c]))) * ub[c];
        }
      }
    } else {
      const u32x4 d = *reinterpret_cast<const u32x4 *>(static_cast<const uint16_t *>(xv) + r * ldx + k);
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
  auto exponent = [&](float mx) { return act_row_exponent(mx, red); };
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
template <bool XF32, int G, bool SWIGLU = false>
void launch_act16(const LinearArgs &a, uint16_t *x16, int *ex, int *ew, int64_t nw,
                  hipStream_t st) {
  const dim3 grid((unsigned)(a.s + (nw + 3) / 4)), block(256);
#define Q8_ACT16(CH)                                                                          \
  hipLaunchKernelGGL((act16_kernel<XF32, CH, G, SWIGLU>), grid, block, 0, st, a.x, a.s, a.m,  \
                     x16, ex, a.w, a.row_bytes, nw, ew, a.up, a.ldx ? a.ldx : a.m)
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

// The pre-pass with the row's RMSNorm folded in (k_rmsnorm_w, after k_res_add
// when res is set): blocks [0, s) form h = x + res (stored to hout) and
// y = bf16(wn) h / sqrt(mean(h^2) + eps) exactly as rmsnorm_kernel does --
// thread t owns elements t, t + 256, ... (at most NV of them), sums their
// squares in that order and the block adds the threads with block_sum256 --
// then y's row exponent and binary16 row exactly as act16_kernel forms them
// from a stored y.  So the GEMM reads the bits that rmsnorm (or add +
// rmsnorm) and then the plain pre-pass give, without y in memory.  Every
// load of a row is issued before its first use; the row stays in registers.
// Blocks [s, s + nwb): weight-row exponents (f32 scales).
template <int NV, int G>
__global__ __launch_bounds__(256) void norm16_kernel(const float *x, const float *res, float *hout,
                                                     const uint16_t *__restrict__ wn, float eps,
                                                     int64_t s, int64_t m,
                                                     uint16_t *__restrict__ x16,
                                                     int *__restrict__ ex,
                                                     const uint8_t *__restrict__ w,
                                                     int64_t row_bytes, int64_t n,
                                                     int *__restrict__ ew) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x;
  if (r >= s) {
    weight_exponents<G>(r - s, w, row_bytes, m, n, ew);
    return;
  }
  float v[NV], u[NV];
  uint16_t wb[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int64_t k = tid + 256 * j;
    v[j] = k < m ? x[r * m + k] : 0.0f;
    u[j] = res && k < m ? res[r * m + k] : 0.0f;
    wb[j] = k < m ? wn[k] : (uint16_t)0;
  }
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    if (tid + 256 * j < m) {
      if (res) v[j] += u[j];
      ss = __builtin_fmaf(v[j], v[j], ss);
    }
  }
  if (res) {
#pragma unroll
    for (int j = 0; j < NV; ++j)
      if (tid + 256 * j < m) hout[r * m + tid + 256 * j] = v[j];
  }
  ss = block_sum256(ss, red);
  const float inv = 1.0f / sqrtf(ss / (float)m + eps);
  float mx = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    if (tid + 256 * j < m) {
      v[j] = bf16_bits_to_f32(wb[j]) * v[j] * inv;
      mx = fmaxf(mx, fabsf(v[j]));
    }
  }
  const int e = act_row_exponent(mx, red);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int64_t k = tid + 256 * j;
    if (k < m) x16[r * m + k] = __builtin_bit_cast(uint16_t, (_Float16)__builtin_ldexpf(v[j], -e));
  }
  if (tid == 0) ex[r] = e;
}

// Rows of at most 16384 elements (the C ABI checks it).
template <int G>
void launch_norm16(const LinearArgs &a, uint16_t *x16, int *ex, int *ew, int64_t nw,
                   hipStream_t st) {
  const dim3 grid((unsigned)(a.s + (nw + 3) / 4)), block(256);
  const float *x = static_cast<const float *>(a.x);
#define Q8_NORM16(NV)                                                                          \
  hipLaunchKernelGGL((norm16_kernel<NV, G>), grid, block, 0, st, x, a.res, a.hout, a.wn,      \
                     a.eps, a.s, a.m, x16, ex, a.w, a.row_bytes, nw, ew)
  if (a.m <= 2048)
    Q8_NORM16(8);
  else if (a.m <= 4096)
    Q8_NORM16(16);
  else if (a.m <= 8192)
    Q8_NORM16(32);
  else
    Q8_NORM16(64);
#undef Q8_NORM16
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

// One workgroup per BM x BN output tile (BM = 32 TM CR, BN = 32 TN (4 /
// CR)), its 4 + NPW waves split by role (12, three per SIMD):
//   * waves 0-3 (consumers) only read MFMA fragments from LDS and issue the
//     MFMAs, each over 32 TM rows and 32 TN columns of the tile (TM x TN
//     accumulator tiles of 32 x 32): with CR = 1 all four share the BM rows
//     and split the columns, with CR = 2 they sit 2 x 2, so a 256 x 128
//     tile dequantizes half the weights per flop of a 128 x 256 one for the
//     same LDS traffic (2048x14336x4096 and 512x16384x2048 about 3 % faster,
//     the same bits);
//   * waves 4 .. 3 + NPW (producers) stream the tiles of later iterations
//     (activations and codes PD iterations ahead, in registers), dequantize
//     each weight once into binary16 q * s 2^-f_j and write both tiles into
//     a double-buffered LDS stage.
// So the dequantizing VALU work runs beside the matrix core instead of in
// the MFMA waves' instruction stream; one barrier per iteration hands the
// stages over.  Tiles hold KS = 64 codes of K (128 on the 64-row tiles);
// LDS rows are padded by 16 bytes (the 16-byte fragment reads of 8
// neighbouring rows fall on different banks).
//
// Measured on the 1B / 8B prefill shapes against one 8-wave role-free form
// (every wave staging, dequantizing its own columns in registers and
// issuing MFMAs, two K parities): 512x16384x2048 63.2 -> 55.4 us,
// 2048x14336x4096 342 -> 307 us, 2048x4096x14336 309 -> 276 us.  Alone,
// the consumers reach 1.45 PFLOP/s on 2048x14336x4096 and the producers
// take 225 us: the producers set the pace (their loads, dequantizing VALU
// and LDS writes run in lockstep phases between the barriers; LDS takes
// about 385 GB/s of 16-byte reads and 174 GB/s of 16-byte writes per CU
// here), and 4 producer waves instead of 8, or 3-4 register stages instead
// of 2, were slower or equal.
constexpr int kIterCodes = 64;     // k per iteration (128 on 64-row tiles)
constexpr int kProducerWaves = 8;
constexpr int kStages = 2;         // register stages of the producers

template <int G, int KIND, int TM, int TN, int CR = 1, int NPW = kProducerWaves, int PD = kStages,
          int KSZ = kIterCodes>
__global__ __launch_bounds__(64 * (4 + NPW)) __attribute__((amdgpu_waves_per_eu(1 + NPW / 4, 1 + NPW / 4)))
void gemm_kernel(const uint8_t *__restrict__ w, int64_t row_bytes,
                    const uint16_t *__restrict__ x16, const int *__restrict__ ex,
                    const int *__restrict__ ew, float *__restrict__ y, int64_t s, int64_t m,
                    int64_t n, int nit, float *__restrict__ ws) {
  constexpr int CC = 4 / CR;                     // consumer waves per row group
  constexpr int BM = 32 * TM * CR, BN = 32 * TN * CC;
  constexpr int SB = ScaleTraits<KIND>::bytes;
  constexpr int NPT = 64 * NPW;                  // producer threads
  constexpr int NT = 256 + NPT;                  // threads
  constexpr int KS = KSZ, LDS_ROW = KSZ + 8;     // k per iteration, halves per LDS row
  constexpr int AC = BM * (KS / 8) / NPT;        // 8-half activation chunks per producer
  constexpr int BC = BN * (KS / 16) / NPT;       // 16-code weight chunks per producer
  static_assert(AC >= 1 && BC >= 1, "tile too small for the producer waves");
  __shared__ __attribute__((aligned(16))) _Float16 As[2][BM * LDS_ROW];
  __shared__ __attribute__((aligned(16))) _Float16 Bs[2][BN * LDS_ROW];
  __shared__ int exs[BM];
  __shared__ int ews[BN];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t n0 = (int64_t)blockIdx.x * BN, m0 = (int64_t)blockIdx.y * BM;
  const int64_t kbase = (int64_t)blockIdx.z * nit * KS;   // this split's first code
  const int64_t arows = s - m0 < BM ? s - m0 : BM;
  const int64_t nrows = n - n0 < BN ? n - n0 : BN;

  // The row exponents are staged by the consumer threads (BM, BN <= 256)
  // and published by the first barrier, which the producers pass only after
  // issuing their first tile loads: the two memory round trips overlap.
  for (int t = tid; t < BM; t += NT) exs[t] = t < arows ? ex[m0 + t] : 0;
  for (int t = tid; t < BN; t += NT) ews[t] = KIND == SCALE_F32 && t < nrows ? ew[n0 + t] : 0;

  if (wid >= 4) {
    // ---- producers ----
    const int pt = tid - 256;
    const rsrc_t wr = make_rsrc(w + n0 * row_bytes, (uint32_t)(nrows * row_bytes));
    const rsrc_t xr = make_rsrc(x16 + m0 * m, (uint32_t)(arows * m * 2));
    // activation chunk u: row c / 8, halves 8 (c % 8) .. +8 of the tile's
    // 64 (c = pt + 256 u; 8 threads read one 128-byte row run); weight chunk
    // u: row c / 4, codes 16 (c % 4) .. +16 (4 threads per 64-byte run).  A
    // 16-code chunk never leaves its quantization group (16 | G).
    uint32_t aoff[AC], boff[BC], soff[BC];
    int arow[AC], akq[AC], brow[BC], bkc[BC];
#pragma unroll
    for (int u = 0; u < AC; ++u) {
      const int c = pt + NPT * u;
      arow[u] = c / (KS / 8);
      akq[u] = c % (KS / 8);
      aoff[u] = (uint32_t)((arow[u] * m + kbase + 8 * akq[u]) * 2);
    }
#pragma unroll
    for (int u = 0; u < BC; ++u) {
      const int c = pt + NPT * u;
      brow[u] = c / (KS / 16);
      bkc[u] = c % (KS / 16);
      boff[u] = (uint32_t)(brow[u] * row_bytes + (m / G) * SB + kbase + 16 * bkc[u]);
      soff[u] = (uint32_t)(brow[u] * row_bytes + ((kbase + 16 * bkc[u]) / G) * SB);
    }
    struct Stage {
      u32x4 a[AC], b[BC];
      uint32_t sc[BC];
    };
    // Loads of iteration it are unconditional: activations past m read
    // zeros, codes past the row read bytes whose scale is forced to 0 below,
    // and iterations past the split's range are never stored.
    auto load = [&](Stage &S, int it) {
#pragma unroll
      for (int u = 0; u < AC; ++u) {
        const bool in = kbase + KS * it + 8 * akq[u] < m;
        S.a[u] = bload16(xr, in ? aoff[u] + (uint32_t)(KS * it * 2) : kOutOfRange);
      }
#pragma unroll
      for (int u = 0; u < BC; ++u) S.b[u] = bload16(wr, boff[u] + (uint32_t)(KS * it));
#pragma unroll
      for (int u = 0; u < BC; ++u) {
        const uint32_t o = soff[u] + (uint32_t)((KS * it / G) * SB);
        if constexpr (KIND == SCALE_F16)
          S.sc[u] = bload2(wr, o);
        else
          S.sc[u] = __builtin_amdgcn_raw_buffer_load_b32(wr, o, 0, 0);
      }
    };
    auto store = [&](const Stage &S, int it, int buf) {
#pragma unroll
      for (int u = 0; u < AC; ++u)
        *reinterpret_cast<u32x4 *>(&As[buf][arow[u] * LDS_ROW + 8 * akq[u]]) = S.a[u];
#pragma unroll
      for (int u = 0; u < BC; ++u) {
        _Float16 hs;
        if constexpr (KIND == SCALE_F16)
          hs = __builtin_bit_cast(_Float16, (uint16_t)S.sc[u]);
        else
          hs = (_Float16)__builtin_ldexpf(__builtin_bit_cast(float, S.sc[u]), -ews[brow[u]]);
        const _Float16 h0 = (_Float16)0.0f;
        hs = kbase + KS * it + 16 * bkc[u] < m ? hs : h0;
        const f16x2 s2 = {hs, hs};
        _Float16 *dst = &Bs[buf][brow[u] * LDS_ROW + 16 * bkc[u]];
        *reinterpret_cast<f16x8 *>(dst) = dequant8(S.b[u].x, S.b[u].y, s2);
        *reinterpret_cast<f16x8 *>(dst + 8) = dequant8(S.b[u].z, S.b[u].w, s2);
      }
    };
    // PD register stages: stage u % PD holds iteration u, loaded PD
    // iterations before its store
    Stage S[PD];
#pragma unroll
    for (int u = 0; u < PD; ++u) load(S[u], u);
    __syncthreads();             // the exponents are staged
    store(S[0], 0, 0);
    load(S[0], PD);
    __syncthreads();
    // iteration it: the consumers read LDS stage it & 1; write stage
    // (it + 1) & 1 (read last in iteration it - 1) from registers, which then
    // load iteration it + 1 + PD
    for (int it0 = 0; it0 < nit; it0 += PD) {
#pragma unroll
      for (int u = 0; u < PD; ++u) {
        const int it = it0 + u;
        if (it >= nit) break;
        if (it + 1 < nit) store(S[(u + 1) % PD], it + 1, (it + 1) & 1);
        load(S[(u + 1) % PD], it + 1 + PD);
        __syncthreads();
      }
    }
    return;
  }

  // ---- consumers ----
  const int lr = lane & 31, lh = lane >> 5;
  const int cb = (wid % CC) * 32 * TN;           // this wave's first column in the tile
  const int rb = (wid / CC) * 32 * TM;           // and its first row
  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int t = 0; t < TN; ++t)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][t][v] = 0.0f;
  __syncthreads();               // the exponents are staged
  __syncthreads();               // the first stage is stored
  for (int it = 0; it < nit; ++it) {
    const _Float16 *at = As[it & 1];
    const _Float16 *bt = Bs[it & 1];
#pragma unroll
    for (int ks = 0; ks < KS / 16; ++ks) {
      // v_mfma_f32_32x32x16_f16 operands: lane (lr, lh) holds row / column lr,
      // k = 16 ks + 8 lh .. +8 of this tile, for both A and B
      f16x8 af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        af[i] = *reinterpret_cast<const f16x8 *>(&at[(rb + i * 32 + lr) * LDS_ROW + 16 * ks + 8 * lh]);
#pragma unroll
      for (int t = 0; t < TN; ++t)
        bf[t] = *reinterpret_cast<const f16x8 *>(&bt[(cb + t * 32 + lr) * LDS_ROW + 16 * ks + 8 * lh]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int t = 0; t < TN; ++t)
          acc[i][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[t], acc[i][t], 0, 0, 0);
    }
    __syncthreads();
  }
  // D layout of v_mfma_f32_32x32x16: lane -> column lane % 32, element v ->
  // row 8 (v / 4) + 4 (lane / 32) + v % 4; each output scaled by 2^(e_i + f_j)
  const int rows_left = (int)(s - m0 - rb - lh * 4);
#pragma unroll
  for (int t = 0; t < TN; ++t) {
    const int jc = cb + t * 32 + lr;
    const int64_t col = n0 + jc;
    if (col < n) {
      float *out = (gridDim.z == 1 ? y : ws + (int64_t)blockIdx.z * s * n) + (m0 + rb + lh * 4) * n + col;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int r = i * 32 + (v >> 2) * 8 + (v & 3);
          if (r < rows_left) out[(int64_t)r * n] = __builtin_ldexpf(acc[i][t][v], exs[rb + r + lh * 4] + ews[jc]);
        }
    }
  }
}

// y[i] = sum over splits z (in order) of ws[z][i]; four outputs per thread.
// The loads of up to 8 splits are issued before their adds, so a thread
// waits for one memory round trip per 8 splits rather than one per split.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float *__restrict__ ws,
                                                            float *__restrict__ y, int64_t count,
                                                            int splits) {
  const int64_t i = 4 * ((int64_t)blockIdx.x * blockDim.x + threadIdx.x);
  if (i >= count) return;
  if (i + 4 <= count && (count & 3) == 0) {
    f32x4 v = *reinterpret_cast<const f32x4 *>(ws + i);
    int z = 1;
    for (; z + 8 <= splits; z += 8) {
      f32x4 t[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) t[u] = *reinterpret_cast<const f32x4 *>(ws + (z + u) * count + i);
#pragma unroll
      for (int u = 0; u < 8; ++u) v += t[u];
    }
    // the last splits mod 8: unconditional loads (an index past the last
    // split rereads it) so they too are issued together
    f32x4 t[7];
#pragma unroll
    for (int u = 0; u < 7; ++u) {
      const int zz = z + u < splits ? z + u : splits - 1;
      t[u] = *reinterpret_cast<const f32x4 *>(ws + zz * count + i);
    }
#pragma unroll
    for (int u = 0; u < 7; ++u) v = z + u < splits ? v + t[u] : v;
    *reinterpret_cast<f32x4 *>(y + i) = v;
  } else {
    for (int64_t e = i; e < i + 4 && e < count; ++e) {
      float v = ws[e];
      for (int z = 1; z < splits; ++z) v += ws[z * count + e];
      y[e] = v;
    }
  }
}

template <int G, int KIND, int TM, int TN, int CR = 1, int NPW = kProducerWaves,
          int KS = kIterCodes>
hipError_t launch_t(const LinearArgs &a, const uint16_t *x16, const int *ex, const int *ew,
                       hipStream_t st) {
  constexpr int BM = 32 * TM * CR, BN = 32 * TN * (4 / CR);
  const int64_t nit_all = (a.m + KS - 1) / KS;
  const int64_t gx = (a.n + BN - 1) / BN, gy = (a.s + BM - 1) / BM;
  // Split K when the output tiles alone leave CUs idle (256 CUs, one
  // workgroup each); every split keeps at least 512 codes.
  int64_t splits = 1;
  if (a.ws) {
    while (gx * gy * splits * 2 <= 256 && (nit_all + 2 * splits - 1) / (2 * splits) >= 512 / KS &&
           2 * splits * a.s * a.n <= a.ws_floats)
      splits *= 2;
  }
  int64_t nit = (nit_all + splits - 1) / splits;
  dim3 grid((unsigned)gx, (unsigned)gy, (unsigned)splits), block(64 * (4 + NPW));
  hipLaunchKernelGGL((gemm_kernel<G, KIND, TM, TN, CR, NPW, kStages, KS>), grid, block, 0, st, a.w, a.row_bytes,
                     x16, ex, ew, a.y, a.s, a.m, a.n, (int)nit, a.ws);
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
  else if (a.wn)
    launch_norm16<G>(a, x16, ex, ew, nw, st);
  else if (a.up)
    launch_act16<true, G, true>(a, x16, ex, ew, nw, st);
  else
    launch_act16<true, G>(a, x16, ex, ew, nw, st);
  // 128-row tiles once the rows fill them; two column tiles per consumer
  // wave when the 256-column tiles still give every CU a workgroup.
  if (a.s > 64) {
    const int64_t tiles256 = (a.n + 255) / 256 * ((a.s + 127) / 128);
    // 256 x 128 tiles (2 x 2 consumer waves) once they give every CU a
    // workgroup, else 128 x 256 ones
    const int64_t tiles_tall = (a.n + 127) / 128 * ((a.s + 255) / 256);
    if (tiles_tall >= 256) return launch_t<G, KIND, 4, 2, 2>(a, x16, ex, ew, st);
    if (tiles256 >= 256) return launch_t<G, KIND, 4, 2>(a, x16, ex, ew, st);
    // Rows of at most 4096 codes: 64-row tiles rather than a K split, which
    // costs a reduce launch (about 5 us here).  64 x 64 tiles (2 x 2
    // consumer waves over one 32 x 32 tile each) when they give at most one
    // workgroup per CU, else 64 x 128 ones if those do
    // (1B prompt of 512 rows: o 512x2048x2048 25.0 -> 21.0 us, q|k|v
    // 512x3072x2048 28.6 -> 24.8 us with their pre-pass and reduce).  Both
    // take 128 codes of K per iteration, half the stage hand-overs of 64
    // (o 21.9 -> 20.0-20.4 us, q|k|v 25.2 -> 24.1-24.3 us; 128 x 128 tiles
    // lose with them: down 44.0 -> 44.7-45.2 us), and 8 producer waves (o
    // with 4: 19.9 -> 18.0-18.2 us with 8; q|k|v 24.0 -> 27.2 us with 4).
    // Longer rows keep 128 x 128 tiles: 64-row tiles read each weight tile
    // for twice as many row blocks (down 512x2048x8192 42.7 -> 50.3 us).
    if (a.m <= 4096) {
      const int64_t rb64 = (a.s + 63) / 64;
      if ((a.n + 63) / 64 * rb64 <= 256) return launch_t<G, KIND, 1, 1, 2, 8, 128>(a, x16, ex, ew, st);
      if ((a.n + 127) / 128 * rb64 <= 256)
        return launch_t<G, KIND, 2, 1, 1, kProducerWaves, 128>(a, x16, ex, ew, st);
    }
    return launch_t<G, KIND, 4, 1>(a, x16, ex, ew, st);
  }
  return launch_t<G, KIND, 2, 1>(a, x16, ex, ew, st);
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
