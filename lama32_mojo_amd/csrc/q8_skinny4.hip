// q8_skinny4.hip -- decode-path Q8 linear for 2 <= s <= 4 activation rows
// (f32 x) on the f32 matrix cores of gfx950.
//
// y[b, j] = sum_g scale[j, g] * sum_{k in g} x[b, k] * q[j, k]
// (k_mm_q8, src/llama_q8.mojo:54-93: unscaled dot per group, then one scale
// multiply per group).
//
// With a handful of rows the layer is HBM-bound and the work per streamed
// code must stay at one or two VALU operations.  v_mfma_f32_4x4x1_16b_f32
// computes 16 independent 4x4 outer products per instruction, with f32
// operands, so x needs no splitting into narrower terms:
//   * block b (lanes 4b .. 4b+3) owns the 16-code run [K0 + 16b, +16) of a
//     256-code slab; lane 4b + c holds weight row c's run and batch row
//     4t + c's 16 matching x values;
//   * instruction e (e = 0..15) feeds code e of every run: A = x[4t + c][k],
//     B = q[c][k] (an exact f32 conversion of the byte), so block b's 4x4
//     result is the unscaled dot of its run for 4 batch rows x 4 weight rows;
//   * a run never leaves its scale group (G = 32 or 64), so after the 16
//     instructions the run's partial is scaled by the lane's own scale and
//     added to the output accumulator: 4 FMAs per 16 codes;
//   * the 16 blocks' partials (lanes with equal c) meet through two DPP
//     rotations and LDS at the end, together with the waves' K ranges.
// Per 16 codes a lane spends 16 conversions, 4 FMAs and one scale
// conversion; the matrix cores spend 16 x 8 cycles per TR row groups.
// Two forms.  skinny4_kernel: a wave covers Q quads of weight rows (x
// loaded once per slab and reused Q times) over a contiguous range of
// slabs, and the KW waves of a workgroup split K.  skinny4x_kernel (wide
// matrices): the waves walk all of K together over their own rows and share
// each x slab through LDS.  Nothing is read from memory in the MFMA layout (lanes 4b .. 4b+3
// sit on four different rows, so neighbouring lanes never touch
// neighbouring bytes and the L1 splits such a load into one access per
// lane): codes are loaded 16 lanes per row (256 contiguous bytes), each x row
// of a slab as one 1 KiB load and the slab's scales as whole dwords, all
// staged in an LDS region private to the wave and read back in the MFMA
// layout (code rows padded to 72 dwords and x rows by 4 floats, so the
// ds_read_b128 passes are conflict-free).  Codes and scales are loaded
// DC - 1 slabs ahead of their use, x one slab ahead.  Every load is a
// range-checked buffer load: runs past m, weight rows past n and batch rows
// past s read zeros (and a run past m gets a zero scale).
#include "q8_device.h"
#include "q8_launch.h"

#include <utility>

namespace q8 {
namespace {

constexpr int kSlab = 256;   // codes of a row per slab (16 runs of 16)

template <int KIND>
__device__ __forceinline__ float scale_bits_to_f32(uint32_t v) {
  if constexpr (KIND == SCALE_F16) return f16_bits_to_f32((uint16_t)v);
  else return __builtin_bit_cast(float, v);
}

template <int I>
__device__ __forceinline__ float code_f32(const u32x4 &q) {
  const uint32_t d = I / 4 == 0 ? q.x : I / 4 == 1 ? q.y : I / 4 == 2 ? q.z : q.w;
  return sbyte_to_f32<I % 4>(d);
}

template <int I>
__device__ __forceinline__ float x_f32(const u32x4 (&xv)[4]) {
  const u32x4 &v = xv[I / 4];
  const uint32_t d = I % 4 == 0 ? v.x : I % 4 == 1 ? v.y : I % 4 == 2 ? v.z : v.w;
  return __builtin_bit_cast(float, d);
}

constexpr int DC = 2;   // slabs of codes and scales held in registers
constexpr int DX = 2;   // slabs of x held in registers
constexpr int kXStages = 2;   // slabs held in registers per wave, shared-x form

// Scales of one slab: 4Q rows x SPS bytes (SPS = 256 / G scales), loaded as
// NDW dwords, lane l taking dwords l, l + 64, ... (rows in order, so a load
// covers whole runs of each row).
template <int G, int KIND, int Q>
struct SlabScales {
  static constexpr int SPS = (kSlab / G) * ScaleTraits<KIND>::bytes;
  static constexpr int NDW = 4 * Q * SPS / 4;
  static constexpr int NL = (NDW + 63) / 64;
};

template <int Q, int NL>
struct CodeSlab {
  u32x4 cq[Q];        // quad q: codes [K0 + 16 (lane % 16), +16) of row 4q + lane / 16
  uint32_t sw[NL];    // this lane's dwords of the slab's scales
};
constexpr int kCodeRow = kSlab + 32;   // LDS bytes per staged code row
template <int TR>
struct XSlab {
  u32x4 xq[TR][4];    // x[4t + r][K0 + 4 lane, +4], row r = 0..3 per row group
};
constexpr int kXRow = kSlab + 4;   // LDS floats per staged x row

template <int TR, int Q, int E>
__device__ __forceinline__ void mfma_step(const u32x4 (&cq)[Q], const u32x4 (&xq)[TR][4],
                                          f32x4 (&d)[Q][TR]) {
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const float bq = code_f32<E>(cq[q]);
#pragma unroll
    for (int t = 0; t < TR; ++t) {
      const f32x4 c0 = E == 0 ? f32x4{0.0f, 0.0f, 0.0f, 0.0f} : d[q][t];
      d[q][t] = __builtin_amdgcn_mfma_f32_4x4x1f32(x_f32<E>(xq[t]), bq, c0, 0, 0, 0);
    }
  }
}

template <int TR, int Q, int... E>
__device__ __forceinline__ void mfma_run(const u32x4 (&cq)[Q], const u32x4 (&xq)[TR][4],
                                         f32x4 (&d)[Q][TR],
                                         std::integer_sequence<int, E...>) {
  (mfma_step<TR, Q, E>(cq, xq, d), ...);
}

template <int G, int KIND, int TR, int Q, int KW>
__global__ __launch_bounds__(64 * KW) void skinny4_kernel(const uint8_t *__restrict__ w,
                                                          int64_t row_bytes,
                                                          const float *__restrict__ x,
                                                          float *__restrict__ y, int s, int m,
                                                          int64_t n, int per) {
  constexpr int SB = ScaleTraits<KIND>::bytes;
  // per wave, per (quad, row group): the four 16-lane rows' sums, lanes c
  __shared__ f32x4 red[KW][Q * TR][16];
  __shared__ __attribute__((aligned(16))) float xs[KW][4 * TR][kXRow];
  typedef SlabScales<G, KIND, Q> SS;
  __shared__ uint32_t ss[KW][SS::NDW];
  __shared__ __attribute__((aligned(16))) uint8_t cs_lds[KW][4 * Q][kCodeRow];

  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int b = lane >> 2, c = lane & 3;
  const int64_t j0 = (int64_t)blockIdx.x * 4 * Q;
  const int64_t nrows = n - j0 < 4 * Q ? n - j0 : 4 * Q;
  const rsrc_t wr = make_rsrc(w + j0 * row_bytes, (uint32_t)(nrows * row_bytes));
  // one buffer per x row (empty past s), so reads past m return zeros
  rsrc_t xr[TR][4];
#pragma unroll
  for (int t = 0; t < TR; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      xr[t][r] = make_rsrc(x + (int64_t)(4 * t + r < s ? 4 * t + r : 0) * m,
                           4 * t + r < s ? (uint32_t)m * 4 : 0u);
  const uint32_t cbase = (uint32_t)((m / G) * SB);

  // offsets of this lane's run and scale dwords in slab 0
  uint32_t co[Q], so[SS::NL];
#pragma unroll
  for (int q = 0; q < Q; ++q)
    co[q] = (uint32_t)((4 * q + (lane >> 4)) * row_bytes) + cbase + 16 * (lane & 15);
#pragma unroll
  for (int j = 0; j < SS::NL; ++j) {
    const int i = lane + 64 * j, row = i / (SS::SPS / 4);
    so[j] = i < SS::NDW ? (uint32_t)(row * row_bytes) + 4 * (i % (SS::SPS / 4)) : kOutOfRange;
  }

  // Slabs [s0, s0 + per) of this wave; per is a multiple of DC.  The loads
  // are unconditional: a slab past s1 reads whatever lies there (or zeros
  // past the buffers) and gets zero scales; in the last slab of a row, x
  // past m reads zeros, the codes there are finite bytes of the next row and
  // their scales are forced to zero as well.
  const int s0 = wid * per, s1 = s0 + per;
  auto load_codes = [&](CodeSlab<Q, SS::NL> &sl, int slab) {
    const int k0 = slab * kSlab;
#pragma unroll
    for (int q = 0; q < Q; ++q) sl.cq[q] = bload16(wr, co[q] + k0);
#pragma unroll
    for (int j = 0; j < SS::NL; ++j)
      sl.sw[j] = __builtin_amdgcn_raw_buffer_load_b32(wr, so[j] + (uint32_t)(slab * SS::SPS), 0, 0);
  };
  auto load_x = [&](XSlab<TR> &sl, int slab) {
    const uint32_t o = (uint32_t)(slab * kSlab * 4) + 16 * lane;
#pragma unroll
    for (int t = 0; t < TR; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) sl.xq[t][r] = bload16(xr[t][r], o);
  };
  // Stage a loaded x slab and read it back in the MFMA layout: lane (b, c)
  // gets x[4t + c][K0 + 16b + 4j, +4] for j = 0..3.  A wave's LDS operations
  // run in order, so the region can be rewritten right after it was read.
  float *xw = &xs[wid][0][0];
  auto stage_x = [&](const XSlab<TR> &sl, u32x4 (&xq)[TR][4]) {
#pragma unroll
    for (int t = 0; t < TR; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        *reinterpret_cast<u32x4 *>(xw + (4 * t + r) * kXRow + 4 * lane) = sl.xq[t][r];
#pragma unroll
    for (int t = 0; t < TR; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        xq[t][j] = *reinterpret_cast<const u32x4 *>(xw + (4 * t + c) * kXRow + 16 * b + 4 * j);
  };

  f32x4 acc[Q][TR];
#pragma unroll
  for (int q = 0; q < Q; ++q)
#pragma unroll
    for (int t = 0; t < TR; ++t) acc[q][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // the slab's codes and scales go through the same region order: written,
  // then lane (b, c) reads run b and scale (16b / G) of row 4q + c
  uint32_t *sw = &ss[wid][0];
  uint8_t *cw = &cs_lds[wid][0][0];
  auto compute = [&](const CodeSlab<Q, SS::NL> &cs, const XSlab<TR> &xg, int slab) {
    u32x4 xq[TR][4];
    stage_x(xg, xq);
    u32x4 cq[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q)
      *reinterpret_cast<u32x4 *>(cw + (4 * q + (lane >> 4)) * kCodeRow + 16 * (lane & 15)) =
          cs.cq[q];
#pragma unroll
    for (int q = 0; q < Q; ++q)
      cq[q] = *reinterpret_cast<const u32x4 *>(cw + (4 * q + c) * kCodeRow + 16 * b);
#pragma unroll
    for (int j = 0; j < SS::NL; ++j)
      if (lane + 64 * j < SS::NDW) sw[lane + 64 * j] = cs.sw[j];
    uint32_t sraw[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      // read as the dwords they were stored as (a narrower access type
      // could be reordered above the store)
      const int byte = (4 * q + c) * SS::SPS + (16 * b / G) * SB;
      const uint32_t wd = sw[byte >> 2];
      sraw[q] = KIND == SCALE_F16 ? (wd >> (8 * (byte & 3))) & 0xffffu : wd;
    }
    f32x4 d[Q][TR];
    mfma_run<TR, Q>(cq, xq, d, std::make_integer_sequence<int, 16>{});
    const bool live = slab < s1 && slab * kSlab + 16 * b < m;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      const float sc = live ? scale_bits_to_f32<KIND>(sraw[q]) : 0.0f;
#pragma unroll
      for (int t = 0; t < TR; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[q][t][v] = __builtin_fmaf(d[q][t][v], sc, acc[q][t][v]);
    }
  };

  // per is a multiple of DC (and of DX); slab u of an unrolled step lives in
  // code slot u and x slot u % DX
  CodeSlab<Q, SS::NL> C[DC];
  XSlab<TR> X[DX];
#pragma unroll
  for (int u = 0; u < DC - 1; ++u) load_codes(C[u], s0 + u);
  load_x(X[0], s0);
  for (int i = 0; i < per; i += DC) {
#pragma unroll
    for (int u = 0; u < DC; ++u) {
      load_codes(C[(u + DC - 1) % DC], s0 + i + u + DC - 1);
      load_x(X[(u + 1) % DX], s0 + i + u + 1);
      compute(C[u], X[u % DX], s0 + i + u);
    }
  }

  // Sum over the 16 blocks: lanes 4b + c of one 16-lane row via two
  // rotations, then the four rows and the KW waves through LDS.
#pragma unroll
  for (int q = 0; q < Q; ++q)
#pragma unroll
    for (int t = 0; t < TR; ++t) {
      f32x4 v = acc[q][t];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] += dpp_mov<0x128>(v[e]);   // row_ror:8
        v[e] += dpp_mov<0x124>(v[e]);   // row_ror:4
      }
      if ((lane & 15) < 4) red[wid][q * TR + t][(lane >> 4) * 4 + c] = v;
    }
  __syncthreads();
  // one output per thread: o -> (row group t, batch row r, quad q, c), with
  // consecutive threads on consecutive weight rows
  constexpr int NOUT = 16 * Q * TR;
  for (int o = threadIdx.x; o < NOUT; o += 64 * KW) {
    const int cc = o & 3, q = (o >> 2) % Q, r = (o / (4 * Q)) & 3, t = o / (16 * Q);
    float sum = 0.0f;
    for (int k = 0; k < KW; ++k)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) sum += red[k][q * TR + t][rr * 4 + cc][r];
    const int64_t j = j0 + 4 * q + cc;
    const int bb = 4 * t + r;
    if (j < n && bb < s) y[(int64_t)bb * n + j] = sum;
  }
}

// Shared-x form, for matrices with many rows: the KW waves of a workgroup
// walk every slab of K together, each over its own Q quads of weight rows,
// so a slab of x (4 TR rows x 1 KiB) is loaded once per workgroup (its rows
// split over the waves, each row one coalesced load) into a double-buffered
// LDS region, with one barrier per slab; a workgroup then reads x once per
// 4 Q KW weight rows instead of once per 4 Q.  Codes and scales go through
// the wave's own LDS region as in skinny4_kernel, and no K ranges meet.
template <int G, int KIND, int TR, int Q, int KW, int PD>
__global__ __launch_bounds__(64 * KW) void skinny4x_kernel(const uint8_t *__restrict__ w,
                                                           int64_t row_bytes,
                                                           const float *__restrict__ x,
                                                           float *__restrict__ y, int s, int m,
                                                           int64_t n, int nslab) {
  constexpr int SB = ScaleTraits<KIND>::bytes;
  constexpr int XR = 4 * TR;                 // staged x rows
  constexpr int XPW = (XR + KW - 1) / KW;    // x rows each wave loads
  static_assert(PD >= 2 && PD % 2 == 0, "register stages pair with the two x buffers");
  typedef SlabScales<G, KIND, Q> SS;
  __shared__ __attribute__((aligned(16))) float xs[2][XR][kXRow];
  __shared__ uint32_t ss[KW][SS::NDW];
  __shared__ __attribute__((aligned(16))) uint8_t cs_lds[KW][4 * Q][kCodeRow];
  __shared__ f32x4 red[KW][Q * TR][16];

  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int b = lane >> 2, c = lane & 3;
  // this wave's rows [j0, j0 + 4Q); a wave past n reads zeros
  const int64_t j0 = ((int64_t)blockIdx.x * KW + wid) * 4 * Q;
  const int64_t nrows = n - j0 < 0 ? 0 : n - j0 < 4 * Q ? n - j0 : 4 * Q;
  const rsrc_t wr = make_rsrc(w + (nrows > 0 ? j0 : 0) * row_bytes, (uint32_t)(nrows * row_bytes));
  // x rows wid, wid + KW, ... of the staged XR (empty buffers past s and XR)
  rsrc_t xr[XPW];
#pragma unroll
  for (int u = 0; u < XPW; ++u) {
    const int r = wid + KW * u;
    xr[u] = make_rsrc(x + (int64_t)(r < s ? r : 0) * m, r < s && r < XR ? (uint32_t)m * 4 : 0u);
  }
  const uint32_t cbase = (uint32_t)((m / G) * SB);
  uint32_t co[Q], so[SS::NL];
#pragma unroll
  for (int q = 0; q < Q; ++q)
    co[q] = (uint32_t)((4 * q + (lane >> 4)) * row_bytes) + cbase + 16 * (lane & 15);
#pragma unroll
  for (int j = 0; j < SS::NL; ++j) {
    const int i = lane + 64 * j, row = i / (SS::SPS / 4);
    so[j] = i < SS::NDW ? (uint32_t)(row * row_bytes) + 4 * (i % (SS::SPS / 4)) : kOutOfRange;
  }

  // ok == false (uniform): the loads go to an empty buffer and read nothing
  const rsrc_t none = make_rsrc(w, 0u);
  auto load_codes = [&](CodeSlab<Q, SS::NL> &sl, int slab, bool ok) {
    const rsrc_t r = ok ? wr : none;
    const int k0 = slab * kSlab;
#pragma unroll
    for (int q = 0; q < Q; ++q) sl.cq[q] = bload16(r, co[q] + k0);
#pragma unroll
    for (int j = 0; j < SS::NL; ++j)
      sl.sw[j] = __builtin_amdgcn_raw_buffer_load_b32(r, so[j] + (uint32_t)(slab * SS::SPS), 0, 0);
  };
  auto load_x = [&](u32x4 (&xg)[XPW], int slab, bool ok) {
    const uint32_t o = (uint32_t)(slab * kSlab * 4) + 16 * lane;
#pragma unroll
    for (int u = 0; u < XPW; ++u) xg[u] = bload16(ok ? xr[u] : none, o);
  };
  auto store_x = [&](const u32x4 (&xg)[XPW], int buf) {
#pragma unroll
    for (int u = 0; u < XPW; ++u)
      if (wid + KW * u < XR)
        *reinterpret_cast<u32x4 *>(&xs[buf][wid + KW * u][4 * lane]) = xg[u];
  };

  f32x4 acc[Q][TR];
#pragma unroll
  for (int q = 0; q < Q; ++q)
#pragma unroll
    for (int t = 0; t < TR; ++t) acc[q][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  uint32_t *sw = &ss[wid][0];
  uint8_t *cw = &cs_lds[wid][0][0];
  auto compute = [&](const CodeSlab<Q, SS::NL> &cs, int buf, int slab) {
    u32x4 xq[TR][4];
#pragma unroll
    for (int t = 0; t < TR; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        xq[t][j] = *reinterpret_cast<const u32x4 *>(&xs[buf][4 * t + c][16 * b + 4 * j]);
    u32x4 cq[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q)
      *reinterpret_cast<u32x4 *>(cw + (4 * q + (lane >> 4)) * kCodeRow + 16 * (lane & 15)) =
          cs.cq[q];
#pragma unroll
    for (int j = 0; j < SS::NL; ++j)
      if (lane + 64 * j < SS::NDW) sw[lane + 64 * j] = cs.sw[j];
#pragma unroll
    for (int q = 0; q < Q; ++q)
      cq[q] = *reinterpret_cast<const u32x4 *>(cw + (4 * q + c) * kCodeRow + 16 * b);
    uint32_t sraw[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      const int byte = (4 * q + c) * SS::SPS + (16 * b / G) * SB;
      const uint32_t wd = sw[byte >> 2];
      sraw[q] = KIND == SCALE_F16 ? (wd >> (8 * (byte & 3))) & 0xffffu : wd;
    }
    f32x4 d[Q][TR];
    mfma_run<TR, Q>(cq, xq, d, std::make_integer_sequence<int, 16>{});
    const bool live = slab * kSlab + 16 * b < m;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      const float sc = live ? scale_bits_to_f32<KIND>(sraw[q]) : 0.0f;
#pragma unroll
      for (int t = 0; t < TR; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[q][t][v] = __builtin_fmaf(d[q][t][v], sc, acc[q][t][v]);
    }
  };

  // Slab i is computed from register stage i % PD and x buffer i % 2.  The
  // codes, scales and x of slab j are loaded PD slabs ahead, in the phase of
  // slab j - PD; x of slab i + 1 is stored after the compute of slab i and
  // before the phase's barrier, so a buffer is rewritten only after the
  // barrier that follows every wave's last read of it.  A slab's x is
  // loaded before its codes, so storing the latest x waits for x alone, not
  // for the codes issued after it (loads return in issue order).  Loads and
  // phases are unconditional: past the last slab the offsets are out of
  // range, the loads read zeros and the phase adds nothing (its scales are
  // zero).  A phase inside a branch let the compiler sink the x load into
  // the branch that stores it, one compute later than issued here.
  CodeSlab<Q, SS::NL> C[PD];
  u32x4 X[PD][XPW];
#pragma unroll
  for (int u = 0; u < PD; ++u) {
    load_x(X[u], u, u < nslab);
    load_codes(C[u], u, u < nslab);
  }
  store_x(X[0], 0);
  __syncthreads();
  for (int i0 = 0; i0 < nslab; i0 += PD) {
#pragma unroll
    for (int u = 0; u < PD; ++u) {
      const int i = i0 + u;
      compute(C[u], u & 1, i);
      store_x(X[(u + 1) % PD], (u + 1) & 1);
      __syncthreads();
      load_x(X[u], i + PD, i + PD < nslab);
      load_codes(C[u], i + PD, i + PD < nslab);
    }
  }

  // Sum over the 16 blocks (two rotations within each 16-lane row, then the
  // four rows through the wave's LDS region) and store.
#pragma unroll
  for (int q = 0; q < Q; ++q)
#pragma unroll
    for (int t = 0; t < TR; ++t) {
      f32x4 v = acc[q][t];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] += dpp_mov<0x128>(v[e]);   // row_ror:8
        v[e] += dpp_mov<0x124>(v[e]);   // row_ror:4
      }
      if ((lane & 15) < 4) red[wid][q * TR + t][(lane >> 4) * 4 + c] = v;
    }
  constexpr int NOUT = 16 * Q * TR;
#pragma unroll
  for (int o0 = 0; o0 < NOUT; o0 += 64) {
    const int o = o0 + lane;
    if (o < NOUT) {
      const int cc = o & 3, q = (o >> 2) % Q, r = (o / (4 * Q)) & 3, t = o / (16 * Q);
      float sum = 0.0f;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) sum += red[wid][q * TR + t][rr * 4 + cc][r];
      const int64_t j = j0 + 4 * q + cc;
      const int bb = 4 * t + r;
      if (j < n && bb < s) y[(int64_t)bb * n + j] = sum;
    }
  }
}

template <int G, int KIND, int TR, int Q, int KW>
hipError_t launch_q(const LinearArgs &a, int per, hipStream_t st) {
  const int64_t blocks = (a.n + 4 * Q - 1) / (4 * Q);
  hipLaunchKernelGGL((skinny4_kernel<G, KIND, TR, Q, KW>), dim3((unsigned)blocks),
                     dim3(64 * KW), 0, st, a.w, a.row_bytes, static_cast<const float *>(a.x),
                     a.y, (int)a.s, (int)a.m, a.n, per);
  return hipGetLastError();
}

template <int G, int KIND, int TR, int Q>
hipError_t launch_kw(const LinearArgs &a, hipStream_t st) {
  // Waves per workgroup: the K split (4, 2 or 1 waves, each a multiple of
  // DC slabs) that leaves the fewest empty slabs, the wider on a tie.
  const int64_t nslab = (a.m + kSlab - 1) / kSlab;
  int best = 4, bper = 0;
  int64_t bwaste = -1;
  for (int kw = 4; kw >= 1; kw /= 2) {
    const int64_t per = ((nslab + kw - 1) / kw + DC - 1) / DC * DC;
    const int64_t waste = per * kw - nslab;
    if (bwaste < 0 || waste < bwaste) {
      best = kw;
      bper = (int)per;
      bwaste = waste;
    }
  }
  if (best == 4) return launch_q<G, KIND, TR, Q, 4>(a, bper, st);
  if (best == 2) return launch_q<G, KIND, TR, Q, 2>(a, bper, st);
  return launch_q<G, KIND, TR, Q, 1>(a, bper, st);
}

template <int G, int KIND, int TR>
hipError_t launch_tr(const LinearArgs &a, hipStream_t st) {
  // Four quads per wave (x reused four times) unless that leaves fewer
  // than 512 workgroups.
  if (a.n >= 4 * 4 * 512) return launch_kw<G, KIND, TR, 4>(a, st);
  if (a.n >= 4 * 2 * 512) return launch_kw<G, KIND, TR, 2>(a, st);
  return launch_kw<G, KIND, TR, 1>(a, st);
}

template <int G, int KIND, int TR, int Q, int KW>
hipError_t launch_x(const LinearArgs &a, hipStream_t st) {
  const int64_t blocks = (a.n + 4 * Q * KW - 1) / (4 * Q * KW);
  const int nslab = (int)((a.m + kSlab - 1) / kSlab);
  hipLaunchKernelGGL((skinny4x_kernel<G, KIND, TR, Q, KW, kXStages>), dim3((unsigned)blocks),
                     dim3(64 * KW), 0, st, a.w, a.row_bytes, static_cast<const float *>(a.x),
                     a.y, (int)a.s, (int)a.m, a.n, nslab);
  return hipGetLastError();
}

template <int G, int KIND>
hipError_t launch_g(const LinearArgs &a, hipStream_t st) {
  // Wide matrices read x once per 32 weight rows (shared-x form: 512 or
  // more workgroups from n = 16384); narrower ones split K over the waves.
  if (a.n >= 16384) return launch_x<G, KIND, 1, 2, 4>(a, st);
  return launch_tr<G, KIND, 1>(a, st);
}

}  // namespace

hipError_t launch_skinny4(const LinearArgs &a, hipStream_t st) {
  if (a.s == 0 || a.n == 0) return hipSuccess;
  if (a.s > kSkinny4MaxRows || a.x_is_bf16) return hipErrorInvalidValue;
  if (a.G == 64 && a.kind == SCALE_F16) return launch_g<64, SCALE_F16>(a, st);
  if (a.G == 64 && a.kind == SCALE_F32) return launch_g<64, SCALE_F32>(a, st);
  if (a.G == 32 && a.kind == SCALE_F16) return launch_g<32, SCALE_F16>(a, st);
  if (a.G == 32 && a.kind == SCALE_F32) return launch_g<32, SCALE_F32>(a, st);
  return hipErrorInvalidValue;
}

}  // namespace q8
