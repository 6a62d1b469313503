// q8_skinny.hip -- decode-path Q8 linear for small batches (5 <= s < 32,
// f32 activations) on gfx950 bf16 MFMA.
//
// y[b, j] = sum_g scale[j, g] * sum_{k in g} x[b, k] * q[j, k]
// (k_mm_q8, src/llama_q8.mojo:54-93: unscaled dot per group, then one scale
// multiply per group).
//
// With a few activation rows the layer is still HBM-bound, but a VALU GEMV
// spends s FMAs and s LDS reads of x per code, which stops keeping up with
// HBM at s of about 4.  Here the products run on v_mfma_f32_16x16x32_bf16 with
// the batch rows zero-padded to 16 per row tile:
//   * x is f32: each value is split into hi = bf16(x) and lo = bf16(x - hi)
//     (x - hi is exact in f32), two MFMAs per k-step; the residual error is
//     below 2^-17 |x|;
//   * |q| <= 127 is exact in bf16; one MFMA k-step (32 codes) is exactly one
//     G=32 group or half a G=64 group, each group's partial starts from 0 and
//     is folded into the output with one f32 FMA;
//   * lane (c, q) of a wave feeds weight row c of a 16-row tile; in k-step t
//     (t = 0, 1) of a 64-code slot it supplies codes 32t + 4q .. +4 and
//     32t + 16 + 4q .. +4 (so a k-step never leaves its group of 32), and the
//     matching x[b][k] of batch row b = c of the row tile (read straight from
//     memory, 64 contiguous bytes per row and load: x is a few KiB and stays
//     in L2);
//   * the codes and scales reach that layout through a small LDS region
//     private to each wave: a chunk of 4 slots of 16 rows is read with loads
//     in which each row is one contiguous 256-byte run (4 rows per
//     instruction), the access pattern HBM streams best, and one more load
//     brings the chunk's scales;
//   * the KW waves of a workgroup split K into contiguous ranges of slots and
//     meet in LDS; a workgroup covers NC tiles of 16 weight rows, NC chosen so
//     that the grid still fills the chip.
// All loads are range-checked buffer loads: batch rows past s and weight rows
// past n read as zero.  Wide matrices take the shared-x form further below.
#include "q8_device.h"
#include "q8_launch.h"

#include <type_traits>

namespace q8 {
namespace {

// Raw scales of one 64-code slot (G=64: one scale, G=32: two).
template <int G, int KIND> struct SkinnyScale {
  static constexpr int bytes = (64 / G) * ScaleTraits<KIND>::bytes;
  uint32_t wd[bytes >= 4 ? bytes / 4 : 1];
  __device__ __forceinline__ float get(int gi) const {
    if constexpr (G == 64 && KIND == SCALE_F16) return f16_bits_to_f32((uint16_t)wd[0]);
    else if constexpr (G == 64) return __builtin_bit_cast(float, wd[0]);
    else if constexpr (KIND == SCALE_F16) return f16_bits_to_f32((uint16_t)(wd[0] >> (16 * gi)));
    else return __builtin_bit_cast(float, wd[gi]);
  }
};

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two f32 -> packed hi = bf16(x) and lo = bf16(x - hi), both rounded to
// nearest even (v_cvt_pk_bf16_f32); x - hi is exact in f32.
__device__ __forceinline__ void split2(uint32_t a, uint32_t b, uint32_t &hi, uint32_t &lo) {
  const f32x2_t v = {__builtin_bit_cast(float, a), __builtin_bit_cast(float, b)};
  const uint32_t h = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
  const f32x2_t hf = {__builtin_bit_cast(float, h << 16), __builtin_bit_cast(float, h & 0xffff0000u)};
  lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(v - hf, bf16x2_t));
  hi = h;
}

// 8 f32 (two dwordx4) -> hi and lo bf16 halves.
__device__ __forceinline__ void split_hi_lo(u32x4 a, u32x4 b, bf16x8_t &hi, bf16x8_t &lo) {
  uint32_t h[4], l[4];
  split2(a.x, a.y, h[0], l[0]);
  split2(a.z, a.w, h[1], l[1]);
  split2(b.x, b.y, h[2], l[2]);
  split2(b.z, b.w, h[3], l[3]);
  hi = __builtin_bit_cast(bf16x8_t, u32x4{h[0], h[1], h[2], h[3]});
  lo = __builtin_bit_cast(bf16x8_t, u32x4{l[0], l[1], l[2], l[3]});
}

constexpr int CH = 4;                // 64-code slots per chunk
constexpr int CRB = CH * 64 + 16;    // LDS bytes per weight row of a chunk (16-byte pad)

// Scales of one chunk (CH slots) of one weight row: 8 (G=64 f16), 16 or 32
// (G=32 f32) bytes.
template <int G, int KIND> struct ChunkScale {
  static constexpr int slot_bytes = (64 / G) * ScaleTraits<KIND>::bytes;
  static constexpr int bytes = CH * slot_bytes;
};

template <int G, int KIND, int NC, int TR, int KW>
__global__ __launch_bounds__(64 * KW) void skinny_kernel(const uint8_t *__restrict__ w,
                                                         int64_t row_bytes,
                                                         const float *__restrict__ x,
                                                         float *__restrict__ y, int64_t s,
                                                         int64_t m, int64_t n) {
  constexpr int SB = ScaleTraits<KIND>::bytes;
  typedef ChunkScale<G, KIND> CS;
  typedef SkinnyScale<G, KIND> SS;
  // per-wave staging of one chunk: codes [NC][16 rows][CRB], scales [NC][16 rows][CS::bytes]
  __shared__ __attribute__((aligned(16))) uint8_t lcode[KW][NC][16 * CRB];
  __shared__ __attribute__((aligned(16))) uint8_t lscale[KW][NC][16 * CS::bytes];
  __shared__ f32x4 red[KW > 1 ? KW - 1 : 1][TR * NC][64];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15, q = lane >> 4;
  const int64_t n0 = (int64_t)blockIdx.x * 16 * NC;

  // slots [sl0, sl1) of this wave, processed in chunks of CH slots
  const int nslot = (int)((m + 63) / 64);
  const int per = ((nslot + KW - 1) / KW + CH - 1) / CH * CH;
  const int sl0 = wid * per;
  const int sl1 = sl0 + per < nslot ? sl0 + per : nslot;
  const int cnt = sl1 > sl0 ? sl1 - sl0 : 0;

  const int64_t nrows = n - n0 < 16 * NC ? n - n0 : 16 * NC;
  const rsrc_t wr = make_rsrc(w + n0 * row_bytes, (uint32_t)(nrows * row_bytes));
  // Chunk loads.  Codes: instruction u of a column tile reads rows 4u .. 4u+3,
  // lane -> row 4u + lane / 16, bytes 16 (lane % 16) .. +16 of the chunk's
  // 256 codes (each row a contiguous 256-byte run).  Scales: lane -> row
  // (lane / (CS::bytes / 16)) % 16, 16 bytes at 16 (lane % (CS::bytes / 16))
  // (for 8-byte chunks, row lane % 16): each row's chunk scales in one run.
  constexpr int SLPR = CS::bytes >= 16 ? CS::bytes / 16 : 1;   // lanes per row for scales
  uint32_t vcc[NC], vsc[NC];
  const int srow = (lane / SLPR) % 16, spart = lane % SLPR;
#pragma unroll
  for (int ct = 0; ct < NC; ++ct) {
    vcc[ct] = (uint32_t)((ct * 16 + (lane >> 4)) * row_bytes + (m / G) * SB + (lane & 15) * 16);
    vsc[ct] = (uint32_t)((ct * 16 + srow) * row_bytes + spart * 16);
  }
  typedef typename std::conditional<CS::bytes >= 16, u32x4, u32x2>::type sraw_t;
  auto load_chunk = [&](u32x4 (&cq)[NC][4], sraw_t (&sq)[NC], int sl) {
#pragma unroll
    for (int ct = 0; ct < NC; ++ct) {
#pragma unroll
      for (int u = 0; u < 4; ++u)
        cq[ct][u] = bload16(wr, vcc[ct] + (uint32_t)(4 * u * row_bytes) + sl * 64);
      if constexpr (CS::bytes >= 16)
        sq[ct] = bload16(wr, vsc[ct] + sl * CS::slot_bytes);
      else
        sq[ct] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(wr, vsc[ct] + sl * CS::slot_bytes, 0, 0));
    }
  };
  // Staging puts a slot's codes in MFMA order: entry q (16 bytes) of a row's
  // slot holds, for k-step t = 0, 1, the codes 32t + 4q .. +4 and
  // 32t + 16 + 4q .. +4.  The loaded 16 codes [16p, 16p + 16) of a slot are
  // dwords d = 0..3 with codes 16p + 4d .. +4, i.e. entry q = d, piece p.
  auto stage_chunk = [&](const u32x4 (&cq)[NC][4], const sraw_t (&sq)[NC]) {
    const int js = (lane & 15) >> 2, pp = lane & 3;
#pragma unroll
    for (int ct = 0; ct < NC; ++ct) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        uint8_t *d = &lcode[wid][ct][(4 * u + (lane >> 4)) * CRB + js * 64 + 4 * pp];
        *reinterpret_cast<uint32_t *>(d) = cq[ct][u].x;
        *reinterpret_cast<uint32_t *>(d + 16) = cq[ct][u].y;
        *reinterpret_cast<uint32_t *>(d + 32) = cq[ct][u].z;
        *reinterpret_cast<uint32_t *>(d + 48) = cq[ct][u].w;
      }
      *reinterpret_cast<sraw_t *>(&lscale[wid][ct][srow * CS::bytes + spart * 16]) = sq[ct];
    }
  };

  const rsrc_t xr = make_rsrc(x, (uint32_t)(s * m * 4));
  uint32_t vx[TR];
#pragma unroll
  for (int tr = 0; tr < TR; ++tr) vx[tr] = (uint32_t)(((tr * 16 + c) * m + 4 * q) * 4);
  // activations of slot sl for lane (c, q), b = 16 tr + c, in the codes' MFMA
  // order: x[b][64 sl + 16u + 4q .. +4] for u = 0..3 (u = 0, 1: k-step 0;
  // u = 2, 3: k-step 1), each load 64 contiguous bytes per batch row; a slot
  // past this wave's range or a second half past m reads zeros
  auto load_x = [&](u32x4 (&xa)[TR][4], int sl) {
    const bool lo_ok = sl < sl1;
    const bool hi_ok = lo_ok && sl * 64 + 32 < m;
#pragma unroll
    for (int tr = 0; tr < TR; ++tr) {
      const uint32_t o0 = lo_ok ? vx[tr] + sl * 256 : kOutOfRange;
      const uint32_t o1 = hi_ok ? vx[tr] + sl * 256 + 128 : kOutOfRange;
      xa[tr][0] = bload16(xr, o0);
      xa[tr][1] = bload16(xr, o0 + 64);
      xa[tr][2] = bload16(xr, o1);
      xa[tr][3] = bload16(xr, o1 + 64);
    }
  };

  f32x4 acc[TR][NC];
#pragma unroll
  for (int tr = 0; tr < TR; ++tr)
#pragma unroll
    for (int ct = 0; ct < NC; ++ct) acc[tr][ct] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  u32x4 cq[NC][4];
  sraw_t sq[NC];
  u32x4 xa[2][TR][4];
  load_chunk(cq, sq, sl0);
  load_x(xa[0], sl0);
  load_x(xa[1], sl0 + 1);

  // Whole chunks: a slot past this wave's range meets zero activations (and
  // finite codes) and has its scales forced to 0.
  for (int i0 = 0; i0 < cnt; i0 += CH) {
    const int slc = sl0 + i0;
    // LDS is private to the wave and a wave's LDS operations run in order,
    // so staging the next chunk after this chunk's reads needs no barrier.
    stage_chunk(cq, sq);
    load_chunk(cq, sq, slc + CH);
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int sl = slc + j;
      const bool live = i0 + j < cnt;
      bf16x8_t xh[TR][2], xl[TR][2];
#pragma unroll
      for (int tr = 0; tr < TR; ++tr) {
        split_hi_lo(xa[j & 1][tr][0], xa[j & 1][tr][1], xh[tr][0], xl[tr][0]);
        split_hi_lo(xa[j & 1][tr][2], xa[j & 1][tr][3], xh[tr][1], xl[tr][1]);
      }
      load_x(xa[j & 1], sl + 2);
      const bool hi_ok = sl * 64 + 32 < m;
#pragma unroll
      for (int ct = 0; ct < NC; ++ct) {
        const u32x4 qq = *reinterpret_cast<const u32x4 *>(&lcode[wid][ct][c * CRB + 64 * j + 16 * q]);
        SS sc;
        const uint8_t *sp = &lscale[wid][ct][c * CS::bytes + j * CS::slot_bytes];
        if constexpr (SS::bytes == 8) {
          const u32x2 v = *reinterpret_cast<const u32x2 *>(sp);
          sc.wd[0] = v.x;
          sc.wd[1] = v.y;
        } else if constexpr (SS::bytes == 4) {
          sc.wd[0] = *reinterpret_cast<const uint32_t *>(sp);
        } else {
          sc.wd[0] = *reinterpret_cast<const uint16_t *>(sp);
        }
        const bf16x8_t b0 = codes_to_bf16(qq.x, qq.y);
        const bf16x8_t b1 = codes_to_bf16(qq.z, qq.w);
        const float s0 = live ? sc.get(0) : 0.0f;
        const float s1 = G == 32 ? (live && hi_ok ? sc.get(1) : 0.0f) : s0;
#pragma unroll
        for (int tr = 0; tr < TR; ++tr) {
          const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
          f32x4 t0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xh[tr][0], b0, z, 0, 0, 0);
          t0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xl[tr][0], b0, t0, 0, 0, 0);
          if constexpr (G == 32) {
            f32x4 t1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xh[tr][1], b1, z, 0, 0, 0);
            t1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xl[tr][1], b1, t1, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              acc[tr][ct][v] = __builtin_fmaf(s0, t0[v], acc[tr][ct][v]);
              acc[tr][ct][v] = __builtin_fmaf(s1, t1[v], acc[tr][ct][v]);
            }
          } else {
            t0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xh[tr][1], b1, t0, 0, 0, 0);
            t0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xl[tr][1], b1, t0, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[tr][ct][v] = __builtin_fmaf(s0, t0[v], acc[tr][ct][v]);
          }
        }
      }
    }
  }

  // The KW K ranges meet in LDS; wave 0 adds them in order and stores.
  if (wid > 0) {
#pragma unroll
    for (int tr = 0; tr < TR; ++tr)
#pragma unroll
      for (int ct = 0; ct < NC; ++ct) red[wid - 1][tr * NC + ct][lane] = acc[tr][ct];
  }
  __syncthreads();
  if (wid == 0) {
#pragma unroll
    for (int tr = 0; tr < TR; ++tr)
#pragma unroll
      for (int ct = 0; ct < NC; ++ct) {
        f32x4 v = acc[tr][ct];
        for (int k = 0; k < KW - 1; ++k) v += red[k][tr * NC + ct][lane];
        // D layout of v_mfma_f32_16x16x32: lane -> weight row lane % 16,
        // element e -> batch row 4 (lane / 16) + e
        const int64_t j = n0 + ct * 16 + c;
        if (j < n) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int64_t b = tr * 16 + 4 * q + e;
            if (b < s) y[b * n + j] = v[e];
          }
        }
      }
  }
}

// ---- shared-x form, for matrices with many rows ---------------------------
// The KW waves of a workgroup walk every 256-code slab of K together, each
// over NC tiles of 16 weight rows of its own.  Per slab, each of the 16 TR
// x rows is loaded once per workgroup (one coalesced 1 KiB load, rows split
// over the waves), split once into bf16 hi and lo and stored in a
// double-buffered LDS region (one barrier per slab), so x is read and split
// once per 16 NC KW weight rows.  Codes are loaded 16 lanes per row (256
// contiguous bytes) and the slab's scales as whole dwords, both staged in
// an LDS region private to the wave, and read back in the MFMA layout:
// in k-step ks lane (c, q) takes codes and x at k = 32 ks + 8 q .. +8 of
// weight row c and batch row c.  A k-step lies in one scale group; its
// partial is folded into the output with the lane's scale (G = 64: every
// two k-steps).  Rows are padded in LDS (x by 16 bf16, codes by 16 bytes)
// and the codes are kept in k-step pair order, so every ds_read is a
// conflict-free 16-byte access.  No K ranges meet: each wave's accumulators
// are its outputs.
constexpr int kXSlab = 256;                // codes of a row per slab
constexpr int kXbRow = kXSlab + 16;        // LDS bf16 per staged x row
constexpr int kCbRow = kXSlab + 16;        // LDS bytes per staged code row
constexpr int kXStages = 2;                // slabs held in registers per wave
// waves per SIMD the register allocation must allow: three 4-wave
// workgroups per CU (their LDS, 53 KiB each, fits three times), two 6-wave
// ones
template <int KW> constexpr int kXWavesPerSimd = KW <= 6 ? 3 : 1;

// Narrow matrices split K over ks_n workgroups per row block (slabs
// [k spk, (k + 1) spk) for workgroup k): each writes its partial tile to
// ws, and a second kernel adds the ks_n tiles in order 0 .. ks_n - 1 (so
// the result does not depend on which workgroup ends first).
template <int G, int KIND, int TR, int NC, int KW, int PD>
__global__ __launch_bounds__(64 * KW) __attribute__((amdgpu_waves_per_eu(kXWavesPerSimd<KW>)))
void skinny_x_kernel(const uint8_t *__restrict__ w, int64_t row_bytes, const float *__restrict__ x,
                     float *__restrict__ y, int s, int m, int64_t n, int nslab, int ks_n, int spk,
                     int kmaj, float *__restrict__ ws) {
  constexpr int SB = ScaleTraits<KIND>::bytes;
  constexpr int XR = 16 * TR;                  // staged x rows
  constexpr int XPW = (XR + KW - 1) / KW;      // x rows each wave loads
  constexpr int SPS = (kXSlab / G) * SB;       // scale bytes of a row per slab
  constexpr int NDW = NC * 16 * SPS / 4;       // scale dwords of a wave per slab
  constexpr int NL = (NDW + 63) / 64;
  constexpr int KPG = G / 32;                  // k-steps per scale group
  static_assert(PD >= 2 && PD % 2 == 0, "register stages pair with the two x buffers");
  __shared__ __attribute__((aligned(16))) uint16_t xh[2][XR][kXbRow];
  __shared__ __attribute__((aligned(16))) uint16_t xl[2][XR][kXbRow];
  __shared__ __attribute__((aligned(16))) uint8_t cs[KW][NC * 16][kCbRow];
  __shared__ uint32_t ss[KW][NDW];

  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15, q = lane >> 4;
  // The workgroups of a launch go to the 8 XCDs in turn.  Split-major
  // (kmaj): the ks_n splits of row block rb are workgroups rb, rb + nrb, ...,
  // so with nrb a multiple of 8 they run on one XCD, as does block rb of the
  // launch that adds their partials.  Row-block-major: workgroup kp + ks_n rb,
  // so with ks_n a multiple of 8 each XCD reads only its own slabs of x.
  const int nrb = (int)gridDim.x / ks_n;
  const int kp = kmaj ? (int)blockIdx.x / nrb : (int)blockIdx.x % ks_n;
  const int rb = kmaj ? (int)blockIdx.x % nrb : (int)blockIdx.x / ks_n;
  // this workgroup's slabs [sb, sb + ns)
  const int sb = kp * spk;
  const int ns = nslab - sb < spk ? nslab - sb : spk;
  // this wave's rows [j0, j0 + 16 NC); a wave past n reads zeros
  const int64_t j0 = ((int64_t)rb * KW + wid) * 16 * NC;
  const int64_t nrows = n - j0 < 0 ? 0 : n - j0 < 16 * NC ? n - j0 : 16 * NC;
  const rsrc_t wr = make_rsrc(w + (nrows > 0 ? j0 : 0) * row_bytes, (uint32_t)(nrows * row_bytes));
  // x rows wid, wid + KW, ... (empty buffers past s: zeros; reads past m: zeros)
  rsrc_t xr[XPW];
#pragma unroll
  for (int u = 0; u < XPW; ++u) {
    const int r = wid + KW * u;
    xr[u] = make_rsrc(x + (int64_t)(r < s ? r : 0) * m,
                      r < s && (XR % KW == 0 || r < XR) ? (uint32_t)m * 4 : 0u);
  }
  const uint32_t cbase = (uint32_t)((m / G) * SB);
  uint32_t co[NC][4], so[NL];
#pragma unroll
  for (int t = 0; t < NC; ++t)
#pragma unroll
    for (int u = 0; u < 4; ++u)
      co[t][u] = (uint32_t)((16 * t + 4 * u + (lane >> 4)) * row_bytes) + cbase + 16 * (lane & 15);
#pragma unroll
  for (int j = 0; j < NL; ++j) {
    const int i = lane + 64 * j, row = i / (SPS / 4);
    so[j] = i < NDW ? (uint32_t)(row * row_bytes) + 4 * (i % (SPS / 4)) : kOutOfRange;
  }

  struct Slab {
    u32x4 cq[NC][4];
    uint32_t sw[NL];
  };
  // ok == false (uniform): the loads go to an empty buffer and read nothing
  const rsrc_t none = make_rsrc(w, 0u);
  auto load_codes = [&](Slab &sl, int slab, bool ok) {
    const rsrc_t r = ok ? wr : none;
#pragma unroll
    for (int t = 0; t < NC; ++t)
#pragma unroll
      for (int u = 0; u < 4; ++u) sl.cq[t][u] = bload16(r, co[t][u] + slab * kXSlab);
#pragma unroll
    for (int j = 0; j < NL; ++j)
      sl.sw[j] = __builtin_amdgcn_raw_buffer_load_b32(r, so[j] + (uint32_t)(slab * SPS), 0, 0);
  };
  auto load_x = [&](u32x4 (&xg)[XPW], int slab, bool ok) {
    const uint32_t o = (uint32_t)(slab * kXSlab * 4) + 16 * lane;
#pragma unroll
    for (int u = 0; u < XPW; ++u) xg[u] = bload16(ok ? xr[u] : none, o);
  };
  // split this lane's 4 values of each loaded row into hi and lo bf16
  auto store_x = [&](const u32x4 (&xg)[XPW], int buf) {
#pragma unroll
    for (int u = 0; u < XPW; ++u) {
      uint32_t h0, l0, h1, l1;
      split2(xg[u].x, xg[u].y, h0, l0);
      split2(xg[u].z, xg[u].w, h1, l1);
      const int r = wid + KW * u;
      if (XR % KW == 0 || r < XR) {
        *reinterpret_cast<u32x2 *>(&xh[buf][r][4 * lane]) = u32x2{h0, h1};
        *reinterpret_cast<u32x2 *>(&xl[buf][r][4 * lane]) = u32x2{l0, l1};
      }
    }
  };

  f32x4 acc[NC][TR];
#pragma unroll
  for (int t = 0; t < NC; ++t)
#pragma unroll
    for (int tr = 0; tr < TR; ++tr) acc[t][tr] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  uint8_t *cw = &cs[wid][0][0];
  uint32_t *sws = &ss[wid][0];
  auto compute = [&](const Slab &sl, int buf, int slab) {
    // codes in k-step pair order: entry (q, ks) of a row (the 8 codes lane
    // q feeds in k-step ks) at 64 (ks / 2) + 16 q + 8 (ks % 2), so a lane
    // reads the codes of two k-steps with one 16-byte access; a loaded run
    // of 16 codes (k-step ks, entries q = 2 hh and 2 hh + 1) is written as
    // two 8-byte pieces
    const int hq = lane & 15, kst = hq >> 1;
    const int po = 32 * (kst & ~1) + 32 * (hq & 1) + 8 * (kst & 1);
#pragma unroll
    for (int t = 0; t < NC; ++t)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        // lanes 8-15 of a row store their second piece first, so each of
        // the two stores covers 16 distinct 8-byte slots of a 128-byte
        // span (LDS bank conflicts of the 16-row gate|up launch 1.38 M ->
        // 0.59 M cycles)
        uint8_t *dst = cw + (16 * t + 4 * u + (lane >> 4)) * kCbRow + po;
        const u32x2 p0 = u32x2{sl.cq[t][u].x, sl.cq[t][u].y};
        const u32x2 p1 = u32x2{sl.cq[t][u].z, sl.cq[t][u].w};
        const bool sw = (hq & 8) != 0;
        *reinterpret_cast<u32x2 *>(dst + (sw ? 16 : 0)) = sw ? p1 : p0;
        *reinterpret_cast<u32x2 *>(dst + (sw ? 0 : 16)) = sw ? p0 : p1;
      }
#pragma unroll
    for (int j = 0; j < NL; ++j)
      if (lane + 64 * j < NDW) sws[lane + 64 * j] = sl.sw[j];
    // The slab runs in blocks of KB k-steps (4, or 2 with several tiles);
    // the LDS reads of a block (codes and x) are issued together, one block
    // ahead of the products that use them.  Within a block the products run as
    // independent chains, one per scale group (hi terms of every chain
    // first, then the lo terms), so no MFMA waits on the one issued just
    // before it; the scale FMAs of the block's groups follow its products.
    constexpr int NG = 8 / KPG;                // scale groups per slab
    constexpr int KB = TR * NC > 1 ? 2 : 4;    // k-steps per block
    constexpr int GB = KB / KPG;               // scale groups per block
    // raw scale words of the slab's groups, read with the first block
    uint32_t swd[NG][NC];
    auto read_scales = [&]() {
#pragma unroll
      for (int g = 0; g < NG; ++g)
#pragma unroll
        for (int t = 0; t < NC; ++t) swd[g][t] = sws[((16 * t + c) * SPS + g * SB) >> 2];
    };
    // scale of group g of the slab (k-steps KPG g ..), forced to 0 past m
    auto scale = [&](int g, int t) {
      const int byte = (16 * t + c) * SPS + g * SB;
      const uint32_t raw = KIND == SCALE_F16 ? (swd[g][t] >> (8 * (byte & 3))) & 0xffffu : swd[g][t];
      const bool live = slab * kXSlab + 32 * KPG * g < m;
      return live ? (KIND == SCALE_F16 ? f16_bits_to_f32((uint16_t)raw) : __builtin_bit_cast(float, raw))
                  : 0.0f;
    };
    // register sets of two blocks: block h + 1 is read before block h runs
    u32x2 qq[2][KB][NC];
    bf16x8_t ah[2][KB][TR], al[2][KB][TR];
    auto read_block = [&](int h) {
      const int r = h & 1;
#pragma unroll
      for (int k = 0; k < KB; k += 2)
#pragma unroll
        for (int t = 0; t < NC; ++t) {
          const u32x4 v = *reinterpret_cast<const u32x4 *>(cw + (16 * t + c) * kCbRow + 32 * (KB * h + k) + 16 * q);
          qq[r][k][t] = u32x2{v.x, v.y};
          qq[r][k + 1][t] = u32x2{v.z, v.w};
        }
#pragma unroll
      for (int k = 0; k < KB; ++k)
#pragma unroll
        for (int tr = 0; tr < TR; ++tr) {
          ah[r][k][tr] = *reinterpret_cast<const bf16x8_t *>(&xh[buf][16 * tr + c][32 * (KB * h + k) + 8 * q]);
          al[r][k][tr] = *reinterpret_cast<const bf16x8_t *>(&xl[buf][16 * tr + c][32 * (KB * h + k) + 8 * q]);
        }
    };
    auto run_block = [&](int h) {
      const int r = h & 1;
      bf16x8_t bq[KB][NC];
#pragma unroll
      for (int k = 0; k < KB; ++k)
#pragma unroll
        for (int t = 0; t < NC; ++t) bq[k][t] = codes_to_bf16(qq[r][k][t].x, qq[r][k][t].y);
      // k-step KB h + k is step kk = k % KPG of the block's group k / KPG;
      // products ordered by (part, kk, group)
      f32x4 d[GB][NC][TR];
#pragma unroll
      for (int part = 0; part < 2; ++part)
#pragma unroll
        for (int kk = 0; kk < KPG; ++kk)
#pragma unroll
          for (int gg = 0; gg < GB; ++gg) {
            const int k = gg * KPG + kk;
#pragma unroll
            for (int t = 0; t < NC; ++t)
#pragma unroll
              for (int tr = 0; tr < TR; ++tr) {
                const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
                const f32x4 cin = part == 0 && kk == 0 ? z : d[gg][t][tr];
                d[gg][t][tr] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    part == 0 ? ah[r][k][tr] : al[r][k][tr], bq[k][t], cin, 0, 0, 0);
              }
          }
#pragma unroll
      for (int gg = 0; gg < GB; ++gg)
#pragma unroll
        for (int t = 0; t < NC; ++t)
#pragma unroll
          for (int tr = 0; tr < TR; ++tr)
#pragma unroll
            for (int v = 0; v < 4; ++v)
              acc[t][tr][v] = __builtin_fmaf(scale(h * GB + gg, t), d[gg][t][tr][v], acc[t][tr][v]);
    };
    read_block(0);
    read_scales();
#pragma unroll
    for (int h = 0; h < 8 / KB; ++h) {
      if (h + 1 < 8 / KB) read_block(h + 1);
      // keep the reads ahead of the block's arithmetic
      __builtin_amdgcn_sched_barrier(0);
      run_block(h);
    }
  };

  // Slab i is computed from register stage i % PD and x buffer i % 2.  The
  // codes, scales and x of slab j are loaded PD slabs ahead, in the phase of
  // slab j - PD, so PD - 1 slabs stay in flight while one is computed; x of
  // slab i + 1 is split and stored after the compute of slab i and before
  // the phase's barrier, so a buffer is rewritten only after the barrier
  // that follows every wave's last read of it.  A slab's x is loaded before
  // its codes: loads return in issue order, so storing x of slab i + 1 (the
  // latest x in flight) waits for x alone and not for the codes of slab
  // i + 2 issued after it (codes first made that store wait for every load:
  // Qwen3-8B gate|up at s = 16 34.6 -> 31.7 us).  The loads are
  // unconditional (a slab past this workgroup's range reads nothing: its
  // offsets are out of range), and a phase past the last slab is skipped by
  // a uniform branch that holds no loads.
  Slab C[PD];
  u32x4 X[PD][XPW];
#pragma unroll
  for (int u = 0; u < PD; ++u) {
    load_x(X[u], sb + u, u < ns);
    load_codes(C[u], sb + u, u < ns);
  }
  store_x(X[0], 0);
  __syncthreads();
  for (int i0 = 0; i0 < ns; i0 += PD) {
#pragma unroll
    for (int u = 0; u < PD; ++u) {
      const int i = i0 + u;
      if (i < ns) {
        compute(C[u], u & 1, sb + i);
        store_x(X[(u + 1) % PD], (u + 1) & 1);
        __syncthreads();
      }
      load_x(X[u], sb + i + PD, i + PD < ns);
      load_codes(C[u], sb + i + PD, i + PD < ns);
    }
  }

  // D layout of v_mfma_f32_16x16x32: lane -> weight row lane % 16, element
  // v -> batch row 4 (lane / 16) + v
  if (ks_n == 1) {
#pragma unroll
    for (int t = 0; t < NC; ++t) {
      const int64_t j = j0 + 16 * t + c;
      if (j < n) {
#pragma unroll
        for (int tr = 0; tr < TR; ++tr)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int bb = 16 * tr + 4 * q + v;
            if (bb < s) y[(int64_t)bb * n + j] = acc[t][tr][v];
          }
      }
    }
    return;
  }
  // A K split writes the first s rows of its partial tile [XR batch rows]
  // [ROWS weight rows] (zeros past n) to tile kp nrb + rb of ws.
  constexpr int ROWS = 16 * NC * KW;
  float *part = ws + ((int64_t)kp * nrb + rb) * (XR * ROWS);
#pragma unroll
  for (int t = 0; t < NC; ++t)
#pragma unroll
    for (int tr = 0; tr < TR; ++tr)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int bb = 16 * tr + 4 * q + v;
        if (bb < s) part[bb * ROWS + wid * 16 * NC + 16 * t + c] = acc[t][tr][v];
      }
}

// y = the sum of the ks_n partial tiles of each row block, added in split
// order 0 .. ks_n - 1 (so the result does not depend on which workgroup
// ended first).  Block rb adds the tiles of row block rb (with a
// split-major grid, on the XCD that wrote them); a thread takes 4
// consecutive entries and issues the loads of up to 8 splits before adding
// them.
template <int XR, int ROWS>
__global__ __launch_bounds__(256) void xsplit_reduce_kernel(const float *__restrict__ ws,
                                                            float *__restrict__ y, int s, int64_t n,
                                                            int nrb, int ks_n) {
  constexpr int PT = XR * ROWS;
  const int rb = blockIdx.x;
  const float *p0 = ws + (int64_t)rb * PT;
  const int64_t stride = (int64_t)nrb * PT;   // between the splits of a tile
  for (int e = 4 * (int)threadIdx.x; e < s * ROWS; e += 1024) {
    f32x4 v = *reinterpret_cast<const f32x4 *>(p0 + e);
    for (int z0 = 1; z0 < ks_n; z0 += 8) {
      f32x4 t[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int z = z0 + u < ks_n ? z0 + u : ks_n - 1;   // past the last: reread it
        t[u] = *reinterpret_cast<const f32x4 *>(p0 + z * stride + e);
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) v = z0 + u < ks_n ? v + t[u] : v;
    }
    const int bb = e / ROWS;
    const int64_t j = (int64_t)rb * ROWS + e % ROWS;
    float *yp = y + (int64_t)bb * n + j;
    if (j + 3 < n && (reinterpret_cast<uintptr_t>(yp) & 15) == 0) {
      *reinterpret_cast<f32x4 *>(yp) = v;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (j + i < n) yp[i] = v[i];
    }
  }
}

// Row blocks of 16 NC KW weight rows; with ks_n > 1 each is split over
// ks_n workgroups of spk slabs, whose partial tiles (ks_n nrb 16 TR ROWS
// floats of the workspace) a second launch adds; kmaj orders the grid
// split-major.
template <int G, int KIND, int TR, int NC, int KW>
hipError_t launch_x(const LinearArgs &a, int ks_n, hipStream_t st, bool kmaj = false) {
  constexpr int ROWS = 16 * NC * KW, XR = 16 * TR;
  const int64_t nrb = (a.n + ROWS - 1) / ROWS;
  const int nslab = (int)((a.m + kXSlab - 1) / kXSlab);
  if (ks_n > nslab) ks_n = nslab;
  if (ks_n > 1 && (!a.ws || ks_n * nrb * XR * ROWS > a.ws_floats)) ks_n = 1;
  const int spk = (nslab + ks_n - 1) / ks_n;
  ks_n = (nslab + spk - 1) / spk;   // no empty split
  constexpr int PD = kXStages;
  hipLaunchKernelGGL((skinny_x_kernel<G, KIND, TR, NC, KW, PD>), dim3((unsigned)(nrb * ks_n)),
                     dim3(64 * KW), 0, st, a.w, a.row_bytes, static_cast<const float *>(a.x),
                     a.y, (int)a.s, (int)a.m, a.n, nslab, ks_n, spk, (int)kmaj, a.ws);
  if (ks_n > 1)
    hipLaunchKernelGGL((xsplit_reduce_kernel<XR, ROWS>), dim3((unsigned)nrb), dim3(256), 0, st,
                       a.ws, a.y, (int)a.s, a.n, (int)nrb, ks_n);
  return hipGetLastError();
}

template <int G, int KIND, int NC, int TR, int KW>
hipError_t launch_nc(const LinearArgs &a, hipStream_t st) {
  const int64_t blocks = (a.n + 16 * NC - 1) / (16 * NC);
  hipLaunchKernelGGL((skinny_kernel<G, KIND, NC, TR, KW>), dim3((unsigned)blocks), dim3(64 * KW),
                     0, st, a.w, a.row_bytes, static_cast<const float *>(a.x), a.y, a.s, a.m, a.n);
  return hipGetLastError();
}

template <int G, int KIND, int TR>
hipError_t launch_tr(const LinearArgs &a, hipStream_t st) {
  // Two column tiles per wave (x is loaded and split once per tile pair)
  // while that keeps >= 512 workgroups (two per CU); short weight matrices
  // split K over 8 waves instead of 4.  (Four tiles per wave need 86 KiB of
  // staging per workgroup, which halves the waves per CU and loses more than
  // the shared x saves.)
  const int64_t tiles = (a.n + 15) / 16;
  if (tiles >= 2 * 512) return launch_nc<G, KIND, 2, TR, 4>(a, st);
  if (tiles >= 256) return launch_nc<G, KIND, 1, TR, 4>(a, st);
  return launch_nc<G, KIND, 1, TR, 8>(a, st);
}

// Shared-x form with K split over ks_n workgroups per 64-row block, ks_n
// chosen for about `target` workgroups in all.  Short rows order the grid
// split-major: the partial tiles (ks_n x 4 KiB per row block) then stay in
// one XCD's L2 for the reduce, while every XCD reads all of x (16 rows x m
// floats, 256 KiB at m = 4096); long rows (m >= 8192) keep x per XCD
// instead (Qwen3-8B at 16 rows, against row-block-major: q|k|v 15.98 ->
// 15.23 us, o 12.57 -> 11.47 us; down 21.6 us split-major, 21.2 not).
template <int G, int KIND>
hipError_t launch_x_split(const LinearArgs &a, int64_t target, hipStream_t st) {
  const int64_t nrb = (a.n + 63) / 64;
  return launch_x<G, KIND, 1, 1, 4>(a, (int)((target + nrb - 1) / nrb), st, a.m < 8192);
}

template <int G, int KIND>
hipError_t launch_g(const LinearArgs &a, hipStream_t st) {
  // Shared x where the matrix gives it enough workgroups (one 16-row tile
  // per wave, 64 rows per workgroup, from n = 16384; with two row tiles,
  // 256 rows per 8-wave workgroup, vocabulary-sized matrices only), or with
  // K split over workgroups: long rows (about 512 workgroups) and, from 9
  // batch rows on, narrower matrices (about 768), where the K split over the
  // waves of the per-wave-x form reads x too often.
  if (a.s <= 16) {
    // 96-row workgroups where they make one per CU and 64-row ones would
    // make between one and two per CU (Qwen3-8B gate|up at s = 16: 36.6 ->
    // 34.1 us); vocabulary-sized matrices keep 64 rows (lm_head 170 us
    // against 210)
    if (a.n > 256 * 64 && a.n <= 256 * 96) return launch_x<G, KIND, 1, 1, 6>(a, 1, st);
    if (a.n >= 16384) return launch_x<G, KIND, 1, 1, 4>(a, 1, st);
    if (a.m >= 8192) return launch_x_split<G, KIND>(a, 512, st);
    if (a.s > 8) return launch_x_split<G, KIND>(a, 768, st);
    return launch_tr<G, KIND, 1>(a, st);
  }
  if (a.n >= 65536) return launch_x<G, KIND, 2, 2, 8>(a, 1, st);
  return launch_tr<G, KIND, 2>(a, st);
}

}  // namespace

hipError_t launch_skinny(const LinearArgs &a, hipStream_t st) {
  if (a.s == 0 || a.n == 0) return hipSuccess;
  if (a.s > 32 || a.x_is_bf16) return hipErrorInvalidValue;
  if (a.G == 64 && a.kind == SCALE_F16) return launch_g<64, SCALE_F16>(a, st);
  if (a.G == 64 && a.kind == SCALE_F32) return launch_g<64, SCALE_F32>(a, st);
  if (a.G == 32 && a.kind == SCALE_F16) return launch_g<32, SCALE_F16>(a, st);
  if (a.G == 32 && a.kind == SCALE_F32) return launch_g<32, SCALE_F32>(a, st);
  return hipErrorInvalidValue;
}

}  // namespace q8
