// q8_launch.h -- host-side launchers of the gfx950 kernels (internal).
//
// The C ABI (q8hip_api.cpp) validates every argument, resolves buffer
// offsets to device pointers and then calls one of these.  Each launcher
// only picks a kernel variant and a grid; it trusts its arguments.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace q8 {

struct PackArgs {
  const void *src;       // first element of row 0 (bf16 or f32)
  int src_is_f32;
  int64_t n, m;
  uint8_t *dst;          // byte address of packed row 0
  int64_t dst_row_bytes; // packed row stride in bytes
  int G, kind;
};
hipError_t launch_pack(const PackArgs &a, hipStream_t st);

struct LinearArgs {
  const uint8_t *w;      // byte address of packed row 0
  int64_t row_bytes;     // packed row stride in bytes
  const void *x;         // activations [s, m] (f32 or bf16), row stride m
  int x_is_bf16;
  float *y;              // outputs [s, n] f32, row stride n
  int64_t s, m, n;
  int G, kind;
  // Split-K workspace for the GEMM (null: no split): room for ws_floats
  // partial sums.
  float *ws = nullptr;
  int64_t ws_floats = 0;
};
// Decode path (s small, f32 x): VALU GEMV.
hipError_t launch_gemv(const LinearArgs &a, hipStream_t st);
// Prefill path: MFMA GEMM (bf16 x, or f32 x split into two bf16 terms).
hipError_t launch_gemm(const LinearArgs &a, hipStream_t st);
// Small batches (2 <= s <= 32, f32 x): MFMA over zero-padded 16-row tiles.
hipError_t launch_skinny(const LinearArgs &a, hipStream_t st);

struct GatherArgs {
  const uint8_t *w;      // byte address of packed row 0 of the table
  int64_t row_bytes;
  const int32_t *ids;
  float *y;
  int64_t s, d, vocab;
  int G, kind;
};
hipError_t launch_embed_gather(const GatherArgs &a, hipStream_t st);

}  // namespace q8
