// q8_calib.hip -- calibration kernels for the measurement side of the Q8
// path (libq8calib.so, loaded only by bench.py --workload calib; not part
// of libq8hip.so or its C ABI).  Each entry point times its own kernels
// with HIP events around replays of a captured graph and returns the
// figure the roofline arguments use:
//   q8calib_empty_node_us   one dependent empty kernel node of a graph (the
//                           kernel-boundary floor every launch of a decode
//                           step pays);
//   q8calib_stream_us       a plain streaming read of `bytes` (16-byte
//                           non-temporal loads, grid-stride), rotated over
//                           copies larger than the 256 MB Infinity Cache
//                           (the practical HBM ceiling at a GEMV's size);
//   q8calib_cu_read_us      `blocks` workgroups each reading its own
//                           bytes_per_block (every load issued before use):
//                           how fast a few CUs pull a small tensor, e.g.
//                           the 2 MB of K and V of one decode layer;
//   q8calib_mfma_tflops     register-only v_mfma_f32_32x32x16_f16 loops on
//                           random binary16 operands (the matrix-core
//                           ceiling a dequant-GEMM can approach).
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdlib>
#include <vector>

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__global__ void empty_kernel(unsigned *out) {
  if (threadIdx.x == 4096) out[0] = 0;            // never true: keeps the kernel
}

__global__ __launch_bounds__(256) void stream_kernel(const u32x4 *__restrict__ src, uint64_t n16,
                                                     unsigned *out) {
  u32x4 acc = {0u, 0u, 0u, 0u};
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  // four independent loads in flight per thread and step
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const u32x4 a = __builtin_nontemporal_load(src + i);
    const u32x4 b = __builtin_nontemporal_load(src + i + stride);
    const u32x4 c = __builtin_nontemporal_load(src + i + 2 * stride);
    const u32x4 d = __builtin_nontemporal_load(src + i + 3 * stride);
    acc ^= a ^ b ^ c ^ d;
  }
  for (; i < n16; i += stride) acc ^= __builtin_nontemporal_load(src + i);
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9e3779b9u) out[1] = 1u;   // data-dependent, rare
}

template <int NL>
__global__ __launch_bounds__(1024) void cu_read_kernel(const u32x4 *__restrict__ src,
                                                       uint64_t per16, unsigned *out) {
  const u32x4 *p = src + (uint64_t)blockIdx.x * per16;
  u32x4 v[NL];
#pragma unroll
  for (int u = 0; u < NL; ++u) {
    const uint64_t k = threadIdx.x + (uint64_t)u * blockDim.x;
    v[u] = k < per16 ? __builtin_nontemporal_load(p + k) : u32x4{0u, 0u, 0u, 0u};
  }
  u32x4 acc = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int u = 0; u < NL; ++u) acc ^= v[u];
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9e3779b9u) out[2] = 1u;
}

// 8 independent accumulator chains per wave; the operands are random
// binary16 values loaded once (per lane) from `ops`.
__global__ __launch_bounds__(256) void mfma_kernel(const f16x8 *__restrict__ ops, int iters,
                                                   float *out) {
  const int lane = threadIdx.x & 63;
  const f16x8 a0 = ops[lane], a1 = ops[64 + lane], b0 = ops[128 + lane], b1 = ops[192 + lane];
  f32x16 acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[j][v] = 0.0f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16((j & 1) ? a1 : a0, (j & 2) ? b1 : b0,
                                                       acc[j], 0, 0, 0);
  }
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int v = 0; v < 16; ++v) s += acc[j][v];
  if (s == 1234.5f) out[0] = s;                    // keeps every chain
}

struct Timer {
  hipEvent_t a = nullptr, b = nullptr;
  Timer() {
    (void)hipEventCreate(&a);
    (void)hipEventCreate(&b);
  }
  ~Timer() {
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
  }
};

// Captures `launch(i)` for i < nodes into one graph on a fresh stream,
// replays it once to warm up, then reps times between two events; returns
// microseconds per node (0 on a HIP error).
template <typename F>
float time_graph(int nodes, int reps, F launch) {
  hipStream_t st = nullptr;
  if (hipStreamCreateWithFlags(&st, hipStreamNonBlocking) != hipSuccess) return 0.0f;
  hipGraph_t g = nullptr;
  hipGraphExec_t ge = nullptr;
  float us = 0.0f;
  if (hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal) == hipSuccess) {
    for (int i = 0; i < nodes; ++i) launch(i, st);
    if (hipStreamEndCapture(st, &g) == hipSuccess &&
        hipGraphInstantiate(&ge, g, nullptr, nullptr, 0) == hipSuccess) {
      Timer t;
      bool ok = hipGraphLaunch(ge, st) == hipSuccess && hipStreamSynchronize(st) == hipSuccess &&
                hipEventRecord(t.a, st) == hipSuccess;
      for (int r = 0; ok && r < reps; ++r) ok = hipGraphLaunch(ge, st) == hipSuccess;
      ok = ok && hipEventRecord(t.b, st) == hipSuccess && hipEventSynchronize(t.b) == hipSuccess;
      float ms = 0.0f;
      if (ok && hipEventElapsedTime(&ms, t.a, t.b) == hipSuccess)
        us = ms * 1000.0f / (float)(reps * nodes);
    }
  }
  if (ge) (void)hipGraphExecDestroy(ge);
  if (g) (void)hipGraphDestroy(g);
  (void)hipStreamDestroy(st);
  return us;
}

}  // namespace

extern "C" {

int q8calib_empty_node_us(int nodes, int reps, float *us) {
  unsigned *out = nullptr;
  if (nodes <= 0 || reps <= 0 || !us || hipMalloc(&out, 64) != hipSuccess) return -1;
  *us = time_graph(nodes, reps, [&](int, hipStream_t st) {
    hipLaunchKernelGGL(empty_kernel, dim3(256), dim3(256), 0, st, out);
  });
  (void)hipFree(out);
  return *us > 0.0f ? 0 : -2;
}

int q8calib_stream_us(uint64_t bytes, int copies, int grid, int reps, float *us) {
  if (bytes < 16 || bytes % 16 || copies <= 0 || grid <= 0 || reps <= 0 || !us) return -1;
  u32x4 *buf = nullptr;
  unsigned *out = nullptr;
  if (hipMalloc(&buf, bytes * (uint64_t)copies) != hipSuccess) return -3;
  if (hipMalloc(&out, 64) != hipSuccess || hipMemset(buf, 0x5a, bytes * (uint64_t)copies) != hipSuccess) {
    (void)hipFree(buf);
    return -3;
  }
  const uint64_t n16 = bytes / 16;
  *us = time_graph(copies, reps, [&](int i, hipStream_t st) {
    hipLaunchKernelGGL(stream_kernel, dim3(grid), dim3(256), 0, st, buf + (uint64_t)i * n16, n16,
                       out);
  });
  (void)hipFree(buf);
  (void)hipFree(out);
  return *us > 0.0f ? 0 : -2;
}

int q8calib_cu_read_us(int blocks, int threads, uint64_t bytes_per_block, int copies, int reps,
                       float *us) {
  if (blocks <= 0 || threads <= 0 || threads > 1024 || threads % 64 || bytes_per_block < 16 ||
      bytes_per_block % 16 || copies <= 0 || reps <= 0 || !us)
    return -1;
  const uint64_t per16 = bytes_per_block / 16;
  const uint64_t nl = (per16 + threads - 1) / threads;
  if (nl > 16) return -1;
  const uint64_t region = (uint64_t)blocks * bytes_per_block;
  u32x4 *buf = nullptr;
  unsigned *out = nullptr;
  if (hipMalloc(&buf, region * (uint64_t)copies) != hipSuccess) return -3;
  if (hipMalloc(&out, 64) != hipSuccess || hipMemset(buf, 0x33, region * (uint64_t)copies) != hipSuccess) {
    (void)hipFree(buf);
    return -3;
  }
  auto launch = [&](int i, hipStream_t st) {
    const u32x4 *src = buf + (uint64_t)i * (region / 16);
    if (nl <= 1)
      hipLaunchKernelGGL(cu_read_kernel<1>, dim3(blocks), dim3(threads), 0, st, src, per16, out);
    else if (nl <= 2)
      hipLaunchKernelGGL(cu_read_kernel<2>, dim3(blocks), dim3(threads), 0, st, src, per16, out);
    else if (nl <= 4)
      hipLaunchKernelGGL(cu_read_kernel<4>, dim3(blocks), dim3(threads), 0, st, src, per16, out);
    else if (nl <= 8)
      hipLaunchKernelGGL(cu_read_kernel<8>, dim3(blocks), dim3(threads), 0, st, src, per16, out);
    else
      hipLaunchKernelGGL(cu_read_kernel<16>, dim3(blocks), dim3(threads), 0, st, src, per16, out);
  };
  *us = time_graph(copies, reps, launch);
  (void)hipFree(buf);
  (void)hipFree(out);
  return *us > 0.0f ? 0 : -2;
}

int q8calib_mfma_tflops(int blocks, int iters, int reps, float *tflops) {
  if (blocks <= 0 || iters <= 0 || reps <= 0 || !tflops) return -1;
  std::vector<uint16_t> host(256 * 8);
  uint32_t r = 12345u;
  for (auto &h : host) {
    r = r * 1664525u + 1013904223u;
    // random binary16 in +-[0.5, 2): sign, exponent 14 or 15, random mantissa
    h = (uint16_t)(((r >> 31) << 15) | ((14u + ((r >> 30) & 1u)) << 10) | ((r >> 8) & 0x3ffu));
  }
  f16x8 *ops = nullptr;
  float *out = nullptr;
  if (hipMalloc(&ops, host.size() * 2) != hipSuccess) return -3;
  if (hipMalloc(&out, 64) != hipSuccess ||
      hipMemcpy(ops, host.data(), host.size() * 2, hipMemcpyHostToDevice) != hipSuccess) {
    (void)hipFree(ops);
    return -3;
  }
  const float us = time_graph(4, reps, [&](int, hipStream_t st) {
    hipLaunchKernelGGL(mfma_kernel, dim3(blocks), dim3(256), 0, st, ops, iters, out);
  });
  (void)hipFree(ops);
  (void)hipFree(out);
  if (us <= 0.0f) return -2;
  const double flops = (double)blocks * 4 * iters * 8 * (2.0 * 32 * 32 * 16);
  *tflops = (float)(flops / (us * 1e-6) / 1e12);
  return 0;
}

}  // extern "C"
