// q8hip_api.cpp -- the C ABI of libq8hip.so (declared in include/q8hip.h).
//
// Host side of the Q8 path: contexts (one HIP stream each), buffers
// (arenas addressed by element offsets, as the reference's Weights / Acts,
// src/resident.mojo:15-58 and src/llama_common.mojo:578-606), argument
// validation, kernel dispatch and HIP-graph capture.  Every entry point
// validates all of its arguments before the first HIP call, so error paths
// behave the same on a host-only context (device Q8_DEVICE_NONE) as on a GPU.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>
#include <string>

#include "../../include/q8hip.h"
#include "q8_launch.h"

struct q8_ctx {
  int device = -1;
  bool host_only = true;
  hipStream_t own = nullptr;
  hipStream_t stream = nullptr;
  std::string err;
  // Split-K workspace of the prefill GEMM (partial sums).  A split only
  // happens while tiles x splits stay within 256 workgroups of 64 x 128
  // outputs, so 2 Mi floats always suffice; 4 Mi leaves room.
  // The decode attention's partial records use it too: both run in stream
  // order on this context.
  float *gemm_ws = nullptr;
  // Binary16 copy of the activation rows of a prefill GEMM and their
  // power-of-two factors (launch_gemm); longer inputs run in row chunks.
  void *act16 = nullptr;
  // Pinned staging for file -> device uploads (q8_st_upload): two halves,
  // allocated on first use.
  void *stage = nullptr;
  hipEvent_t stage_ev[2] = {nullptr, nullptr};
};

namespace {
constexpr int64_t kGemmWsFloats = (int64_t)4 << 20;
constexpr int64_t kAct16Bytes = (int64_t)64 << 20;
}

struct q8_buf {
  void *ptr = nullptr;
  uint64_t size = 0;
  bool owned = false;
  q8_ctx *ctx = nullptr;
};

namespace {

// Message of the last failing q8_create or q8_linear_noalloc on this thread
// (calls that have no context to hold it).
thread_local std::string g_create_err;

int fail(q8_ctx *ctx, int code, const char *fmt, ...) {
  char msg[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(msg, sizeof msg, fmt, ap);
  va_end(ap);
  if (ctx) ctx->err = msg;
  else g_create_err = msg;
  return code;
}

int ok(q8_ctx *ctx) {
  if (ctx) ctx->err.clear();
  return Q8_OK;
}

int hip_fail(q8_ctx *ctx, hipError_t e, const char *what) {
  return fail(ctx, Q8_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

bool valid_layout(int G, int kind) {
  return (G == 32 || G == 64) && (kind == Q8_SCALE_F16 || kind == Q8_SCALE_F32);
}

int64_t rowstride_u16(int64_t m, int G, int kind) {
  return (m / G) * (kind == Q8_SCALE_F32 ? 2 : 1) + m / 2;
}

// a * b + c <= limit without overflow (all non-negative).
bool fits(uint64_t off, uint64_t count, uint64_t elem, uint64_t limit_bytes) {
  unsigned __int128 end = ((unsigned __int128)off + count) * elem;
  return end <= limit_bytes;
}

bool overlaps(uint64_t a0, uint64_t a1, uint64_t b0, uint64_t b1) {
  return a0 < b1 && b0 < a1;
}

int check_ctx(q8_ctx *ctx) {
  if (!ctx) return fail(nullptr, Q8_ERR_ARG, "null context");
  return Q8_OK;
}

int set_device(q8_ctx *ctx) {
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipSetDevice");
  return Q8_OK;
}

uint8_t *bytes(q8_buf *b, uint64_t off) {
  return static_cast<uint8_t *>(b->ptr) + off;
}

int check_layout(q8_ctx *ctx, int64_t m, int G, int kind, const char *what) {
  if (!valid_layout(G, kind))
    return fail(ctx, Q8_ERR_ARG, "%s: unsupported layout G=%d scale_dtype=%d "
                "(G must be 32 or 64, scale_dtype Q8_SCALE_F16 or Q8_SCALE_F32)",
                what, G, kind);
  if (m <= 0 || m % G != 0)
    return fail(ctx, Q8_ERR_SHAPE, "%s: m=%lld must be a positive multiple of G=%d",
                what, (long long)m, G);
  return Q8_OK;
}

}  // namespace

extern "C" {

int q8_version(void) { return 100; }

uint64_t q8_rowstride_u16(int64_t m, int G, int scale_dtype) {
  if (!valid_layout(G, scale_dtype) || m <= 0 || m % G != 0) return 0;
  return (uint64_t)rowstride_u16(m, G, scale_dtype);
}

int q8_create(int device_ordinal, q8_ctx **out) {
  if (!out) return fail(nullptr, Q8_ERR_ARG, "q8_create: null output pointer");
  *out = nullptr;
  if (device_ordinal < Q8_DEVICE_NONE)
    return fail(nullptr, Q8_ERR_ARG, "q8_create: bad device ordinal %d", device_ordinal);
  q8_ctx *ctx = new (std::nothrow) q8_ctx();
  if (!ctx) return fail(nullptr, Q8_ERR_NOMEM, "q8_create: out of host memory");
  ctx->device = device_ordinal;
  ctx->host_only = device_ordinal == Q8_DEVICE_NONE;
  if (!ctx->host_only) {
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || device_ordinal >= count) {
      delete ctx;
      return fail(nullptr, Q8_ERR_HIP, "q8_create: device %d not available (%s, %d devices)",
                  device_ordinal, hipGetErrorString(e), count);
    }
    e = hipSetDevice(device_ordinal);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&ctx->own, hipStreamNonBlocking);
    if (e != hipSuccess) {
      delete ctx;
      return fail(nullptr, Q8_ERR_HIP, "q8_create: %s", hipGetErrorString(e));
    }
    ctx->stream = ctx->own;
    // Split-K workspace of the prefill GEMM, allocated up front so that
    // calls captured into HIP graphs can use it too.
    if (hipMalloc(&ctx->gemm_ws, kGemmWsFloats * sizeof(float)) != hipSuccess ||
        hipMalloc(&ctx->act16, kAct16Bytes) != hipSuccess ||
        hipDeviceSynchronize() != hipSuccess) {
      if (ctx->gemm_ws) (void)hipFree(ctx->gemm_ws);
      if (ctx->act16) (void)hipFree(ctx->act16);
      (void)hipStreamDestroy(ctx->own);
      delete ctx;
      return fail(nullptr, Q8_ERR_NOMEM, "q8_create: cannot allocate the GEMM workspace");
    }

  }
  *out = ctx;
  return Q8_OK;
}

void q8_destroy(q8_ctx *ctx) {
  if (!ctx) return;
  if (!ctx->host_only) {
    (void)hipSetDevice(ctx->device);
    if (ctx->own) {
      (void)hipStreamSynchronize(ctx->own);
      (void)hipStreamDestroy(ctx->own);
    }
    if (ctx->gemm_ws) (void)hipFree(ctx->gemm_ws);
    if (ctx->act16) (void)hipFree(ctx->act16);
    if (ctx->stage) (void)hipHostFree(ctx->stage);
    for (hipEvent_t &ev : ctx->stage_ev)
      if (ev) (void)hipEventDestroy(ev);
  }
  delete ctx;
}

int q8_set_stream(q8_ctx *ctx, void *hip_stream) {
  if (int rc = check_ctx(ctx)) return rc;
  if (ctx->host_only) return fail(ctx, Q8_ERR_NODEVICE, "q8_set_stream: host-only context");
  ctx->stream = hip_stream ? static_cast<hipStream_t>(hip_stream) : ctx->own;
  return ok(ctx);
}

void *q8_get_stream(q8_ctx *ctx) { return ctx ? static_cast<void *>(ctx->stream) : nullptr; }

int q8_sync(q8_ctx *ctx) {
  if (int rc = check_ctx(ctx)) return rc;
  if (ctx->host_only) return ok(ctx);
  if (int rc = set_device(ctx)) return rc;
  hipError_t e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "q8_sync");
  return ok(ctx);
}

const char *q8_last_error(q8_ctx *ctx) {
  return ctx ? ctx->err.c_str() : g_create_err.c_str();
}

// ---- buffers -------------------------------------------------------------------

int q8_buf_alloc(q8_ctx *ctx, uint64_t nbytes, q8_buf **out) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!out) return fail(ctx, Q8_ERR_ARG, "q8_buf_alloc: null output pointer");
  *out = nullptr;
  q8_buf *b = new (std::nothrow) q8_buf();
  if (!b) return fail(ctx, Q8_ERR_NOMEM, "q8_buf_alloc: out of host memory");
  b->size = nbytes;
  b->ctx = ctx;
  b->owned = true;
  if (!ctx->host_only && nbytes > 0) {
    if (int rc = set_device(ctx)) { delete b; return rc; }
    hipError_t e = hipMalloc(&b->ptr, nbytes);
    if (e != hipSuccess) {
      delete b;
      return fail(ctx, Q8_ERR_NOMEM, "q8_buf_alloc(%llu bytes): %s",
                  (unsigned long long)nbytes, hipGetErrorString(e));
    }
  }
  *out = b;
  return ok(ctx);
}

int q8_buf_wrap(q8_ctx *ctx, void *device_ptr, uint64_t nbytes, q8_buf **out) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!out) return fail(ctx, Q8_ERR_ARG, "q8_buf_wrap: null output pointer");
  *out = nullptr;
  if (!device_ptr && nbytes > 0 && !ctx->host_only)
    return fail(ctx, Q8_ERR_ARG, "q8_buf_wrap: null device pointer");
  q8_buf *b = new (std::nothrow) q8_buf();
  if (!b) return fail(ctx, Q8_ERR_NOMEM, "q8_buf_wrap: out of host memory");
  b->ptr = device_ptr;
  b->size = nbytes;
  b->ctx = ctx;
  b->owned = false;
  *out = b;
  return ok(ctx);
}

void q8_buf_free(q8_ctx *ctx, q8_buf *buf) {
  if (!buf) return;
  if (buf->owned && buf->ptr && ctx && !ctx->host_only) {
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    (void)hipFree(buf->ptr);
  }
  delete buf;
}

uint64_t q8_buf_size(const q8_buf *buf) { return buf ? buf->size : 0; }
void *q8_buf_device_ptr(const q8_buf *buf) { return buf ? buf->ptr : nullptr; }

int q8_buf_upload(q8_ctx *ctx, q8_buf *buf, uint64_t byte_off, const void *src, uint64_t nbytes) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!buf || (!src && nbytes)) return fail(ctx, Q8_ERR_ARG, "q8_buf_upload: null argument");
  if (!fits(byte_off, nbytes, 1, buf->size))
    return fail(ctx, Q8_ERR_RANGE, "q8_buf_upload: [%llu, +%llu) exceeds buffer of %llu bytes",
                (unsigned long long)byte_off, (unsigned long long)nbytes,
                (unsigned long long)buf->size);
  if (ctx->host_only) return fail(ctx, Q8_ERR_NODEVICE, "q8_buf_upload: host-only context");
  if (nbytes == 0) return ok(ctx);
  if (int rc = set_device(ctx)) return rc;
  hipError_t e = hipMemcpyAsync(bytes(buf, byte_off), src, nbytes, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "q8_buf_upload");
  return ok(ctx);
}

namespace {
constexpr uint64_t kStageHalf = (uint64_t)32 << 20;   // bytes per staging half
}

int q8_st_upload(q8_ctx *ctx, const q8_st *st, int64_t i, uint64_t src_off, uint64_t nbytes,
                 q8_buf *buf, uint64_t byte_off) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!st || !buf) return fail(ctx, Q8_ERR_ARG, "q8_st_upload: null argument");
  uint64_t size = 0;
  const char *name = nullptr;
  if (q8_st_info(st, i, &name, nullptr, nullptr, nullptr, nullptr, nullptr, &size) != Q8_OK)
    return fail(ctx, Q8_ERR_ARG, "q8_st_upload: %s", q8_st_error());
  if (src_off > size || nbytes > size - src_off)
    return fail(ctx, Q8_ERR_RANGE, "q8_st_upload: [%llu, +%llu) exceeds '%s' (%llu bytes)",
                (unsigned long long)src_off, (unsigned long long)nbytes, name,
                (unsigned long long)size);
  if (!fits(byte_off, nbytes, 1, buf->size))
    return fail(ctx, Q8_ERR_RANGE, "q8_st_upload: [%llu, +%llu) exceeds buffer of %llu bytes",
                (unsigned long long)byte_off, (unsigned long long)nbytes,
                (unsigned long long)buf->size);
  if (ctx->host_only) return fail(ctx, Q8_ERR_NODEVICE, "q8_st_upload: host-only context");
  if (nbytes == 0) return ok(ctx);
  if (int rc = set_device(ctx)) return rc;
  hipError_t e = hipSuccess;
  if (!ctx->stage) {
    e = hipHostMalloc(&ctx->stage, 2 * kStageHalf, hipHostMallocDefault);
    if (e != hipSuccess) {
      ctx->stage = nullptr;
      return hip_fail(ctx, e, "q8_st_upload: pinned staging");
    }
    for (hipEvent_t &ev : ctx->stage_ev)
      if (e == hipSuccess) e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e != hipSuccess) return hip_fail(ctx, e, "q8_st_upload: events");
  }
  // read chunk k into half k % 2 while the copy of chunk k - 1 runs
  uint64_t done = 0;
  for (int k = 0; done < nbytes && e == hipSuccess; ++k) {
    const int h = k & 1;
    const uint64_t n = nbytes - done < kStageHalf ? nbytes - done : kStageHalf;
    char *half = static_cast<char *>(ctx->stage) + h * kStageHalf;
    if (k >= 2) e = hipEventSynchronize(ctx->stage_ev[h]);   // half h is free again
    if (e != hipSuccess) break;
    if (q8_st_read(st, i, src_off + done, half, n) != Q8_OK) {
      (void)hipStreamSynchronize(ctx->stream);
      return fail(ctx, Q8_ERR_ARG, "q8_st_upload: %s", q8_st_error());
    }
    e = hipMemcpyAsync(bytes(buf, byte_off + done), half, n, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipEventRecord(ctx->stage_ev[h], ctx->stream);
    done += n;
  }
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "q8_st_upload");
  return ok(ctx);
}

int q8_buf_download(q8_ctx *ctx, q8_buf *buf, uint64_t byte_off, void *dst, uint64_t nbytes) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!buf || (!dst && nbytes)) return fail(ctx, Q8_ERR_ARG, "q8_buf_download: null argument");
  if (!fits(byte_off, nbytes, 1, buf->size))
    return fail(ctx, Q8_ERR_RANGE, "q8_buf_download: [%llu, +%llu) exceeds buffer of %llu bytes",
                (unsigned long long)byte_off, (unsigned long long)nbytes,
                (unsigned long long)buf->size);
  if (ctx->host_only) return fail(ctx, Q8_ERR_NODEVICE, "q8_buf_download: host-only context");
  if (nbytes == 0) return ok(ctx);
  if (int rc = set_device(ctx)) return rc;
  hipError_t e = hipMemcpyAsync(dst, bytes(buf, byte_off), nbytes, hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "q8_buf_download");
  return ok(ctx);
}

// ---- Q8 path ------------------------------------------------------------------------

int q8_quantize_pack(q8_ctx *ctx, q8_buf *src, uint64_t src_off, int src_dtype, int64_t n,
                     int64_t m, q8_buf *dst, uint64_t dst_off_u16, int G, int scale_dtype) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!src || !dst) return fail(ctx, Q8_ERR_ARG, "q8_quantize_pack: null buffer");
  if (src_dtype != Q8_SRC_BF16 && src_dtype != Q8_SRC_F32)
    return fail(ctx, Q8_ERR_ARG, "q8_quantize_pack: bad src_dtype %d", src_dtype);
  if (int rc = check_layout(ctx, m, G, scale_dtype, "q8_quantize_pack")) return rc;
  if (n < 0) return fail(ctx, Q8_ERR_SHAPE, "q8_quantize_pack: n=%lld < 0", (long long)n);
  const uint64_t es = src_dtype == Q8_SRC_F32 ? 4 : 2;
  const uint64_t rs = (uint64_t)rowstride_u16(m, G, scale_dtype);
  const uint64_t ne = (uint64_t)n * (uint64_t)m;
  if (!fits(src_off, ne, es, src->size))
    return fail(ctx, Q8_ERR_RANGE, "q8_quantize_pack: source [%llu, +%llu) elements exceeds buffer",
                (unsigned long long)src_off, (unsigned long long)ne);
  if (!fits(dst_off_u16, (uint64_t)n * rs, 2, dst->size))
    return fail(ctx, Q8_ERR_RANGE, "q8_quantize_pack: packed output [%llu, +%llu) u16 exceeds buffer",
                (unsigned long long)dst_off_u16, (unsigned long long)((uint64_t)n * rs));
  if (src == dst && overlaps(src_off * es, (src_off + ne) * es, dst_off_u16 * 2,
                             (dst_off_u16 + (uint64_t)n * rs) * 2))
    return fail(ctx, Q8_ERR_ARG, "q8_quantize_pack: source and destination overlap");
  if (ctx->host_only) return fail(ctx, Q8_ERR_NODEVICE, "q8_quantize_pack: host-only context");
  if (n == 0) return ok(ctx);
  if (int rc = set_device(ctx)) return rc;
  q8::PackArgs a;
  a.src = bytes(src, src_off * es);
  a.src_is_f32 = src_dtype == Q8_SRC_F32;
  a.n = n;
  a.m = m;
  a.dst = bytes(dst, dst_off_u16 * 2);
  a.dst_row_bytes = (int64_t)rs * 2;
  a.G = G;
  a.kind = scale_dtype;
  hipError_t e = q8::launch_pack(a, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "q8_quantize_pack launch");
  return ok(ctx);
}

namespace {

// Shapes and ranges shared by q8_linear and q8_linear_bf16act.
int check_linear(q8_ctx *ctx, const char *what, q8_buf *w, uint64_t owt, int64_t s, int64_t m,
                 int64_t n, int G, int kind) {
  if (!w) return fail(ctx, Q8_ERR_ARG, "%s: null weight buffer", what);
  if (int rc = check_layout(ctx, m, G, kind, what)) return rc;
  if (s < 0 || n < 0)
    return fail(ctx, Q8_ERR_SHAPE, "%s: s=%lld and n=%lld must be >= 0", what, (long long)s,
                (long long)n);
  const uint64_t rs = (uint64_t)rowstride_u16(m, G, kind);
  if (!fits(owt, (uint64_t)n * rs, 2, w->size))
    return fail(ctx, Q8_ERR_RANGE, "%s: weights [%llu, +%llu) u16 exceed the weight buffer (%llu bytes)",
                what, (unsigned long long)owt, (unsigned long long)((uint64_t)n * rs),
                (unsigned long long)w->size);
  return Q8_OK;
}

bool gemm_aligned(const q8::LinearArgs &a) {
  const int sb = a.kind == Q8_SCALE_F32 ? 4 : 2;
  const uintptr_t xw = reinterpret_cast<uintptr_t>(a.x);
  return reinterpret_cast<uintptr_t>(a.w) % 16 == 0 && a.row_bytes % 16 == 0 &&
         ((a.m / a.G) * sb) % 16 == 0 && xw % 16 == 0 && a.m % 8 == 0;
}

// Activation rows at which the W8A32 path switches from the VALU GEMV to the
// small-batch MFMA kernels (f32 4x4 blocks up to q8::kSkinny4MaxRows rows,
// then f32 x split into two bf16 terms), and from those to the dequant-GEMM
// on f16 MFMA.
constexpr int64_t kSkinnyMinRows = 2;
constexpr int64_t kGemmMinRows = 32;

// Attach the context's split-K workspace to a launch.
void attach_gemm_workspace(q8_ctx *ctx, q8::LinearArgs &la) {
  la.ws = ctx->gemm_ws;
  la.ws_floats = kGemmWsFloats;
}

// Layout of a GEMM activation buffer of `bytes`: the weight-row exponents
// (n ints) at the end, 256-byte aligned, and before them as many binary16
// activation rows (2 m bytes each) plus one int exponent per row as fit.
// Zero rows: the shape does not fit (the C ABI rejects it first).
int64_t gemm_act_rows(int64_t bytes, int64_t m, int64_t n) {
  const int64_t tail = (4 * n + 255) / 256 * 256;
  return bytes > tail ? (bytes - tail) / (2 * m + 4) : 0;
}

bool gemm_fits(int64_t bytes, int64_t m, int64_t n) {
  return m < ((int64_t)1 << 40) && n < ((int64_t)1 << 40) && gemm_act_rows(bytes, m, n) > 0;
}

// Prefill GEMM on f16 MFMA through a binary16 activation buffer of `bytes`
// at act16, in chunks of as many rows as it holds (stream order keeps the
// chunks from overlapping).
hipError_t run_gemm_in(q8::LinearArgs la, void *act16, int64_t bytes, hipStream_t st) {
  const int64_t rows = gemm_act_rows(bytes, la.m, la.n);
  uint8_t *base = static_cast<uint8_t *>(act16);
  uint16_t *x16 = reinterpret_cast<uint16_t *>(base);
  int *ex = reinterpret_cast<int *>(base + rows * la.m * 2);
  int *ew = reinterpret_cast<int *>(base + bytes - (4 * la.n + 255) / 256 * 256);
  const int64_t xb = la.x_is_bf16 ? 2 : 4;
  const int64_t ldx = la.ldx ? la.ldx : la.m;
  const uint8_t *x0 = static_cast<const uint8_t *>(la.x);
  const float *u0 = la.up, *res0 = la.res;
  float *y0 = la.y, *h0 = la.hout;
  const int64_t s = la.s;
  for (int64_t r0 = 0; r0 < s; r0 += rows) {
    la.s = s - r0 < rows ? s - r0 : rows;
    la.x = x0 + r0 * ldx * xb;
    if (u0) la.up = u0 + r0 * ldx;
    if (res0) la.res = res0 + r0 * la.m;
    if (h0) la.hout = h0 + r0 * la.m;
    la.y = y0 + r0 * la.n;
    hipError_t e = q8::launch_gemm(la, x16, ex, ew, r0 == 0, st);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t run_gemm(q8_ctx *ctx, q8::LinearArgs la) {
  attach_gemm_workspace(ctx, la);
  return run_gemm_in(la, ctx->act16, kAct16Bytes, ctx->stream);
}

// Device memory a W8A32 linear may use besides its inputs and outputs: the
// split-K partial sums and the GEMM's binary16 activation buffer.
struct Scratch {
  float *ws;
  int64_t ws_floats;
  void *act16;
  int64_t act_bytes;
};

// The W8A32 linear of q8_linear on resolved pointers: GEMM from
// kGemmMinRows rows, the few-row and small-batch MFMA kernels from
// kSkinnyMinRows, the GEMV otherwise (and for unaligned operands).
hipError_t dispatch_linear(q8::LinearArgs la, const Scratch &sc, hipStream_t st) {
  la.ws = sc.ws;
  la.ws_floats = sc.ws_floats;
  if (la.s >= kGemmMinRows && gemm_aligned(la)) return run_gemm_in(la, sc.act16, sc.act_bytes, st);
  if (la.s >= kSkinnyMinRows && la.s <= q8::kSkinny4MaxRows && gemm_aligned(la))
    return q8::launch_skinny4(la, st);
  if (la.s >= kSkinnyMinRows && gemm_aligned(la)) return q8::launch_skinny(la, st);
  return q8::launch_gemv(la, st);
}

Scratch ctx_scratch(q8_ctx *ctx) {
  return Scratch{ctx->gemm_ws, kGemmWsFloats, ctx->act16, kAct16Bytes};
}

}  // namespace

int q8_linear(q8_ctx *ctx, q8_buf *w, uint64_t owt_u16, q8_buf *a, uint64_t ox_f32,
              uint64_t oy_f32, int64_t s, int64_t m, int64_t n, int G, int scale_dtype) {
  if (int rc = check_ctx(ctx)) return rc;
  if (int rc = check_linear(ctx, "q8_linear", w, owt_u16, s, m, n, G, scale_dtype)) return rc;
  if (!a) return fail(ctx, Q8_ERR_ARG, "q8_linear: null activation buffer");
  const uint64_t nx = (uint64_t)s * (uint64_t)m, ny = (uint64_t)s * (uint64_t)n;
  if (!fits(ox_f32, nx, 4, a->size))
    return fail(ctx, Q8_ERR_RANGE, "q8_linear: x [%llu, +%llu) f32 exceeds the activation buffer",
                (unsigned long long)ox_f32, (unsigned long long)nx);
  if (!fits(oy_f32, ny, 4, a->size))
    return fail(ctx, Q8_ERR_RANGE, "q8_linear: y [%llu, +%llu) f32 exceeds the activation buffer",
                (unsigned long long)oy_f32, (unsigned long long)ny);
  if (nx && ny && overlaps(ox_f32, ox_f32 + nx, oy_f32, oy_f32 + ny))
    return fail(ctx, Q8_ERR_ARG, "q8_linear: x and y overlap");
  if (s >= kGemmMinRows && !gemm_fits(kAct16Bytes, m, n))
    return fail(ctx, Q8_ERR_SHAPE, "q8_linear: m=%lld, n=%lld too large for the GEMM's "
                "activation buffer (%lld bytes)", (long long)m, (long long)n,
                (long long)kAct16Bytes);
  if (ctx->host_only) return fail(ctx, Q8_ERR_NODEVICE, "q8_linear: host-only context");
  if (s == 0 || n == 0) return ok(ctx);
  if (int rc = set_device(ctx)) return rc;
  q8::LinearArgs la;
  la.w = bytes(w, owt_u16 * 2);
  la.row_bytes = rowstride_u16(m, G, scale_dtype) * 2;
  la.x = bytes(a, ox_f32 * 4);
  la.x_is_bf16 = 0;
  la.y = reinterpret_cast<float *>(bytes(a, oy_f32 * 4));
  la.s = s;
  la.m = m;
  la.n = n;
  la.G = G;
  la.kind = scale_dtype;
  hipError_t e = dispatch_linear(la, ctx_scratch(ctx), ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "q8_linear launch");
  return ok(ctx);
}

int q8_linear_bf16act(q8_ctx *ctx, q8_buf *w, uint64_t owt_u16, q8_buf *x, uint64_t ox_bf16,
                      q8_buf *y, uint64_t oy_f32, int64_t s, int64_t m, int64_t n, int G,
                      int scale_dtype) {
  if (int rc = check_ctx(ctx)) return rc;
  if (int rc = check_linear(ctx, "q8_linear_bf16act", w, owt_u16, s, m, n, G, scale_dtype))
    return rc;
  if (!x || !y) return fail(ctx, Q8_ERR_ARG, "q8_linear_bf16act: null activation buffer");
  const uint64_t nx = (uint64_t)s * (uint64_t)m, ny = (uint64_t)s * (uint64_t)n;
  if (!fits(ox_bf16, nx, 2, x->size))
    return fail(ctx, Q8_ERR_RANGE, "q8_linear_bf16act: x [%llu, +%llu) bf16 exceeds its buffer",
                (unsigned long long)ox_bf16, (unsigned long long)nx);
  if (!fits(oy_f32, ny, 4, y->size))
    return fail(ctx, Q8_ERR_RANGE, "q8_linear_bf16act: y [%llu, +%llu) f32 exceeds its buffer",
                (unsigned long long)oy_f32, (unsigned long long)ny);
  if (x == y && nx && ny && overlaps(ox_bf16 * 2, (ox_bf16 + nx) * 2, oy_f32 * 4, (oy_f32 + ny) * 4))
    return fail(ctx, Q8_ERR_ARG, "q8_linear_bf16act: x and y overlap");
  if (!gemm_fits(kAct16Bytes, m, n))
    return fail(ctx, Q8_ERR_SHAPE, "q8_linear_bf16act: m=%lld, n=%lld too large for the "
                "GEMM's activation buffer (%lld bytes)", (long long)m, (long long)n,
                (long long)kAct16Bytes);
  if (ctx->host_only) return fail(ctx, Q8_ERR_NODEVICE, "q8_linear_bf16act: host-only context");
  if (s == 0 || n == 0) return ok(ctx);
  if (int rc = set_device(ctx)) return rc;
  q8::LinearArgs la;
  la.w = bytes(w, owt_u16 * 2);
  la.row_bytes = rowstride_u16(m, G, scale_dtype) * 2;
  la.x = bytes(x, ox_bf16 * 2);
  la.x_is_bf16 = 1;
  la.y = reinterpret_cast<float *>(bytes(y, oy_f32 * 4));
  la.s = s;
  la.m = m;
  la.n = n;
  la.G = G;
  la.kind = scale_dtype;
  hipError_t e;
  if (gemm_aligned(la)) {
    e = run_gemm(ctx, la);
  } else {
    e = q8::launch_gemv(la, ctx->stream);
  }
  if (e != hipSuccess) return hip_fail(ctx, e, "q8_linear_bf16act launch");
  return ok(ctx);
}

// ---- allocation-free linear -----------------------------------------------------
//
// q8_linear_noalloc keeps its scratch in one fixed device array per GPU
// instead of a context's workspace: 16 MiB of split-K partial sums (the size
// of a context's, so it makes the same split decisions as q8_linear), then
// the GEMM's 16 MiB binary16 activation buffer.  The array's name is a host-side stand-in: host code
// only ever passes the address hipGetSymbolAddress returns for the current
// device (noalloc_scratch).

namespace {
constexpr int64_t kNoAllocWsFloats = kGemmWsFloats;
constexpr int64_t kNoAllocAct16Bytes = (int64_t)16 << 20;
constexpr int64_t kNoAllocBytes =
    kNoAllocWsFloats * 4 + kNoAllocAct16Bytes;
static_assert(kNoAllocBytes == Q8_NOALLOC_SCRATCH_BYTES, "scratch size differs from the header");
}  // namespace

static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

namespace {

constexpr int kNoAllocMaxDevices = 64;
std::mutex g_noalloc_mu;
void *g_noalloc_ptr[kNoAllocMaxDevices];   // scratch's device address per device

// Set-up, once per device (the first call on it), with that device current:
// resolve this device's copy of `scratch`.  No part of it needs clearing:
// every kernel writes the partials and activation rows it reads back.
int noalloc_scratch(int dev, Scratch *out) {
  std::lock_guard<std::mutex> lock(g_noalloc_mu);
  void *base = g_noalloc_ptr[dev];
  if (!base) {
    // The first call may come while this thread captures a stream into a
    // graph: the symbol lookup (which can load the code object) is not a
    // stream operation, so it runs with this thread's capture mode relaxed
    // for its duration, then the caller's mode is restored.
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    hipError_t e = hipThreadExchangeStreamCaptureMode(&mode);
    if (e != hipSuccess)
      return hip_fail(nullptr, e, "q8_linear_noalloc: hipThreadExchangeStreamCaptureMode");
    e = hipGetSymbolAddress(&base, HIP_SYMBOL(scratch));
    hipError_t e2 = hipThreadExchangeStreamCaptureMode(&mode);
    if (e == hipSuccess && e2 != hipSuccess) e = e2;
    if (e != hipSuccess || !base)
      return hip_fail(nullptr, e != hipSuccess ? e : hipErrorInvalidSymbol,
                      "q8_linear_noalloc: hipGetSymbolAddress(scratch)");
    g_noalloc_ptr[dev] = base;
  }
  uint8_t *b = static_cast<uint8_t *>(base);
  out->ws = reinterpret_cast<float *>(b);
  out->ws_floats = kNoAllocWsFloats;
  out->act16 = b + kNoAllocWsFloats * 4;
  out->act_bytes = kNoAllocAct16Bytes;
  return Q8_OK;
}

}  // namespace

int q8_linear_noalloc(void *hip_stream, const void *w, const float *x, float *y, int64_t s,
                      int64_t m, int64_t n, int G, int scale_dtype) {
  const char *what = "q8_linear_noalloc";
  if (int rc = check_layout(nullptr, m, G, scale_dtype, what)) return rc;
  if (s < 0 || n < 0)
    return fail(nullptr, Q8_ERR_SHAPE, "%s: s=%lld and n=%lld must be >= 0", what, (long long)s,
                (long long)n);
  if (s == 0 || n == 0) return Q8_OK;
  if (!w || !x || !y) return fail(nullptr, Q8_ERR_ARG, "%s: null weight, x or y pointer", what);
  // the alignment q8_linear's element offsets give: u16 weights, f32 x and y
  if ((reinterpret_cast<uintptr_t>(w) & 1) || (reinterpret_cast<uintptr_t>(x) & 3) ||
      (reinterpret_cast<uintptr_t>(y) & 3))
    return fail(nullptr, Q8_ERR_ARG, "%s: w must be 2-byte aligned, x and y 4-byte aligned",
                what);
  const unsigned __int128 xb = (unsigned __int128)s * (uint64_t)m * 4,
                          yb = (unsigned __int128)s * (uint64_t)n * 4;
  if (xb >= ((unsigned __int128)1 << 62) || yb >= ((unsigned __int128)1 << 62))
    return fail(nullptr, Q8_ERR_SHAPE, "%s: s=%lld, m=%lld, n=%lld out of range", what,
                (long long)s, (long long)m, (long long)n);
  const uintptr_t x0 = reinterpret_cast<uintptr_t>(x), y0 = reinterpret_cast<uintptr_t>(y);
  if (overlaps(x0, x0 + (uint64_t)xb, y0, y0 + (uint64_t)yb))
    return fail(nullptr, Q8_ERR_ARG, "%s: x and y overlap", what);
  if (s >= kGemmMinRows && !gemm_fits(kNoAllocAct16Bytes, m, n))
    return fail(nullptr, Q8_ERR_SHAPE, "%s: m=%lld, n=%lld exceed the %lld-byte activation "
                "buffer of the allocation-free scratch (one row of 2 m + 4 bytes plus 4 n "
                "bytes must fit)", what, (long long)m, (long long)n,
                (long long)kNoAllocAct16Bytes);
  hipStream_t st = static_cast<hipStream_t>(hip_stream);
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(nullptr, e, "q8_linear_noalloc: hipGetDevice");
  if (dev < 0 || dev >= kNoAllocMaxDevices)
    return fail(nullptr, Q8_ERR_ARG, "%s: device %d out of range", what, dev);
  if (st) {
    int sdev = -1;
    e = hipStreamGetDevice(st, &sdev);
    if (e != hipSuccess) return hip_fail(nullptr, e, "q8_linear_noalloc: hipStreamGetDevice");
    if (sdev != dev)
      return fail(nullptr, Q8_ERR_ARG, "%s: the stream belongs to device %d, the current "
                  "device is %d", what, sdev, dev);
  }
  Scratch sc;
  if (int rc = noalloc_scratch(dev, &sc)) return rc;
  q8::LinearArgs la;
  la.w = static_cast<const uint8_t *>(w);
  la.row_bytes = rowstride_u16(m, G, scale_dtype) * 2;
  la.x = x;
  la.x_is_bf16 = 0;
  la.y = y;
  la.s = s;
  la.m = m;
  la.n = n;
  la.G = G;
  la.kind = scale_dtype;
  e = dispatch_linear(la, sc, st);
  if (e != hipSuccess) return hip_fail(nullptr, e, "q8_linear_noalloc launch");
  return Q8_OK;
}

int q8_embed_gather(q8_ctx *ctx, q8_buf *w, uint64_t oemb_u16, q8_buf *ids, uint64_t oids_i32,
                    q8_buf *a, uint64_t oy_f32, int64_t s, int64_t d, int64_t vocab, int G,
                    int scale_dtype) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!w || !ids || !a) return fail(ctx, Q8_ERR_ARG, "q8_embed_gather: null buffer");
  if (int rc = check_layout(ctx, d, G, scale_dtype, "q8_embed_gather")) return rc;
  if (s < 0 || vocab < 0)
    return fail(ctx, Q8_ERR_SHAPE, "q8_embed_gather: s=%lld and vocab=%lld must be >= 0",
                (long long)s, (long long)vocab);
  const uint64_t rs = (uint64_t)rowstride_u16(d, G, scale_dtype);
  if (!fits(oemb_u16, (uint64_t)vocab * rs, 2, w->size))
    return fail(ctx, Q8_ERR_RANGE, "q8_embed_gather: table of %lld rows exceeds the weight buffer",
                (long long)vocab);
  if (!fits(oids_i32, (uint64_t)s, 4, ids->size))
    return fail(ctx, Q8_ERR_RANGE, "q8_embed_gather: ids [%llu, +%lld) exceed their buffer",
                (unsigned long long)oids_i32, (long long)s);
  if (!fits(oy_f32, (uint64_t)s * (uint64_t)d, 4, a->size))
    return fail(ctx, Q8_ERR_RANGE, "q8_embed_gather: output exceeds the activation buffer");
  if (ctx->host_only) return fail(ctx, Q8_ERR_NODEVICE, "q8_embed_gather: host-only context");
  if (s == 0) return ok(ctx);
  if (int rc = set_device(ctx)) return rc;
  q8::GatherArgs ga;
  ga.w = bytes(w, oemb_u16 * 2);
  ga.row_bytes = (int64_t)rs * 2;
  ga.ids = reinterpret_cast<const int32_t *>(bytes(ids, oids_i32 * 4));
  ga.y = reinterpret_cast<float *>(bytes(a, oy_f32 * 4));
  ga.s = s;
  ga.d = d;
  ga.vocab = vocab;
  ga.G = G;
  ga.kind = scale_dtype;
  hipError_t e = q8::launch_embed_gather(ga, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "q8_embed_gather launch");
  return ok(ctx);
}

// ---- decode-step layer kernels -------------------------------------------------

namespace {

float *fptr(q8_buf *b, uint64_t off_f32) { return reinterpret_cast<float *>(bytes(b, off_f32 * 4)); }

// An output range may coincide with an input range or be disjoint from it.
bool bad_alias(uint64_t o0, uint64_t n, uint64_t i0, uint64_t m) {
  return o0 != i0 && overlaps(o0, o0 + n, i0, i0 + m);
}

int check_f32(q8_ctx *ctx, q8_buf *a, uint64_t off, uint64_t count, const char *what,
              const char *name) {
  if (!fits(off, count, 4, a->size))
    return fail(ctx, Q8_ERR_RANGE, "%s: %s [%llu, +%llu) f32 exceeds the activation buffer", what,
                name, (unsigned long long)off, (unsigned long long)count);
  return Q8_OK;
}

// Position source shared by q8_rope_kv and q8_attention.
int check_pos(q8_ctx *ctx, q8_buf *posbuf, uint64_t opos, int64_t pos0, int64_t s, int64_t maxlen,
              const char *what) {
  if (posbuf) {
    if (!fits(opos, 1, 4, posbuf->size))
      return fail(ctx, Q8_ERR_RANGE, "%s: position offset %llu exceeds its buffer", what,
                  (unsigned long long)opos);
    return Q8_OK;
  }
  if (pos0 < 0 || pos0 + s > maxlen)
    return fail(ctx, Q8_ERR_RANGE, "%s: rows %lld .. %lld exceed the KV cache of %lld rows "
                "(KV cache full)", what, (long long)pos0, (long long)(pos0 + s),
                (long long)maxlen);
  return Q8_OK;
}

int check_heads(q8_ctx *ctx, int nheads, int nkv, int head_dim, const char *what) {
  if (nheads <= 0 || nkv <= 0 || nheads % nkv != 0 || head_dim <= 0 || head_dim % 2 != 0)
    return fail(ctx, Q8_ERR_SHAPE, "%s: nheads=%d, nkv=%d, head_dim=%d (need nkv | nheads and "
                "an even head_dim)", what, nheads, nkv, head_dim);
  return Q8_OK;
}

int64_t attn_nsplit(int64_t maxlen) { return (maxlen + 63) / 64; }

// The attention kernels address a layer's K or V block through 32-bit
// buffer offsets: maxlen * nkv * head_dim binary16 values must stay under
// 2 GiB.
bool cache_block_ok(int64_t maxlen, int nkv, int head_dim) {
  return (uint64_t)maxlen * (uint64_t)nkv * (uint64_t)head_dim * 2 < ((uint64_t)1 << 31);
}

}  // namespace

int q8_linear_fused(q8_ctx *ctx, q8_buf *w, uint64_t owt_u16, q8_buf *a, uint64_t ox_f32,
                    uint64_t oy_f32, int64_t m, int64_t n, int G, int scale_dtype, int pre,
                    uint64_t onorm_u16, float eps, int post, uint64_t ores_f32) {
  if (int rc = check_ctx(ctx)) return rc;
  if (int rc = check_linear(ctx, "q8_linear_fused", w, owt_u16, 1, m, n, G, scale_dtype))
    return rc;
  if (!a) return fail(ctx, Q8_ERR_ARG, "q8_linear_fused: null activation buffer");
  if (pre != Q8_PRE_NONE && pre != Q8_PRE_RMSNORM && pre != Q8_PRE_SWIGLU)
    return fail(ctx, Q8_ERR_ARG, "q8_linear_fused: pre=%d", pre);
  if (post != Q8_POST_STORE && post != Q8_POST_RESIDUAL && post != Q8_POST_SWIGLU)
    return fail(ctx, Q8_ERR_ARG, "q8_linear_fused: post=%d", post);
  if (post == Q8_POST_SWIGLU && n % 2 != 0)
    return fail(ctx, Q8_ERR_SHAPE, "q8_linear_fused: n=%lld must be even (gate and up rows)",
                (long long)n);
  const uint64_t nx = (uint64_t)(pre == Q8_PRE_SWIGLU ? 2 : 1) * (uint64_t)m;
  const uint64_t ny = post == Q8_POST_SWIGLU ? (uint64_t)n / 2 : (uint64_t)n;
  if (int rc = check_f32(ctx, a, ox_f32, nx, "q8_linear_fused", "x")) return rc;
  if (int rc = check_f32(ctx, a, oy_f32, ny, "q8_linear_fused", "y")) return rc;
  if (nx && ny && overlaps(ox_f32, ox_f32 + nx, oy_f32, oy_f32 + ny))
    return fail(ctx, Q8_ERR_ARG, "q8_linear_fused: x and y overlap");
  if (post == Q8_POST_RESIDUAL) {
    if (int rc = check_f32(ctx, a, ores_f32, ny, "q8_linear_fused", "residual")) return rc;
    if (bad_alias(oy_f32, ny, ores_f32, ny))
      return fail(ctx, Q8_ERR_ARG, "q8_linear_fused: y partially overlaps the residual");
  }
  if (pre == Q8_PRE_RMSNORM && !fits(onorm_u16, (uint64_t)m, 2, w->size))
    return fail(ctx, Q8_ERR_RANGE, "q8_linear_fused: norm weights exceed the weight buffer");
  q8::FusedLinearArgs f;
  q8::LinearArgs &la = f.lin;
  la.w = bytes(w, owt_u16 * 2);
  la.row_bytes = rowstride_u16(m, G, scale_dtype) * 2;
  la.x = bytes(a, ox_f32 * 4);
  la.x_is_bf16 = 0;
  la.y = fptr(a, oy_f32);
  la.s = 1;
  la.m = m;
  la.n = n;
  la.G = G;
  la.kind = scale_dtype;
  f.pre = pre;
  f.post = post;
  f.wn = pre == Q8_PRE_RMSNORM ? reinterpret_cast<const uint16_t *>(bytes(w, onorm_u16 * 2))
                               : nullptr;
  f.eps = eps;
  f.res = post == Q8_POST_RESIDUAL ? fptr(a, ores_f32) : nullptr;
  if (!q8::gemv_fused_supported(f))
    return fail(ctx, Q8_ERR_UNSUPPORTED, "q8_linear_fused: m=%lld (needs m %% 32 == 0, 16-byte "
                "aligned rows and x, 8-byte aligned norm weights and, with a prologue, "
                "m <= 16384)", (long long)m);
  if (ctx->host_only) return fail(ctx, Q8_ERR_NODEVICE, "q8_linear_fused: host-only context");
  if (n == 0) return ok(ctx);
  if (int rc = set_device(ctx)) return rc;
  hipError_t e = q8::launch_gemv_fused(f, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "q8_linear_fused launch");
  return ok(ctx);
}

// Floats spanned by s rows of `width` floats at a row stride of ld.
static uint64_t rows_span(int64_t s, int64_t ld, uint64_t width) {
  return s == 0 ? 0 : (uint64_t)(s - 1) * (uint64_t)ld + width;
}

// Rows of wa floats at a and rows of wb floats at b, both at row stride ld
// (wa, wb <= ld): true when no element of one is an element of the other
// for any pair of rows, i.e. b's columns taken modulo ld from a's row start
// lie in [wa, ld) without wrapping.
static bool stride_disjoint(uint64_t a, int64_t wa, uint64_t b, int64_t wb, int64_t ld) {
  const int64_t d = (int64_t)(b - a);             // both lie inside one arena
  const int64_t r = (d % ld + ld) % ld;
  return r >= wa && r + wb <= ld;
}

int q8_linear_swiglu(q8_ctx *ctx, q8_buf *w, uint64_t owt_u16, q8_buf *a, uint64_t og_f32,
                     uint64_t ou_f32, uint64_t oy_f32, int64_t s, int64_t m, int64_t n, int G,
                     int scale_dtype, int64_t ld) {
  if (int rc = check_ctx(ctx)) return rc;
  if (int rc = check_linear(ctx, "q8_linear_swiglu", w, owt_u16, s, m, n, G, scale_dtype))
    return rc;
  if (!a) return fail(ctx, Q8_ERR_ARG, "q8_linear_swiglu: null activation buffer");
  if (ld != 0 && (ld < m || ld > INT32_MAX))
    return fail(ctx, Q8_ERR_SHAPE, "q8_linear_swiglu: row stride %lld (0, or at least m=%lld)",
                (long long)ld, (long long)m);
  if (ld == 0) ld = m;
  const uint64_t nx = rows_span(s, ld, (uint64_t)m), ny = (uint64_t)s * (uint64_t)n;
  if (int rc = check_f32(ctx, a, og_f32, nx, "q8_linear_swiglu", "gate")) return rc;
  if (int rc = check_f32(ctx, a, ou_f32, nx, "q8_linear_swiglu", "up")) return rc;
  if (int rc = check_f32(ctx, a, oy_f32, ny, "q8_linear_swiglu", "y")) return rc;
  if (nx && ny && (overlaps(og_f32, og_f32 + nx, oy_f32, oy_f32 + ny) ||
                   overlaps(ou_f32, ou_f32 + nx, oy_f32, oy_f32 + ny)))
    return fail(ctx, Q8_ERR_ARG, "q8_linear_swiglu: gate or up overlaps y");
  if (s < kGemmMinRows)
    return fail(ctx, Q8_ERR_UNSUPPORTED, "q8_linear_swiglu: s=%lld (from %lld rows; fewer: "
                "q8_swiglu, then q8_linear)", (long long)s, (long long)kGemmMinRows);
  if (!gemm_fits(kAct16Bytes, m, n))
    return fail(ctx, Q8_ERR_SHAPE, "q8_linear_swiglu: m=%lld, n=%lld too large for the GEMM's "
                "activation buffer (%lld bytes)", (long long)m, (long long)n,
                (long long)kAct16Bytes);
  q8::LinearArgs la;
  la.w = bytes(w, owt_u16 * 2);
  la.row_bytes = rowstride_u16(m, G, scale_dtype) * 2;
  la.x = bytes(a, og_f32 * 4);
  la.x_is_bf16 = 0;
  la.up = reinterpret_cast<const float *>(bytes(a, ou_f32 * 4));
  la.y = reinterpret_cast<float *>(bytes(a, oy_f32 * 4));
  la.s = s;
  la.m = m;
  la.n = n;
  la.G = G;
  la.kind = scale_dtype;
  la.ldx = ld;
  if (!gemm_aligned(la) || reinterpret_cast<uintptr_t>(la.up) % 16 != 0 || ld % 4 != 0)
    return fail(ctx, Q8_ERR_UNSUPPORTED, "q8_linear_swiglu: gate, up and the weight rows must "
                "be 16-byte aligned, m a multiple of 8, the row stride a multiple of 4");
  if (ctx->host_only) return fail(ctx, Q8_ERR_NODEVICE, "q8_linear_swiglu: host-only context");
  if (n == 0) return ok(ctx);
  if (int rc = set_device(ctx)) return rc;
  hipError_t e = run_gemm(ctx, la);
  if (e != hipSuccess) return hip_fail(ctx, e, "q8_linear_swiglu launch");
  return ok(ctx);
}

int q8_linear_rmsnorm(q8_ctx *ctx, q8_buf *w, uint64_t owt_u16, uint64_t onorm_u16, float eps,
                      q8_buf *a, uint64_t ox_f32, int has_res, uint64_t ores_f32,
                      uint64_t oh_f32, uint64_t oy_f32, int64_t s, int64_t m, int64_t n, int G,
                      int scale_dtype) {
  if (int rc = check_ctx(ctx)) return rc;
  if (int rc = check_linear(ctx, "q8_linear_rmsnorm", w, owt_u16, s, m, n, G, scale_dtype))
    return rc;
  if (!a) return fail(ctx, Q8_ERR_ARG, "q8_linear_rmsnorm: null activation buffer");
  if (!fits(onorm_u16, (uint64_t)m, 2, w->size))
    return fail(ctx, Q8_ERR_RANGE, "q8_linear_rmsnorm: norm weights exceed the weight buffer");
  const uint64_t nx = (uint64_t)s * (uint64_t)m, ny = (uint64_t)s * (uint64_t)n;
  if (int rc = check_f32(ctx, a, ox_f32, nx, "q8_linear_rmsnorm", "x")) return rc;
  if (int rc = check_f32(ctx, a, oy_f32, ny, "q8_linear_rmsnorm", "y")) return rc;
  if (has_res) {
    if (int rc = check_f32(ctx, a, ores_f32, nx, "q8_linear_rmsnorm", "res")) return rc;
    if (int rc = check_f32(ctx, a, oh_f32, nx, "q8_linear_rmsnorm", "h")) return rc;
    // h may be x or res itself (each element is read before the same thread
    // writes it), but not a shifted copy of either
    if (bad_alias(oh_f32, nx, ox_f32, nx) || bad_alias(oh_f32, nx, ores_f32, nx))
      return fail(ctx, Q8_ERR_ARG, "q8_linear_rmsnorm: h partially overlaps x or res");
  }
  // y is written while later row chunks of x (res, h) are still to be read
  if (nx && ny &&
      (overlaps(ox_f32, ox_f32 + nx, oy_f32, oy_f32 + ny) ||
       (has_res && (overlaps(ores_f32, ores_f32 + nx, oy_f32, oy_f32 + ny) ||
                    overlaps(oh_f32, oh_f32 + nx, oy_f32, oy_f32 + ny)))))
    return fail(ctx, Q8_ERR_ARG, "q8_linear_rmsnorm: y overlaps x, res or h");
  if (s < kGemmMinRows)
    return fail(ctx, Q8_ERR_UNSUPPORTED, "q8_linear_rmsnorm: s=%lld (from %lld rows; fewer: "
                "q8_rmsnorm or q8_add_rmsnorm, then q8_linear)", (long long)s,
                (long long)kGemmMinRows);
  if (m > 16384)
    return fail(ctx, Q8_ERR_UNSUPPORTED, "q8_linear_rmsnorm: m=%lld (at most 16384; longer "
                "rows: q8_rmsnorm, then q8_linear)", (long long)m);
  if (!gemm_fits(kAct16Bytes, m, n))
    return fail(ctx, Q8_ERR_SHAPE, "q8_linear_rmsnorm: m=%lld, n=%lld too large for the GEMM's "
                "activation buffer (%lld bytes)", (long long)m, (long long)n,
                (long long)kAct16Bytes);
  q8::LinearArgs la;
  la.w = bytes(w, owt_u16 * 2);
  la.row_bytes = rowstride_u16(m, G, scale_dtype) * 2;
  la.x = bytes(a, ox_f32 * 4);
  la.x_is_bf16 = 0;
  la.y = reinterpret_cast<float *>(bytes(a, oy_f32 * 4));
  la.s = s;
  la.m = m;
  la.n = n;
  la.G = G;
  la.kind = scale_dtype;
  la.wn = reinterpret_cast<const uint16_t *>(bytes(w, onorm_u16 * 2));
  la.eps = eps;
  if (has_res) {
    la.res = reinterpret_cast<const float *>(bytes(a, ores_f32 * 4));
    la.hout = reinterpret_cast<float *>(bytes(a, oh_f32 * 4));
  }
  if (!gemm_aligned(la))
    return fail(ctx, Q8_ERR_UNSUPPORTED, "q8_linear_rmsnorm: x and the weight rows must be "
                "16-byte aligned, m a multiple of 8");
  if (ctx->host_only) return fail(ctx, Q8_ERR_NODEVICE, "q8_linear_rmsnorm: host-only context");
  if (n == 0) return ok(ctx);
  if (int rc = set_device(ctx)) return rc;
  hipError_t e = run_gemm(ctx, la);
  if (e != hipSuccess) return hip_fail(ctx, e, "q8_linear_rmsnorm launch");
  return ok(ctx);
}

int q8_head_argmax(q8_ctx *ctx, q8_buf *w, uint64_t owt_u16, uint64_t onorm_u16, float eps,
                   q8_buf *a, uint64_t ox_f32, uint64_t oy_f32, int64_t m, int64_t n, int G,
                   int scale_dtype, q8_buf *ids, uint64_t oid_i32, q8_buf *posbuf,
                   uint64_t opos_i32, int64_t pos_step, int gather, uint64_t oemb_u16,
                   uint64_t onext_f32) {
  if (int rc = check_ctx(ctx)) return rc;
  if (int rc = check_linear(ctx, "q8_head_argmax", w, owt_u16, 1, m, n, G, scale_dtype))
    return rc;
  if (!a || !ids) return fail(ctx, Q8_ERR_ARG, "q8_head_argmax: null buffer");
  if (n < 1 || n > INT32_MAX)
    return fail(ctx, Q8_ERR_SHAPE, "q8_head_argmax: n=%lld", (long long)n);
  if (int rc = check_f32(ctx, a, ox_f32, (uint64_t)m, "q8_head_argmax", "x")) return rc;
  if (int rc = check_f32(ctx, a, oy_f32, (uint64_t)n, "q8_head_argmax", "logits")) return rc;
  if (overlaps(ox_f32, ox_f32 + (uint64_t)m, oy_f32, oy_f32 + (uint64_t)n))
    return fail(ctx, Q8_ERR_ARG, "q8_head_argmax: x and logits overlap");
  if (!fits(onorm_u16, (uint64_t)m, 2, w->size))
    return fail(ctx, Q8_ERR_RANGE, "q8_head_argmax: norm weights exceed the weight buffer");
  if (!fits(oid_i32, 1, 4, ids->size))
    return fail(ctx, Q8_ERR_RANGE, "q8_head_argmax: id slot exceeds its buffer");
  if (posbuf && !fits(opos_i32, 1, 4, posbuf->size))
    return fail(ctx, Q8_ERR_RANGE, "q8_head_argmax: position slot exceeds its buffer");
  if (pos_step < INT32_MIN || pos_step > INT32_MAX)
    return fail(ctx, Q8_ERR_ARG, "q8_head_argmax: pos_step=%lld", (long long)pos_step);
  const uint64_t rs = (uint64_t)rowstride_u16(m, G, scale_dtype);
  if (gather) {
    // the next token's embedding: n packed rows of m at oemb (vocab = n)
    if (!fits(oemb_u16, (uint64_t)n * rs, 2, w->size))
      return fail(ctx, Q8_ERR_RANGE, "q8_head_argmax: embedding table exceeds the weight buffer");
    if (int rc = check_f32(ctx, a, onext_f32, (uint64_t)m, "q8_head_argmax", "x_next")) return rc;
    if (overlaps(onext_f32, onext_f32 + (uint64_t)m, oy_f32, oy_f32 + (uint64_t)n))
      return fail(ctx, Q8_ERR_ARG, "q8_head_argmax: x_next overlaps the logits");
  }
  q8::FusedLinearArgs f;
  q8::LinearArgs &la = f.lin;
  la.w = bytes(w, owt_u16 * 2);
  la.row_bytes = (int64_t)rs * 2;
  la.x = bytes(a, ox_f32 * 4);
  la.x_is_bf16 = 0;
  la.y = fptr(a, oy_f32);
  la.s = 1;
  la.m = m;
  la.n = n;
  la.G = G;
  la.kind = scale_dtype;
  f.pre = q8::PRE_RMSNORM;
  f.post = q8::POST_ARGMAX;
  f.wn = reinterpret_cast<const uint16_t *>(bytes(w, onorm_u16 * 2));
  f.eps = eps;
  f.res = nullptr;
  f.part = ctx->gemm_ws;   // 2 x 8192 words of partials, read by the second launch
  int grid = 0;
  f.grid_out = &grid;
  if (!q8::gemv_fused_supported(f))
    return fail(ctx, Q8_ERR_UNSUPPORTED, "q8_head_argmax: m=%lld (needs m <= 16384, m %% 32 == 0, "
                "16-byte aligned rows and x, 8-byte aligned norm weights)", (long long)m);
  if (ctx->host_only) return fail(ctx, Q8_ERR_NODEVICE, "q8_head_argmax: host-only context");
  if (int rc = set_device(ctx)) return rc;
  hipError_t e = q8::launch_gemv_fused(f, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "q8_head_argmax launch");
  q8::ArgmaxFinishArgs fa;
  fa.part = ctx->gemm_ws;
  fa.nblocks = grid;
  fa.logits = la.y;
  fa.ids = reinterpret_cast<int32_t *>(bytes(ids, oid_i32 * 4));
  fa.pos = posbuf ? reinterpret_cast<int *>(bytes(posbuf, opos_i32 * 4)) : nullptr;
  fa.pos_step = (int)pos_step;
  fa.emb = gather ? bytes(w, oemb_u16 * 2) : nullptr;
  fa.row_bytes = (int64_t)rs * 2;
  fa.vocab = n;
  fa.d = m;
  fa.G = G;
  fa.kind = scale_dtype;
  fa.xnext = gather ? fptr(a, onext_f32) : nullptr;
  e = q8::launch_argmax_finish(fa, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "q8_head_argmax finish launch");
  return ok(ctx);
}

int q8_head_rmsnorm(q8_ctx *ctx, q8_buf *w, uint64_t owt_u16, q8_buf *a, uint64_t ox_f32,
                    uint64_t oy_f32, int64_t tokens, int64_t heads, int64_t head_dim, int64_t ld,
                    float eps) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!w || !a) return fail(ctx, Q8_ERR_ARG, "q8_head_rmsnorm: null buffer");
  if (tokens < 0 || heads <= 0 || head_dim <= 0 || heads > INT32_MAX / head_dim ||
      tokens > INT32_MAX / heads)
    return fail(ctx, Q8_ERR_SHAPE, "q8_head_rmsnorm: tokens=%lld, heads=%lld, head_dim=%lld",
                (long long)tokens, (long long)heads, (long long)head_dim);
  const int64_t width = heads * head_dim;
  if (ld == 0) ld = width;
  if (ld < width)
    return fail(ctx, Q8_ERR_SHAPE, "q8_head_rmsnorm: row stride %lld (0, or at least "
                "heads * head_dim = %lld)", (long long)ld, (long long)width);
  if (!fits(owt_u16, (uint64_t)head_dim, 2, w->size))
    return fail(ctx, Q8_ERR_RANGE, "q8_head_rmsnorm: norm weights exceed the weight buffer");
  const uint64_t span = rows_span(tokens, ld, (uint64_t)width);
  if (int rc = check_f32(ctx, a, ox_f32, span, "q8_head_rmsnorm", "x")) return rc;
  if (int rc = check_f32(ctx, a, oy_f32, span, "q8_head_rmsnorm", "y")) return rc;
  // y is x itself (in place) or apart from every row of x
  if (oy_f32 != ox_f32 && span && overlaps(ox_f32, ox_f32 + span, oy_f32, oy_f32 + span))
    return fail(ctx, Q8_ERR_ARG, "q8_head_rmsnorm: y overlaps x without being x");
  if (ctx->host_only) return fail(ctx, Q8_ERR_NODEVICE, "q8_head_rmsnorm: host-only context");
  if (tokens == 0) return ok(ctx);
  if (int rc = set_device(ctx)) return rc;
  hipError_t e = q8::launch_rmsnorm(reinterpret_cast<const uint16_t *>(bytes(w, owt_u16 * 2)),
                                    fptr(a, ox_f32), nullptr, nullptr, fptr(a, oy_f32),
                                    tokens * heads, head_dim, eps, ctx->stream, heads, ld);
  if (e != hipSuccess) return hip_fail(ctx, e, "q8_head_rmsnorm launch");
  return ok(ctx);
}

int q8_rmsnorm(q8_ctx *ctx, q8_buf *w, uint64_t owt_u16, q8_buf *a, uint64_t ox_f32,
               uint64_t oy_f32, int64_t rows, int64_t d, float eps) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!w || !a) return fail(ctx, Q8_ERR_ARG, "q8_rmsnorm: null buffer");
  if (rows < 0 || d <= 0)
    return fail(ctx, Q8_ERR_SHAPE, "q8_rmsnorm: rows=%lld, d=%lld", (long long)rows, (long long)d);
  const uint64_t n = (uint64_t)rows * (uint64_t)d;
  if (!fits(owt_u16, (uint64_t)d, 2, w->size))
    return fail(ctx, Q8_ERR_RANGE, "q8_rmsnorm: norm weights exceed the weight buffer");
  if (int rc = check_f32(ctx, a, ox_f32, n, "q8_rmsnorm", "x")) return rc;
  if (int rc = check_f32(ctx, a, oy_f32, n, "q8_rmsnorm", "y")) return rc;
  if (bad_alias(oy_f32, n, ox_f32, n))
    return fail(ctx, Q8_ERR_ARG, "q8_rmsnorm: y partially overlaps x");
  if (ctx->host_only) return fail(ctx, Q8_ERR_NODEVICE, "q8_rmsnorm: host-only context");
  if (rows == 0) return ok(ctx);
  if (int rc = set_device(ctx)) return rc;
  hipError_t e = q8::launch_rmsnorm(reinterpret_cast<const uint16_t *>(bytes(w, owt_u16 * 2)),
                                    fptr(a, ox_f32), nullptr, nullptr, fptr(a, oy_f32), rows, d,
                                    eps, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "q8_rmsnorm launch");
  return ok(ctx);
}

int q8_add_rmsnorm(q8_ctx *ctx, q8_buf *w, uint64_t owt_u16, q8_buf *a, uint64_t ox_f32,
                   uint64_t oo_f32, uint64_t oh_f32, uint64_t oy_f32, int64_t rows, int64_t d,
                   float eps) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!w || !a) return fail(ctx, Q8_ERR_ARG, "q8_add_rmsnorm: null buffer");
  if (rows < 0 || d <= 0)
    return fail(ctx, Q8_ERR_SHAPE, "q8_add_rmsnorm: rows=%lld, d=%lld", (long long)rows,
                (long long)d);
  const uint64_t n = (uint64_t)rows * (uint64_t)d;
  if (!fits(owt_u16, (uint64_t)d, 2, w->size))
    return fail(ctx, Q8_ERR_RANGE, "q8_add_rmsnorm: norm weights exceed the weight buffer");
  const uint64_t offs[4] = {ox_f32, oo_f32, oh_f32, oy_f32};
  const char *names[4] = {"x", "o", "h", "y"};
  for (int i = 0; i < 4; ++i)
    if (int rc = check_f32(ctx, a, offs[i], n, "q8_add_rmsnorm", names[i])) return rc;
  if (bad_alias(oh_f32, n, ox_f32, n) || bad_alias(oh_f32, n, oo_f32, n) ||
      bad_alias(oy_f32, n, ox_f32, n) || bad_alias(oy_f32, n, oo_f32, n) ||
      bad_alias(oy_f32, n, oh_f32, n))
    return fail(ctx, Q8_ERR_ARG, "q8_add_rmsnorm: an output partially overlaps another range");
  if (ctx->host_only) return fail(ctx, Q8_ERR_NODEVICE, "q8_add_rmsnorm: host-only context");
  if (rows == 0) return ok(ctx);
  if (int rc = set_device(ctx)) return rc;
  hipError_t e = q8::launch_rmsnorm(reinterpret_cast<const uint16_t *>(bytes(w, owt_u16 * 2)),
                                    fptr(a, ox_f32), fptr(a, oo_f32), fptr(a, oh_f32),
                                    fptr(a, oy_f32), rows, d, eps, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "q8_add_rmsnorm launch");
  return ok(ctx);
}

int q8_rope_kv(q8_ctx *ctx, q8_buf *a, uint64_t oq_f32, uint64_t ok_f32, uint64_t ov_f32,
               uint64_t oinv_f32, q8_buf *kv, uint64_t okc_f16, uint64_t ovc_f16, int64_t maxlen,
               int64_t s, int64_t pos0, q8_buf *posbuf, uint64_t opos_i32, int nheads, int nkv,
               int head_dim, int64_t ld) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!a || !kv) return fail(ctx, Q8_ERR_ARG, "q8_rope_kv: null buffer");
  if (int rc = check_heads(ctx, nheads, nkv, head_dim, "q8_rope_kv")) return rc;
  if (s < 0 || maxlen <= 0 || maxlen > INT32_MAX)
    return fail(ctx, Q8_ERR_SHAPE, "q8_rope_kv: s=%lld, maxlen=%lld", (long long)s,
                (long long)maxlen);
  if (!cache_block_ok(maxlen, nkv, head_dim))
    return fail(ctx, Q8_ERR_SHAPE, "q8_rope_kv: maxlen=%lld (a cache block must stay under "
                "2 GiB)", (long long)maxlen);
  const int64_t qdim = (int64_t)nheads * head_dim, kvdim = (int64_t)nkv * head_dim;
  if (ld != 0 && (ld < qdim || ld < kvdim || ld > INT32_MAX || s > INT32_MAX))
    return fail(ctx, Q8_ERR_SHAPE, "q8_rope_kv: row stride %lld (0, or at least the q and k "
                "row widths %lld, %lld)", (long long)ld, (long long)qdim, (long long)kvdim);
  const int64_t ldq = ld ? ld : qdim, ldk = ld ? ld : kvdim;
  const uint64_t qn = rows_span(s, ldq, qdim), kn = rows_span(s, ldk, kvdim);
  const uint64_t cn = (uint64_t)maxlen * nkv * head_dim;
  if (int rc = check_f32(ctx, a, oq_f32, qn, "q8_rope_kv", "q")) return rc;
  if (int rc = check_f32(ctx, a, ok_f32, kn, "q8_rope_kv", "k")) return rc;
  if (int rc = check_f32(ctx, a, ov_f32, kn, "q8_rope_kv", "v")) return rc;
  if (int rc = check_f32(ctx, a, oinv_f32, (uint64_t)head_dim / 2, "q8_rope_kv", "inv_freq"))
    return rc;
  // q and k are rotated in place while v and inv_freq are read by the same
  // launch: no element of v or inv_freq may be a q or k element, nor q a k
  // element.
  if (ld == 0) {
    if (overlaps(oq_f32, oq_f32 + qn, ok_f32, ok_f32 + kn))
      return fail(ctx, Q8_ERR_ARG, "q8_rope_kv: q and k overlap");
    if (overlaps(ov_f32, ov_f32 + kn, oq_f32, oq_f32 + qn) ||
        overlaps(ov_f32, ov_f32 + kn, ok_f32, ok_f32 + kn))
      return fail(ctx, Q8_ERR_ARG, "q8_rope_kv: v overlaps q or k");
  } else {
    // rows of one stride: k's (v's) columns, taken modulo ld from q's (k's)
    // row start, must lie in [width, ld), wrapped rows included
    if (!stride_disjoint(oq_f32, qdim, ok_f32, kvdim, ld))
      return fail(ctx, Q8_ERR_ARG, "q8_rope_kv: q and k rows overlap at stride %lld",
                  (long long)ld);
    if (!stride_disjoint(oq_f32, qdim, ov_f32, kvdim, ld) ||
        !stride_disjoint(ok_f32, kvdim, ov_f32, kvdim, ld))
      return fail(ctx, Q8_ERR_ARG, "q8_rope_kv: v rows overlap q or k rows at stride %lld",
                  (long long)ld);
  }
  {
    const uint64_t oi = oinv_f32, ni = (uint64_t)head_dim / 2;
    if (overlaps(oi, oi + ni, oq_f32, oq_f32 + qn) || overlaps(oi, oi + ni, ok_f32, ok_f32 + kn))
      return fail(ctx, Q8_ERR_ARG, "q8_rope_kv: inv_freq overlaps the q or k rows");
  }
  if (!fits(okc_f16, cn, 2, kv->size) || !fits(ovc_f16, cn, 2, kv->size))
    return fail(ctx, Q8_ERR_RANGE, "q8_rope_kv: K or V cache block exceeds the KV buffer");
  if (overlaps(okc_f16, okc_f16 + cn, ovc_f16, ovc_f16 + cn))
    return fail(ctx, Q8_ERR_ARG, "q8_rope_kv: K and V cache blocks overlap");
  if (int rc = check_pos(ctx, posbuf, opos_i32, pos0, s, maxlen, "q8_rope_kv")) return rc;
  if (ctx->host_only) return fail(ctx, Q8_ERR_NODEVICE, "q8_rope_kv: host-only context");
  if (s == 0) return ok(ctx);
  if (int rc = set_device(ctx)) return rc;
  __half *kvp = reinterpret_cast<__half *>(kv->ptr);
  const int *posp = posbuf ? reinterpret_cast<const int *>(bytes(posbuf, opos_i32 * 4)) : nullptr;
  hipError_t e = q8::launch_rope_kv(fptr(a, oq_f32), fptr(a, ok_f32), fptr(a, ov_f32),
                                    kvp + okc_f16, kvp + ovc_f16, fptr(a, oinv_f32), (int)s, posp,
                                    (int)pos0, nheads, nkv, head_dim, maxlen, ldq, ldk,
                                    ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "q8_rope_kv launch");
  return ok(ctx);
}

uint64_t q8_attention_scratch_floats(int64_t s, int nheads, int head_dim, int64_t maxlen) {
  if (s < 0 || nheads <= 0 || head_dim <= 0 || maxlen <= 0 || s >= q8::kPrefillMinRows) return 0;
  return (uint64_t)s * nheads * attn_nsplit(maxlen) * (uint64_t)(head_dim + 2);
}

int q8_attention(q8_ctx *ctx, q8_buf *a, uint64_t oq_f32, q8_buf *kv, uint64_t okc_f16,
                 uint64_t ovc_f16, int64_t maxlen, uint64_t oy_f32, uint64_t oscratch_f32,
                 int64_t s, int64_t pos0, q8_buf *posbuf, uint64_t opos_i32, int nheads, int nkv,
                 int head_dim, int64_t ldq) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!a || !kv) return fail(ctx, Q8_ERR_ARG, "q8_attention: null buffer");
  if (int rc = check_heads(ctx, nheads, nkv, head_dim, "q8_attention")) return rc;
  const int grp = nheads / nkv;
  if ((head_dim != 64 && head_dim != 128) || (grp != 1 && grp != 2 && grp != 4 && grp != 8))
    return fail(ctx, Q8_ERR_UNSUPPORTED, "q8_attention: head_dim=%d, nheads/nkv=%d "
                "(supported: head_dim 64 or 128, nheads/nkv 1, 2, 4 or 8)", head_dim, grp);
  if (s < 0 || s > 65535 || maxlen <= 0 || maxlen > INT32_MAX)
    return fail(ctx, Q8_ERR_SHAPE, "q8_attention: s=%lld, maxlen=%lld", (long long)s,
                (long long)maxlen);
  if (!cache_block_ok(maxlen, nkv, head_dim))
    return fail(ctx, Q8_ERR_SHAPE, "q8_attention: maxlen=%lld (a cache block must stay under "
                "2 GiB)", (long long)maxlen);
  const int64_t qdim = (int64_t)nheads * head_dim;
  if (ldq != 0 && (ldq < qdim || ldq > INT32_MAX))
    return fail(ctx, Q8_ERR_SHAPE, "q8_attention: q row stride %lld (0, or at least %lld)",
                (long long)ldq, (long long)qdim);
  if (ldq == 0) ldq = qdim;
  const uint64_t qn = (uint64_t)s * qdim, qspan = rows_span(s, ldq, qdim);
  const uint64_t cn = (uint64_t)maxlen * nkv * head_dim;
  const uint64_t sn = q8_attention_scratch_floats(s, nheads, head_dim, maxlen);
  if (int rc = check_f32(ctx, a, oq_f32, qspan, "q8_attention", "q")) return rc;
  if (int rc = check_f32(ctx, a, oy_f32, qn, "q8_attention", "out")) return rc;
  if (int rc = check_f32(ctx, a, oscratch_f32, sn, "q8_attention", "scratch")) return rc;
  if (overlaps(oy_f32, oy_f32 + qn, oq_f32, oq_f32 + qspan) ||
      overlaps(oscratch_f32, oscratch_f32 + sn, oq_f32, oq_f32 + qspan) ||
      overlaps(oscratch_f32, oscratch_f32 + sn, oy_f32, oy_f32 + qn))
    return fail(ctx, Q8_ERR_ARG, "q8_attention: q, out and scratch must not overlap");
  // The one-pass kernel moves q and out rows as 16-byte vectors.
  const uintptr_t abase = reinterpret_cast<uintptr_t>(a->ptr);
  if (s >= q8::kPrefillMinRows &&
      ((abase + oq_f32 * 4) % 16 != 0 || (abase + oy_f32 * 4) % 16 != 0 || ldq % 4 != 0))
    return fail(ctx, Q8_ERR_UNSUPPORTED, "q8_attention: from %d rows on, q and out must start "
                "16-byte aligned and the q row stride be a multiple of 4", q8::kPrefillMinRows);
  if (!fits(okc_f16, cn, 2, kv->size) || !fits(ovc_f16, cn, 2, kv->size))
    return fail(ctx, Q8_ERR_RANGE, "q8_attention: K or V cache block exceeds the KV buffer");
  if (int rc = check_pos(ctx, posbuf, opos_i32, pos0, s, maxlen, "q8_attention")) return rc;
  if (ctx->host_only) return fail(ctx, Q8_ERR_NODEVICE, "q8_attention: host-only context");
  if (s == 0) return ok(ctx);
  if (int rc = set_device(ctx)) return rc;
  const __half *kvp = reinterpret_cast<const __half *>(kv->ptr);
  q8::AttnArgs aa;
  aa.q = fptr(a, oq_f32);
  aa.kc = kvp + okc_f16;
  aa.vc = kvp + ovc_f16;
  aa.part = fptr(a, oscratch_f32);
  aa.out = fptr(a, oy_f32);
  aa.s = (int)s;
  aa.nheads = nheads;
  aa.nkv = nkv;
  aa.head_dim = head_dim;
  aa.nsplit = (int)attn_nsplit(maxlen);
  aa.posp = posbuf ? reinterpret_cast<const int *>(bytes(posbuf, opos_i32 * 4)) : nullptr;
  aa.pos0 = (int)pos0;
  aa.maxlen = (int)maxlen;
  aa.ldq = ldq;
  hipError_t e = q8::launch_attention(aa, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "q8_attention launch");
  return ok(ctx);
}

int q8_decode_attention(q8_ctx *ctx, q8_buf *a, uint64_t oq_f32, uint64_t ok_f32,
                        uint64_t ov_f32, uint64_t oinv_f32, q8_buf *kv, uint64_t okc_f16,
                        uint64_t ovc_f16, int64_t maxlen, uint64_t oy_f32, int64_t pos0,
                        q8_buf *posbuf, uint64_t opos_i32, int nheads, int nkv, int head_dim,
                        q8_buf *wn, uint64_t oqnorm_u16, uint64_t oknorm_u16, float eps) {
  if (int rc = check_ctx(ctx)) return rc;
  if (wn && (!fits(oqnorm_u16, (uint64_t)(head_dim > 0 ? head_dim : 0), 2, wn->size) ||
             !fits(oknorm_u16, (uint64_t)(head_dim > 0 ? head_dim : 0), 2, wn->size)))
    return fail(ctx, Q8_ERR_RANGE, "q8_decode_attention: q/k norm weights exceed the weight "
                "buffer");
  if (!a || !kv) return fail(ctx, Q8_ERR_ARG, "q8_decode_attention: null buffer");
  if (int rc = check_heads(ctx, nheads, nkv, head_dim, "q8_decode_attention")) return rc;
  const int grp = nheads / nkv;
  if ((head_dim != 64 && head_dim != 128) || (grp != 1 && grp != 2 && grp != 4 && grp != 8))
    return fail(ctx, Q8_ERR_UNSUPPORTED, "q8_decode_attention: head_dim=%d, nheads/nkv=%d "
                "(supported: head_dim 64 or 128, nheads/nkv 1, 2, 4 or 8)", head_dim, grp);
  const uint64_t qn = (uint64_t)nheads * head_dim, kn = (uint64_t)nkv * head_dim;
  // cache rows are read through 32-bit buffer offsets
  if (maxlen <= 0 || (uint64_t)maxlen * kn * 2 >= ((uint64_t)1 << 31))
    return fail(ctx, Q8_ERR_SHAPE, "q8_decode_attention: maxlen=%lld (a cache block must stay "
                "under 2 GiB)", (long long)maxlen);
  const uint64_t cn = (uint64_t)maxlen * kn;
  const int nsplit = q8::decode_attn_nsplit(maxlen, head_dim, grp);
  if ((uint64_t)nheads * nsplit * (head_dim + 2) > (uint64_t)kGemmWsFloats)
    return fail(ctx, Q8_ERR_UNSUPPORTED, "q8_decode_attention: nheads=%d exceeds the context's "
                "attention scratch", nheads);
  if (int rc = check_f32(ctx, a, oq_f32, qn, "q8_decode_attention", "q")) return rc;
  if (int rc = check_f32(ctx, a, ok_f32, kn, "q8_decode_attention", "k")) return rc;
  if (int rc = check_f32(ctx, a, ov_f32, kn, "q8_decode_attention", "v")) return rc;
  if (int rc = check_f32(ctx, a, oinv_f32, (uint64_t)head_dim / 2, "q8_decode_attention",
                         "inv_freq"))
    return rc;
  if (int rc = check_f32(ctx, a, oy_f32, qn, "q8_decode_attention", "out")) return rc;
  if (overlaps(oy_f32, oy_f32 + qn, oq_f32, oq_f32 + qn) ||
      overlaps(oy_f32, oy_f32 + qn, ok_f32, ok_f32 + kn) ||
      overlaps(oy_f32, oy_f32 + qn, ov_f32, ov_f32 + kn))
    return fail(ctx, Q8_ERR_ARG, "q8_decode_attention: out overlaps q, k or v");
  if (!fits(okc_f16, cn, 2, kv->size) || !fits(ovc_f16, cn, 2, kv->size))
    return fail(ctx, Q8_ERR_RANGE, "q8_decode_attention: K or V cache block exceeds the KV buffer");
  if (overlaps(okc_f16, okc_f16 + cn, ovc_f16, ovc_f16 + cn))
    return fail(ctx, Q8_ERR_ARG, "q8_decode_attention: K and V cache blocks overlap");
  if (int rc = check_pos(ctx, posbuf, opos_i32, pos0, 1, maxlen, "q8_decode_attention")) return rc;
  if (ctx->host_only) return fail(ctx, Q8_ERR_NODEVICE, "q8_decode_attention: host-only context");
  if (int rc = set_device(ctx)) return rc;
  __half *kvp = reinterpret_cast<__half *>(kv->ptr);
  q8::DecodeAttnArgs da;
  da.q = fptr(a, oq_f32);
  da.k = fptr(a, ok_f32);
  da.v = fptr(a, ov_f32);
  da.inv = fptr(a, oinv_f32);
  da.kc = kvp + okc_f16;
  da.vc = kvp + ovc_f16;
  da.out = fptr(a, oy_f32);
  da.part = ctx->gemm_ws;
  if (wn) {
    da.qnorm = reinterpret_cast<const uint16_t *>(bytes(wn, oqnorm_u16 * 2));
    da.knorm = reinterpret_cast<const uint16_t *>(bytes(wn, oknorm_u16 * 2));
    da.eps = eps;
  }
  da.nheads = nheads;
  da.nkv = nkv;
  da.head_dim = head_dim;
  da.nsplit = nsplit;
  da.posp = posbuf ? reinterpret_cast<const int *>(bytes(posbuf, opos_i32 * 4)) : nullptr;
  da.pos0 = (int)pos0;
  da.maxlen = (int)maxlen;
  hipError_t e = q8::launch_decode_attention(da, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "q8_decode_attention launch");
  return ok(ctx);
}

int q8_swiglu(q8_ctx *ctx, q8_buf *a, uint64_t og_f32, uint64_t ou_f32, int64_t n) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!a) return fail(ctx, Q8_ERR_ARG, "q8_swiglu: null buffer");
  if (n < 0) return fail(ctx, Q8_ERR_SHAPE, "q8_swiglu: n=%lld", (long long)n);
  if (int rc = check_f32(ctx, a, og_f32, (uint64_t)n, "q8_swiglu", "g")) return rc;
  if (int rc = check_f32(ctx, a, ou_f32, (uint64_t)n, "q8_swiglu", "u")) return rc;
  if (overlaps(og_f32, og_f32 + n, ou_f32, ou_f32 + n))
    return fail(ctx, Q8_ERR_ARG, "q8_swiglu: g and u overlap");
  if (ctx->host_only) return fail(ctx, Q8_ERR_NODEVICE, "q8_swiglu: host-only context");
  if (n == 0) return ok(ctx);
  if (int rc = set_device(ctx)) return rc;
  hipError_t e = q8::launch_swiglu(fptr(a, og_f32), fptr(a, ou_f32), n, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "q8_swiglu launch");
  return ok(ctx);
}

int q8_res_add(q8_ctx *ctx, q8_buf *a, uint64_t ox_f32, uint64_t oo_f32, uint64_t oy_f32,
               int64_t n) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!a) return fail(ctx, Q8_ERR_ARG, "q8_res_add: null buffer");
  if (n < 0) return fail(ctx, Q8_ERR_SHAPE, "q8_res_add: n=%lld", (long long)n);
  const uint64_t offs[3] = {ox_f32, oo_f32, oy_f32};
  const char *names[3] = {"x", "o", "y"};
  for (int i = 0; i < 3; ++i)
    if (int rc = check_f32(ctx, a, offs[i], (uint64_t)n, "q8_res_add", names[i])) return rc;
  if (bad_alias(oy_f32, n, ox_f32, n) || bad_alias(oy_f32, n, oo_f32, n))
    return fail(ctx, Q8_ERR_ARG, "q8_res_add: y partially overlaps an input");
  if (ctx->host_only) return fail(ctx, Q8_ERR_NODEVICE, "q8_res_add: host-only context");
  if (n == 0) return ok(ctx);
  if (int rc = set_device(ctx)) return rc;
  hipError_t e = q8::launch_res_add(fptr(a, ox_f32), fptr(a, oo_f32), fptr(a, oy_f32), n,
                                    ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "q8_res_add launch");
  return ok(ctx);
}

int q8_add(q8_ctx *ctx, q8_buf *a, uint64_t ox_f32, uint64_t oy_f32, int64_t n) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!a) return fail(ctx, Q8_ERR_ARG, "q8_add: null buffer");
  if (n < 0) return fail(ctx, Q8_ERR_SHAPE, "q8_add: n=%lld", (long long)n);
  if (int rc = check_f32(ctx, a, ox_f32, (uint64_t)n, "q8_add", "x")) return rc;
  if (int rc = check_f32(ctx, a, oy_f32, (uint64_t)n, "q8_add", "y")) return rc;
  if (bad_alias(oy_f32, n, ox_f32, n))
    return fail(ctx, Q8_ERR_ARG, "q8_add: y partially overlaps x");
  if (ctx->host_only) return fail(ctx, Q8_ERR_NODEVICE, "q8_add: host-only context");
  if (n == 0) return ok(ctx);
  if (int rc = set_device(ctx)) return rc;
  hipError_t e = q8::launch_add(fptr(a, ox_f32), fptr(a, oy_f32), n, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "q8_add launch");
  return ok(ctx);
}

int q8_argmax(q8_ctx *ctx, q8_buf *a, uint64_t ox_f32, int64_t n, q8_buf *ids, uint64_t oid_i32) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!a || !ids) return fail(ctx, Q8_ERR_ARG, "q8_argmax: null buffer");
  if (n <= 0 || n > INT32_MAX) return fail(ctx, Q8_ERR_SHAPE, "q8_argmax: n=%lld", (long long)n);
  if (int rc = check_f32(ctx, a, ox_f32, (uint64_t)n, "q8_argmax", "x")) return rc;
  if (!fits(oid_i32, 1, 4, ids->size))
    return fail(ctx, Q8_ERR_RANGE, "q8_argmax: id offset exceeds its buffer");
  if (ctx->host_only) return fail(ctx, Q8_ERR_NODEVICE, "q8_argmax: host-only context");
  if (int rc = set_device(ctx)) return rc;
  hipError_t e = q8::launch_argmax(fptr(a, ox_f32), n,
                                   reinterpret_cast<int32_t *>(bytes(ids, oid_i32 * 4)),
                                   ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "q8_argmax launch");
  return ok(ctx);
}

int q8_pos_advance(q8_ctx *ctx, q8_buf *posbuf, uint64_t opos_i32, int64_t s) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!posbuf) return fail(ctx, Q8_ERR_ARG, "q8_pos_advance: null buffer");
  if (s < 0 || s > INT32_MAX) return fail(ctx, Q8_ERR_SHAPE, "q8_pos_advance: s=%lld", (long long)s);
  if (!fits(opos_i32, 1, 4, posbuf->size))
    return fail(ctx, Q8_ERR_RANGE, "q8_pos_advance: offset exceeds its buffer");
  if (ctx->host_only) return fail(ctx, Q8_ERR_NODEVICE, "q8_pos_advance: host-only context");
  if (int rc = set_device(ctx)) return rc;
  hipError_t e = q8::launch_pos_advance(reinterpret_cast<int *>(bytes(posbuf, opos_i32 * 4)),
                                        (int)s, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "q8_pos_advance launch");
  return ok(ctx);
}

// ---- HIP graphs -------------------------------------------------------------------

struct q8_graph {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
};

int q8_graph_begin(q8_ctx *ctx) {
  if (int rc = check_ctx(ctx)) return rc;
  if (ctx->host_only) return fail(ctx, Q8_ERR_NODEVICE, "q8_graph_begin: host-only context");
  if (int rc = set_device(ctx)) return rc;
  hipError_t e = hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal);
  if (e != hipSuccess) return hip_fail(ctx, e, "q8_graph_begin");
  return ok(ctx);
}

int q8_graph_end(q8_ctx *ctx, void **graph) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!graph) return fail(ctx, Q8_ERR_ARG, "q8_graph_end: null output pointer");
  *graph = nullptr;
  if (ctx->host_only) return fail(ctx, Q8_ERR_NODEVICE, "q8_graph_end: host-only context");
  if (int rc = set_device(ctx)) return rc;
  q8_graph *g = new (std::nothrow) q8_graph();
  hipGraph_t hg = nullptr;
  hipError_t e = hipStreamEndCapture(ctx->stream, &hg);
  if (!g) {
    if (hg) (void)hipGraphDestroy(hg);
    return fail(ctx, Q8_ERR_NOMEM, "q8_graph_end: out of host memory");
  }
  if (e != hipSuccess) {
    delete g;
    return hip_fail(ctx, e, "q8_graph_end (capture)");
  }
  g->graph = hg;
  e = hipGraphInstantiate(&g->exec, hg, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    (void)hipGraphDestroy(hg);
    delete g;
    return hip_fail(ctx, e, "q8_graph_end (instantiate)");
  }
  *graph = g;
  return ok(ctx);
}

int q8_graph_launch(q8_ctx *ctx, void *graph) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!graph) return fail(ctx, Q8_ERR_ARG, "q8_graph_launch: null graph");
  if (ctx->host_only) return fail(ctx, Q8_ERR_NODEVICE, "q8_graph_launch: host-only context");
  if (int rc = set_device(ctx)) return rc;
  hipError_t e = hipGraphLaunch(static_cast<q8_graph *>(graph)->exec, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "q8_graph_launch");
  return ok(ctx);
}

void q8_graph_destroy(void *graph) {
  if (!graph) return;
  q8_graph *g = static_cast<q8_graph *>(graph);
  if (g->exec) (void)hipGraphExecDestroy(g->exec);
  if (g->graph) (void)hipGraphDestroy(g->graph);
  delete g;
}

}  // extern "C"
