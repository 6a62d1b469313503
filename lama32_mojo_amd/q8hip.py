"""ctypes binding of libq8hip.so (C ABI declared in include/q8hip.h).

This is the same binding a Mojo host would make with sys.ffi: plain ints and
pointers only.  The library must be built (``python -m lama32_mojo_amd.build``);
there is no CPU fallback -- loading fails loudly when it is missing.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libq8hip.so")

Q8_OK = 0
Q8_ERR_ARG = -1
Q8_ERR_SHAPE = -2
Q8_ERR_RANGE = -3
Q8_ERR_HIP = -4
Q8_ERR_NOMEM = -5
Q8_ERR_NODEVICE = -6
Q8_ERR_UNSUPPORTED = -7

Q8_SCALE_F16 = 1
Q8_SCALE_F32 = 2
Q8_SRC_BF16 = 1
Q8_SRC_F32 = 2
Q8_DEVICE_NONE = -1

SCALE = {"f16": Q8_SCALE_F16, "f32": Q8_SCALE_F32}


def scale_code(scale) -> int:
    """"f16" / "f32" -> Q8_SCALE_*; integers pass through unchanged (so the
    library itself rejects unknown codes)."""
    return scale if isinstance(scale, int) else SCALE[scale]

ERROR_NAMES = {
    Q8_ERR_ARG: "Q8_ERR_ARG", Q8_ERR_SHAPE: "Q8_ERR_SHAPE",
    Q8_ERR_RANGE: "Q8_ERR_RANGE", Q8_ERR_HIP: "Q8_ERR_HIP",
    Q8_ERR_NOMEM: "Q8_ERR_NOMEM", Q8_ERR_NODEVICE: "Q8_ERR_NODEVICE",
    Q8_ERR_UNSUPPORTED: "Q8_ERR_UNSUPPORTED",
}

# Every symbol include/q8hip.h declares, with (restype, argtypes).
_P = ctypes.c_void_p
_U64 = ctypes.c_uint64
_I64 = ctypes.c_int64
_I = ctypes.c_int
SIGNATURES = {
    "q8_version": (_I, []),
    "q8_rowstride_u16": (_U64, [_I64, _I, _I]),
    "q8_create": (_I, [_I, ctypes.POINTER(_P)]),
    "q8_destroy": (None, [_P]),
    "q8_set_stream": (_I, [_P, _P]),
    "q8_get_stream": (_P, [_P]),
    "q8_sync": (_I, [_P]),
    "q8_last_error": (ctypes.c_char_p, [_P]),
    "q8_buf_alloc": (_I, [_P, _U64, ctypes.POINTER(_P)]),
    "q8_buf_wrap": (_I, [_P, _P, _U64, ctypes.POINTER(_P)]),
    "q8_buf_free": (None, [_P, _P]),
    "q8_buf_size": (_U64, [_P]),
    "q8_buf_device_ptr": (_P, [_P]),
    "q8_buf_upload": (_I, [_P, _P, _U64, _P, _U64]),
    "q8_buf_download": (_I, [_P, _P, _U64, _P, _U64]),
    "q8_quantize_pack": (_I, [_P, _P, _U64, _I, _I64, _I64, _P, _U64, _I, _I]),
    "q8_linear": (_I, [_P, _P, _U64, _P, _U64, _U64, _I64, _I64, _I64, _I, _I]),
    "q8_linear_bf16act": (_I, [_P, _P, _U64, _P, _U64, _P, _U64, _I64, _I64, _I64, _I, _I]),
    "q8_linear_noalloc": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I, _I]),
    "q8_embed_gather": (_I, [_P, _P, _U64, _P, _U64, _P, _U64, _I64, _I64, _I64, _I, _I]),
    "q8_linear_fused": (_I, [_P, _P, _U64, _P, _U64, _U64, _I64, _I64, _I, _I, _I, _U64,
                            ctypes.c_float, _I, _U64]),
    "q8_head_argmax": (_I, [_P, _P, _U64, _U64, ctypes.c_float, _P, _U64, _U64, _I64, _I64, _I,
                           _I, _P, _U64, _P, _U64, _I64, _I, _U64, _U64]),
    "q8_rmsnorm": (_I, [_P, _P, _U64, _P, _U64, _U64, _I64, _I64, ctypes.c_float]),
    "q8_head_rmsnorm": (_I, [_P, _P, _U64, _P, _U64, _U64, _I64, _I64, _I64, _I64,
                             ctypes.c_float]),
    "q8_st_open": (_I, [ctypes.c_char_p, ctypes.POINTER(_P)]),
    "q8_st_close": (None, [_P]),
    "q8_st_error": (ctypes.c_char_p, []),
    "q8_st_count": (_I64, [_P]),
    "q8_st_find": (_I64, [_P, ctypes.c_char_p]),
    "q8_st_info": (_I, [_P, _I64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_char_p),
                        ctypes.POINTER(_I), ctypes.POINTER(ctypes.POINTER(_I64)),
                        ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_U64),
                        ctypes.POINTER(_U64)]),
    "q8_st_metadata_count": (_I64, [_P]),
    "q8_st_metadata": (_I, [_P, _I64, ctypes.POINTER(ctypes.c_char_p),
                            ctypes.POINTER(ctypes.c_char_p)]),
    "q8_st_read": (_I, [_P, _I64, _U64, _P, _U64]),
    "q8_st_upload": (_I, [_P, _P, _I64, _U64, _U64, _P, _U64]),
    "q8_stw_open": (_I, [ctypes.c_char_p, _I64, ctypes.POINTER(ctypes.c_char_p),
                         ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_I),
                         ctypes.POINTER(_I64), _I64, ctypes.POINTER(ctypes.c_char_p),
                         ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_P)]),
    "q8_stw_put": (_I, [_P, _I64, _P, _U64]),
    "q8_stw_close": (_I, [_P]),
    "q8_add_rmsnorm": (_I, [_P, _P, _U64, _P, _U64, _U64, _U64, _U64, _I64, _I64,
                           ctypes.c_float]),
    "q8_rope_kv": (_I, [_P, _P, _U64, _U64, _U64, _U64, _P, _U64, _U64, _I64, _I64, _I64, _P,
                       _U64, _I, _I, _I, _I64]),
    "q8_attention_scratch_floats": (_U64, [_I64, _I, _I, _I64]),
    "q8_attention": (_I, [_P, _P, _U64, _P, _U64, _U64, _I64, _U64, _U64, _I64, _I64, _P, _U64,
                         _I, _I, _I, _I64]),
    "q8_decode_attention": (_I, [_P, _P, _U64, _U64, _U64, _U64, _P, _U64, _U64, _I64, _U64,
                                _I64, _P, _U64, _I, _I, _I, _P, _U64, _U64, ctypes.c_float]),
    "q8_linear_swiglu": (_I, [_P, _P, _U64, _P, _U64, _U64, _U64, _I64, _I64, _I64, _I, _I,
                              _I64]),
    "q8_linear_rmsnorm": (_I, [_P, _P, _U64, _U64, ctypes.c_float, _P, _U64, _I, _U64, _U64,
                               _U64, _I64, _I64, _I64, _I, _I]),
    "q8_swiglu": (_I, [_P, _P, _U64, _U64, _I64]),
    "q8_res_add": (_I, [_P, _P, _U64, _U64, _U64, _I64]),
    "q8_add": (_I, [_P, _P, _U64, _U64, _I64]),
    "q8_argmax": (_I, [_P, _P, _U64, _I64, _P, _U64]),
    "q8_pos_advance": (_I, [_P, _P, _U64, _I64]),
    "q8_graph_begin": (_I, [_P]),
    "q8_graph_end": (_I, [_P, ctypes.POINTER(_P)]),
    "q8_graph_launch": (_I, [_P, _P]),
    "q8_graph_destroy": (None, [_P]),
}


class Q8Error(RuntimeError):
    """A libq8hip call returned a negative status."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"{ERROR_NAMES.get(code, code)}: {msg}")
        self.code = code
        self.msg = msg


_LIB = None


def lib() -> ctypes.CDLL:
    """Load libq8hip.so once; raise if it has not been built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} not found: build it with `python -m lama32_mojo_amd.build`")
        # torch ships its own libamdhip64.so.7 under the same SONAME; whichever
        # copy loads first serves the whole process.  Load torch's first when
        # torch is present, so the process has one HIP runtime in one order
        # whether or not the caller touches torch later (torch cannot find the
        # GPU when it comes second).
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        cdll = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(cdll, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = cdll
    return _LIB


def rowstride_u16(m: int, G: int = 64, scale="f16") -> int:
    """Packed row length in u16 (q8_rowstride, src/llama_q8.mojo:26-28)."""
    r = lib().q8_rowstride_u16(int(m), int(G), scale_code(scale))
    if r == 0:
        raise Q8Error(Q8_ERR_SHAPE, f"invalid layout m={m} G={G} scale={scale}")
    return int(r)


class Context:
    """One device + one HIP stream (the reference's DeviceContext)."""

    def __init__(self, device: int = 0):
        self._lib = lib()
        h = ctypes.c_void_p()
        rc = self._lib.q8_create(int(device), ctypes.byref(h))
        if rc != Q8_OK:
            raise Q8Error(rc, self._lib.q8_last_error(None).decode())
        self.h = h
        self.device = device

    def check(self, rc: int) -> None:
        if rc != Q8_OK:
            raise Q8Error(rc, self._lib.q8_last_error(self.h).decode())

    @property
    def host_only(self) -> bool:
        return self.device == Q8_DEVICE_NONE

    def sync(self) -> None:
        self.check(self._lib.q8_sync(self.h))

    def set_stream(self, hip_stream: int | None) -> None:
        self.check(self._lib.q8_set_stream(self.h, hip_stream or None))

    @property
    def stream(self) -> int:
        return self._lib.q8_get_stream(self.h) or 0

    def close(self) -> None:
        if getattr(self, "h", None):
            self._lib.q8_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ---- buffers ------------------------------------------------------------
    def alloc(self, nbytes: int) -> "Buffer":
        return Buffer.alloc(self, nbytes)

    def wrap(self, device_ptr: int, nbytes: int) -> "Buffer":
        return Buffer.wrap(self, device_ptr, nbytes)

    # ---- graphs -------------------------------------------------------------
    def graph_begin(self) -> None:
        self.check(self._lib.q8_graph_begin(self.h))

    def graph_end(self) -> "Graph":
        g = ctypes.c_void_p()
        self.check(self._lib.q8_graph_end(self.h, ctypes.byref(g)))
        return Graph(self, g)


class Graph:
    def __init__(self, ctx: Context, h):
        self.ctx = ctx
        self.h = h

    def launch(self) -> None:
        self.ctx.check(self.ctx._lib.q8_graph_launch(self.ctx.h, self.h))

    def destroy(self) -> None:
        if self.h:
            self.ctx._lib.q8_graph_destroy(self.h)
            self.h = None


class Buffer:
    """A device allocation (arena) owned by the library, or a wrapped view."""

    def __init__(self, ctx: Context, h, nbytes: int):
        self.ctx = ctx
        self.h = h
        self.nbytes = nbytes

    @classmethod
    def alloc(cls, ctx: Context, nbytes: int) -> "Buffer":
        h = ctypes.c_void_p()
        ctx.check(ctx._lib.q8_buf_alloc(ctx.h, int(nbytes), ctypes.byref(h)))
        return cls(ctx, h, int(nbytes))

    @classmethod
    def wrap(cls, ctx: Context, device_ptr: int, nbytes: int) -> "Buffer":
        h = ctypes.c_void_p()
        ctx.check(ctx._lib.q8_buf_wrap(ctx.h, ctypes.c_void_p(device_ptr), int(nbytes),
                                       ctypes.byref(h)))
        return cls(ctx, h, int(nbytes))

    @property
    def ptr(self) -> int:
        return self.ctx._lib.q8_buf_device_ptr(self.h) or 0

    def upload(self, arr: np.ndarray, byte_off: int = 0) -> None:
        arr = np.ascontiguousarray(arr)
        self.ctx.check(self.ctx._lib.q8_buf_upload(
            self.ctx.h, self.h, int(byte_off), arr.ctypes.data_as(ctypes.c_void_p), arr.nbytes))

    def download(self, shape, dtype, byte_off: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        self.ctx.check(self.ctx._lib.q8_buf_download(
            self.ctx.h, self.h, int(byte_off), out.ctypes.data_as(ctypes.c_void_p), out.nbytes))
        return out

    def free(self) -> None:
        if self.h:
            self.ctx._lib.q8_buf_free(self.ctx.h, self.h)
            self.h = None


# ---- Q8 entry points (thin, argument order as in include/q8hip.h) -----------

def quantize_pack(ctx: Context, src: Buffer, src_off: int, src_dtype: int, n: int, m: int,
                  dst: Buffer, dst_off_u16: int, G: int = 64, scale="f16") -> None:
    ctx.check(ctx._lib.q8_quantize_pack(ctx.h, src.h, int(src_off), int(src_dtype), int(n),
                                        int(m), dst.h, int(dst_off_u16), int(G), scale_code(scale)))


def linear(ctx: Context, w: Buffer, owt_u16: int, a: Buffer, ox_f32: int, oy_f32: int,
           s: int, m: int, n: int, G: int = 64, scale="f16") -> None:
    ctx.check(ctx._lib.q8_linear(ctx.h, w.h, int(owt_u16), a.h, int(ox_f32), int(oy_f32),
                                 int(s), int(m), int(n), int(G), scale_code(scale)))


def linear_swiglu(ctx: Context, w: Buffer, owt_u16: int, a: Buffer, og_f32: int, ou_f32: int,
                  oy_f32: int, s: int, m: int, n: int, G: int = 64, scale="f16",
                  ld: int = 0) -> None:
    """y = W (silu(g) * u) over s >= 32 rows, the swiglu folded into the
    GEMM's binary16 pre-pass: q8_linear_swiglu (ld: row stride of g and u,
    0 for m)."""
    ctx.check(ctx._lib.q8_linear_swiglu(ctx.h, w.h, int(owt_u16), a.h, int(og_f32), int(ou_f32),
                                        int(oy_f32), int(s), int(m), int(n), int(G),
                                        scale_code(scale), int(ld)))


def linear_rmsnorm(ctx: Context, w: Buffer, owt_u16: int, onorm_u16: int, eps: float, a: Buffer,
                   ox_f32: int, oy_f32: int, s: int, m: int, n: int, G: int = 64, scale="f16",
                   ores_f32: int | None = None, oh_f32: int | None = None) -> None:
    """y = W rmsnorm(x [+ res]) over s >= 32 rows, the norm (and the residual
    add, stored to oh when ores is given) folded into the GEMM's binary16
    pre-pass: q8_linear_rmsnorm."""
    has_res = ores_f32 is not None
    if has_res and oh_f32 is None:
        raise ValueError("linear_rmsnorm: a residual needs oh_f32 for x + res")
    ctx.check(ctx._lib.q8_linear_rmsnorm(ctx.h, w.h, int(owt_u16), int(onorm_u16), float(eps),
                                         a.h, int(ox_f32), int(has_res),
                                         int(ores_f32 or 0), int(oh_f32 or 0), int(oy_f32),
                                         int(s), int(m), int(n), int(G), scale_code(scale)))


PRE_NONE, PRE_RMSNORM, PRE_SWIGLU = 0, 1, 2
POST_STORE, POST_RESIDUAL, POST_SWIGLU = 0, 1, 2


def linear_fused(ctx: Context, w: Buffer, owt_u16: int, a: Buffer, ox_f32: int, oy_f32: int,
                 m: int, n: int, G: int = 64, scale="f16", pre: int = PRE_NONE,
                 onorm_u16: int = 0, eps: float = 0.0, post: int = POST_STORE,
                 ores_f32: int = 0) -> None:
    """One-row linear with rmsnorm or swiglu folded into the x load and a
    residual add or the swiglu of gate|up rows folded into the store:
    q8_linear_fused."""
    ctx.check(ctx._lib.q8_linear_fused(ctx.h, w.h, int(owt_u16), a.h, int(ox_f32), int(oy_f32),
                                       int(m), int(n), int(G), scale_code(scale), int(pre),
                                       int(onorm_u16), float(eps), int(post), int(ores_f32)))


def head_argmax(ctx: Context, w: Buffer, owt_u16: int, onorm_u16: int, eps: float, a: Buffer,
                ox_f32: int, oy_f32: int, m: int, n: int, G: int, scale, ids: Buffer,
                oid_i32: int = 0, posbuf: Buffer | None = None, opos_i32: int = 0,
                pos_step: int = 1, oemb_u16: int | None = None, onext_f32: int = 0) -> None:
    """rmsnorm + lm_head + argmax -> ids[oid] (+ position step, + the next
    token's embedding row into onext_f32 when oemb_u16 is given):
    q8_head_argmax."""
    gather = oemb_u16 is not None
    ctx.check(ctx._lib.q8_head_argmax(ctx.h, w.h, int(owt_u16), int(onorm_u16), float(eps), a.h,
                                      int(ox_f32), int(oy_f32), int(m), int(n), int(G),
                                      scale_code(scale), ids.h, int(oid_i32), _h(posbuf),
                                      int(opos_i32), int(pos_step), int(gather),
                                      int(oemb_u16) if gather else 0, int(onext_f32)))


def linear_bf16act(ctx: Context, w: Buffer, owt_u16: int, x: Buffer, ox_bf16: int, y: Buffer,
                   oy_f32: int, s: int, m: int, n: int, G: int = 64, scale="f16") -> None:
    ctx.check(ctx._lib.q8_linear_bf16act(ctx.h, w.h, int(owt_u16), x.h, int(ox_bf16), y.h,
                                         int(oy_f32), int(s), int(m), int(n), int(G),
                                         scale_code(scale)))


NOALLOC_SCRATCH_BYTES = 33554432


def linear_noalloc(hip_stream: int | None, w_ptr: int, x_ptr: int, y_ptr: int, s: int, m: int,
                   n: int, G: int = 64, scale="f16") -> None:
    """q8_linear on raw device pointers with no allocation (scratch in the
    library's fixed per-GPU array): q8_linear_noalloc.  Raises Q8Error with
    the calling thread's message on failure."""
    L = lib()
    rc = L.q8_linear_noalloc(hip_stream or None, ctypes.c_void_p(w_ptr), ctypes.c_void_p(x_ptr),
                             ctypes.c_void_p(y_ptr), int(s), int(m), int(n), int(G),
                             scale_code(scale))
    if rc != Q8_OK:
        msg = L.q8_last_error(None)
        raise Q8Error(rc, msg.decode() if isinstance(msg, bytes) else str(msg))


def embed_gather(ctx: Context, w: Buffer, oemb_u16: int, ids: Buffer, oids_i32: int, a: Buffer,
                 oy_f32: int, s: int, d: int, vocab: int, G: int = 64, scale="f16") -> None:
    ctx.check(ctx._lib.q8_embed_gather(ctx.h, w.h, int(oemb_u16), ids.h, int(oids_i32), a.h,
                                       int(oy_f32), int(s), int(d), int(vocab), int(G),
                                       scale_code(scale)))


# ---- decode-step layer kernels ---------------------------------------------------

def _h(buf):
    return None if buf is None else buf.h


def rmsnorm(ctx: Context, w: Buffer, owt_u16: int, a: Buffer, ox_f32: int, oy_f32: int,
            rows: int, d: int, eps: float) -> None:
    ctx.check(ctx._lib.q8_rmsnorm(ctx.h, w.h, int(owt_u16), a.h, int(ox_f32), int(oy_f32),
                                  int(rows), int(d), float(eps)))


def head_rmsnorm(ctx: Context, w: Buffer, owt_u16: int, a: Buffer, ox_f32: int, oy_f32: int,
                 tokens: int, heads: int, head_dim: int, ld: int = 0, eps: float = 1e-6) -> None:
    """Per-head RMSNorm of `heads` head rows in each of `tokens` rows at row
    stride ld (0: dense), y in x's layout (in place allowed): q8_head_rmsnorm."""
    ctx.check(ctx._lib.q8_head_rmsnorm(ctx.h, w.h, int(owt_u16), a.h, int(ox_f32), int(oy_f32),
                                       int(tokens), int(heads), int(head_dim), int(ld),
                                       float(eps)))


def add_rmsnorm(ctx: Context, w: Buffer, owt_u16: int, a: Buffer, ox_f32: int, oo_f32: int,
                oh_f32: int, oy_f32: int, rows: int, d: int, eps: float) -> None:
    ctx.check(ctx._lib.q8_add_rmsnorm(ctx.h, w.h, int(owt_u16), a.h, int(ox_f32), int(oo_f32),
                                      int(oh_f32), int(oy_f32), int(rows), int(d), float(eps)))


def rope_kv(ctx: Context, a: Buffer, oq: int, ok: int, ov: int, oinv: int, kv: Buffer,
            okc_f16: int, ovc_f16: int, maxlen: int, s: int, pos0: int, nheads: int, nkv: int,
            head_dim: int, posbuf: Buffer | None = None, opos_i32: int = 0,
            ld: int = 0) -> None:
    """ld: row stride of q, k and v in floats (0: each dense)."""
    ctx.check(ctx._lib.q8_rope_kv(ctx.h, a.h, int(oq), int(ok), int(ov), int(oinv), kv.h,
                                  int(okc_f16), int(ovc_f16), int(maxlen), int(s), int(pos0),
                                  _h(posbuf), int(opos_i32), int(nheads), int(nkv),
                                  int(head_dim), int(ld)))


def attention_scratch_floats(s: int, nheads: int, head_dim: int, maxlen: int) -> int:
    return int(lib().q8_attention_scratch_floats(int(s), int(nheads), int(head_dim),
                                                 int(maxlen)))


def attention(ctx: Context, a: Buffer, oq: int, kv: Buffer, okc_f16: int, ovc_f16: int,
              maxlen: int, oy: int, oscratch: int, s: int, pos0: int, nheads: int, nkv: int,
              head_dim: int, posbuf: Buffer | None = None, opos_i32: int = 0,
              ldq: int = 0) -> None:
    """ldq: row stride of q in floats (0: dense); out is dense."""
    ctx.check(ctx._lib.q8_attention(ctx.h, a.h, int(oq), kv.h, int(okc_f16), int(ovc_f16),
                                    int(maxlen), int(oy), int(oscratch), int(s), int(pos0),
                                    _h(posbuf), int(opos_i32), int(nheads), int(nkv),
                                    int(head_dim), int(ldq)))


def decode_attention(ctx: Context, a: Buffer, oq: int, ok: int, ov: int, oinv: int, kv: Buffer,
                     okc_f16: int, ovc_f16: int, maxlen: int, oy: int, pos0: int, nheads: int,
                     nkv: int, head_dim: int, posbuf: Buffer | None = None,
                     opos_i32: int = 0, wn: Buffer | None = None, oqnorm_u16: int = 0,
                     oknorm_u16: int = 0, eps: float = 0.0) -> None:
    """One-token attention step; with wn, per-head RMSNorm of q and k first
    (the q_norm / k_norm weights at oqnorm_u16 / oknorm_u16 of wn)."""
    ctx.check(ctx._lib.q8_decode_attention(ctx.h, a.h, int(oq), int(ok), int(ov), int(oinv), kv.h,
                                           int(okc_f16), int(ovc_f16), int(maxlen), int(oy),
                                           int(pos0), _h(posbuf), int(opos_i32), int(nheads),
                                           int(nkv), int(head_dim), _h(wn), int(oqnorm_u16),
                                           int(oknorm_u16), float(eps)))


def swiglu(ctx: Context, a: Buffer, og: int, ou: int, n: int) -> None:
    ctx.check(ctx._lib.q8_swiglu(ctx.h, a.h, int(og), int(ou), int(n)))


def res_add(ctx: Context, a: Buffer, ox: int, oo: int, oy: int, n: int) -> None:
    ctx.check(ctx._lib.q8_res_add(ctx.h, a.h, int(ox), int(oo), int(oy), int(n)))


def add(ctx: Context, a: Buffer, ox: int, oy: int, n: int) -> None:
    ctx.check(ctx._lib.q8_add(ctx.h, a.h, int(ox), int(oy), int(n)))


def argmax(ctx: Context, a: Buffer, ox: int, n: int, ids: Buffer, oid_i32: int) -> None:
    ctx.check(ctx._lib.q8_argmax(ctx.h, a.h, int(ox), int(n), ids.h, int(oid_i32)))


def pos_advance(ctx: Context, posbuf: Buffer, opos_i32: int, s: int) -> None:
    ctx.check(ctx._lib.q8_pos_advance(ctx.h, posbuf.h, int(opos_i32), int(s)))
