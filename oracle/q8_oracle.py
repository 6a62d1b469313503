"""CPU oracle for the INT8 group-quantized (W8A32) linear-layer path.

TEST INFRASTRUCTURE ONLY.  This module is the checker.  It may be imported by
tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline leg, and by
nothing else; the product path (lama32_mojo_amd, libq8hip.so) never imports,
loads or calls it.

Two independent restatements live here:

* ``pack_q8_np`` -- numpy restatement of ``pack_q8``
  (qwen3_mojo/scripts/quantize.py:31-43), using the same numpy dtype rules
  (f32 arithmetic, NEP 50 weak python scalars, ``astype(float16)`` RNE with
  subnormals, ``rint`` half-to-even, ``clip``, float->int8 cast).
* ``COracle`` -- ctypes binding of ``oracle/libq8oracle.so`` built from
  ``oracle/q8_oracle.c`` (plain C; own f16 conversion, pack, float64 closed
  form and group-major fp32 linear, embedding gather).

Layout modes: ``(G, scale)`` = ``(64, "f16")`` is the reference layout
(quantize.py:28,37; src/llama_q8.mojo:23-28); ``(32, "f32")`` is the same
algorithm with group 32 and the scale kept in f32 (no f16 rounding).
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

SCALE_F16 = 1
SCALE_F32 = 2
_SCALE_KIND = {"f16": SCALE_F16, "f32": SCALE_F32}

_HERE = os.path.dirname(os.path.abspath(__file__))
C_LIB_PATH = os.path.join(_HERE, "libq8oracle.so")


def scale_kind(scale: str | int) -> int:
    if isinstance(scale, int):
        return scale
    return _SCALE_KIND[scale]


def rowstride_u16(m: int, G: int = 64, scale: str | int = "f16") -> int:
    """Packed row length in u16 elements (src/llama_q8.mojo:26-28)."""
    su = 2 if scale_kind(scale) == SCALE_F32 else 1
    return (m // G) * su + m // 2


# --------------------------------------------------------------------------
# numpy restatement
# --------------------------------------------------------------------------

def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) -> float32, exact (quantize.py:34 w.float())."""
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns, round to nearest even (no NaN inputs)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = u + 0x7FFF + ((u >> 16) & 1)
    return (u >> 16).astype(np.uint16)


def pack_q8_np(w: np.ndarray, G: int = 64, scale: str = "f16") -> np.ndarray:
    """Pack f32 weights [n, m] into uint16 rows [n, rowstride_u16(m)].

    Restates quantize.py:31-43 step by step:
      :36  scale = max|w_g| / 127                  (f32)
      :37  scale = max(scale, 1e-8) -> float16     (f32 compare, RNE to f16)
      :38  q = rint(w / f32(scale16))               (f32 divide, half-to-even)
      :39  q = clip(q, -127, 127).astype(int8)      (NaN -> 0)
      :41  row = [scale bits | int8 bytes] viewed as little-endian u16
    For scale == "f32" the f16 rounding at :37 is skipped and each scale takes
    two u16 elements (little-endian f32).
    """
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, m = w.shape
    assert m % G == 0 and m % 2 == 0, (n, m, G)
    x = w.reshape(n, m // G, G)
    # scales past binary16's range round to inf, as the reference's cast does
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        s = np.abs(x).max(axis=2) / 127.0
        s = np.maximum(s, 1e-8)
        if scale == "f16":
            s = s.astype(np.float16)
            sf = s.astype(np.float32)
            sbits = s.view(np.uint16)
        elif scale == "f32":
            s = s.astype(np.float32)
            sf = s
            sbits = s.view(np.uint16).reshape(n, -1)
        else:
            raise ValueError(scale)
        q = np.rint(x / sf[:, :, None])
        q = np.clip(q, -127, 127)
        q = np.where(np.isnan(q), 0, q).astype(np.int8).reshape(n, m)
    return np.concatenate([sbits.reshape(n, -1), q.view(np.uint16)], axis=1)


def unpack_q8_np(packed: np.ndarray, m: int, G: int = 64, scale: str = "f16"):
    """Split packed rows into (codes int8 [n, m], scales f32 [n, m/G])."""
    packed = np.ascontiguousarray(packed, dtype=np.uint16)
    n = packed.shape[0]
    ng = m // G
    if scale == "f16":
        s = packed[:, :ng].view(np.float16).astype(np.float32)
        codes = packed[:, ng:].view(np.int8)
    else:
        s = packed[:, : 2 * ng].copy().view(np.float32)
        codes = packed[:, 2 * ng:].view(np.int8)
    return codes.reshape(n, m), s.reshape(n, ng)


def linear_f64_np(packed, x, m, G=64, scale="f16"):
    """float64 closed form y = x . deq(W)^T via an explicit dequantisation.

    Independent of the C closed form: dequantise every weight to float64
    (q * s, exact), then one float64 matmul (gen_oracle.py's ``x @ W.T``
    form, scripts/gen_oracle.py:76-95)."""
    codes, s = unpack_q8_np(packed, m, G, scale)
    wd = codes.astype(np.float64) * np.repeat(s.astype(np.float64), G, axis=1)
    return np.asarray(x, dtype=np.float64) @ wd.T


def embed_gather_np(packed, ids, d, G=64, scale="f16"):
    """y[i, c] = f32(q[id_i, c]) * f32(s[id_i, c // G]) (src/llama_q8.mojo:96-109)."""
    codes, s = unpack_q8_np(packed, d, G, scale)
    ids = np.asarray(ids, dtype=np.int64)
    return codes[ids].astype(np.float32) * np.repeat(s[ids], G, axis=1)


def max_rel_err(y, y_ref) -> float:
    """Normwise max relative error  max|y - y*| / max|y*|  (0 when both are 0)."""
    y = np.asarray(y, dtype=np.float64)
    y_ref = np.asarray(y_ref, dtype=np.float64)
    den = np.max(np.abs(y_ref)) if y_ref.size else 0.0
    num = np.max(np.abs(y - y_ref)) if y_ref.size else 0.0
    if den == 0.0:
        return float(num)
    return float(num / den)


def abs_packed(packed, m: int, G: int = 64, scale: str = "f16") -> np.ndarray:
    """Packed rows of |W|: every scale's sign bit cleared and every code
    replaced by its magnitude (codes lie in [-127, 127]), so the linear over
    them is sum_k |x_k| |w_jk| when given |x|."""
    out = np.array(packed, dtype=np.uint16, copy=True)
    ng = m // G
    if scale == "f16":
        out[:, :ng] &= np.uint16(0x7FFF)
        codes = out[:, ng:].view(np.int8)
    else:
        out[:, 1:2 * ng:2] &= np.uint16(0x7FFF)     # high halves of the f32 scales
        codes = out[:, 2 * ng:].view(np.int8)
    np.abs(codes, out=codes)
    return out


def elementwise_err(y, y_ref, y_abs) -> float:
    """Elementwise relative error max_i |y_i - y*_i| / a_i, where a_i =
    sum_k |x_k| |w_ik| is output i's own scale: the standard componentwise
    bound of a dot product, so the bar holds for every output, those that
    cancel to near zero included (0 where a_i is 0 and y_i equals y*_i)."""
    y = np.asarray(y, dtype=np.float64)
    y_ref = np.asarray(y_ref, dtype=np.float64)
    a = np.asarray(y_abs, dtype=np.float64)
    d = np.abs(y - y_ref)
    if d.size == 0:
        return 0.0
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.where(d == 0.0, 0.0, d / a)
    return float(np.max(r))


# --------------------------------------------------------------------------
# C restatement (ctypes)
# --------------------------------------------------------------------------

class COracle:
    """ctypes binding of oracle/libq8oracle.so (build with ``make -C oracle``)."""

    def __init__(self, path: str = C_LIB_PATH):
        if not os.path.exists(path):
            raise FileNotFoundError(
                f"{path} is missing; build it with `make -C oracle`")
        lib = ctypes.CDLL(path)
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        I = ctypes.c_int
        lib.q8o_f32_to_f16.argtypes = [ctypes.c_float]
        lib.q8o_f32_to_f16.restype = ctypes.c_uint16
        lib.q8o_f16_to_f32.argtypes = [ctypes.c_uint16]
        lib.q8o_f16_to_f32.restype = ctypes.c_float
        lib.q8o_rowstride_u16.argtypes = [I64, I, I]
        lib.q8o_rowstride_u16.restype = I64
        lib.q8o_pack_f32.argtypes = [P, I64, I64, I, I, P]
        lib.q8o_pack_f32.restype = I
        lib.q8o_pack_bf16.argtypes = [P, I64, I64, I, I, P]
        lib.q8o_pack_bf16.restype = I
        lib.q8o_linear_f64.argtypes = [P, P, I64, I64, I64, I, I, P]
        lib.q8o_linear_f64.restype = None
        lib.q8o_linear_f64x.argtypes = [P, P, I64, I64, I64, I, I, P]
        lib.q8o_linear_f64x.restype = None
        lib.q8o_linear_f32.argtypes = [P, P, I64, I64, I64, I, I, P]
        lib.q8o_linear_f32.restype = None
        lib.q8o_embed_gather.argtypes = [P, P, I64, I64, I, I, P]
        lib.q8o_embed_gather.restype = None
        lib.q8o_f32_to_f16_array.argtypes = [P, I64, P]
        lib.q8o_f32_to_f16_array.restype = None
        lib.q8o_f16_to_f32_array.argtypes = [P, I64, P]
        lib.q8o_f16_to_f32_array.restype = None
        lib.q8o_set_threads.argtypes = [I]
        lib.q8o_set_threads.restype = None
        lib.q8o_get_threads.argtypes = []
        lib.q8o_get_threads.restype = I
        self.lib = lib

    def set_threads(self, n: int) -> None:
        """OpenMP threads of the parallel loops (linear_f32, linear_f64)."""
        self.lib.q8o_set_threads(int(n))

    def threads(self) -> int:
        return int(self.lib.q8o_get_threads())

    @staticmethod
    def _p(a: np.ndarray):
        return a.ctypes.data_as(ctypes.c_void_p)

    def f32_to_f16(self, f: float) -> int:
        return int(self.lib.q8o_f32_to_f16(float(f)))

    def f32_to_f16_array(self, x) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(x.shape, dtype=np.uint16)
        self.lib.q8o_f32_to_f16_array(self._p(x), x.size, self._p(out))
        return out

    def f16_to_f32_array(self, h) -> np.ndarray:
        h = np.ascontiguousarray(h, dtype=np.uint16)
        out = np.empty(h.shape, dtype=np.float32)
        self.lib.q8o_f16_to_f32_array(self._p(h), h.size, self._p(out))
        return out

    def pack_f32(self, w, G=64, scale="f16") -> np.ndarray:
        w = np.ascontiguousarray(w, dtype=np.float32)
        n, m = w.shape
        out = np.empty((n, rowstride_u16(m, G, scale)), dtype=np.uint16)
        rc = self.lib.q8o_pack_f32(self._p(w), n, m, G, scale_kind(scale), self._p(out))
        if rc != 0:
            raise ValueError(f"pack_f32 rejected shape {(n, m)} G={G}")
        return out

    def pack_bf16(self, wbits, G=64, scale="f16") -> np.ndarray:
        wbits = np.ascontiguousarray(wbits, dtype=np.uint16)
        n, m = wbits.shape
        out = np.empty((n, rowstride_u16(m, G, scale)), dtype=np.uint16)
        rc = self.lib.q8o_pack_bf16(self._p(wbits), n, m, G, scale_kind(scale), self._p(out))
        if rc != 0:
            raise ValueError(f"pack_bf16 rejected shape {(n, m)} G={G}")
        return out

    def linear_f64(self, packed, x, G=64, scale="f16") -> np.ndarray:
        packed = np.ascontiguousarray(packed, dtype=np.uint16)
        x = np.ascontiguousarray(x, dtype=np.float32)
        s, m = x.shape
        n = packed.shape[0]
        assert packed.shape[1] == rowstride_u16(m, G, scale)
        y = np.empty((s, n), dtype=np.float64)
        self.lib.q8o_linear_f64(self._p(packed), self._p(x), s, m, n, G,
                                scale_kind(scale), self._p(y))
        return y

    def linear_f64x(self, packed, x, G=64, scale="f16") -> np.ndarray:
        """float64 closed form for float64 activations x [s, m]."""
        packed = np.ascontiguousarray(packed, dtype=np.uint16)
        x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float64)
        s, m = x.shape
        n = packed.shape[0]
        assert packed.shape[1] == rowstride_u16(m, G, scale)
        y = np.empty((s, n), dtype=np.float64)
        self.lib.q8o_linear_f64x(self._p(packed), self._p(x), s, m, n, G,
                                 scale_kind(scale), self._p(y))
        return y

    def linear_abs(self, packed, x, G=64, scale="f16") -> np.ndarray:
        """sum_k |x_ik| |w_jk| in float64: each output's scale for
        elementwise_err."""
        x = np.abs(np.atleast_2d(np.asarray(x, dtype=np.float64)))
        return self.linear_f64x(abs_packed(packed, x.shape[1], G, scale), x, G, scale)

    def linear_f32(self, packed, x, G=64, scale="f16") -> np.ndarray:
        packed = np.ascontiguousarray(packed, dtype=np.uint16)
        x = np.ascontiguousarray(x, dtype=np.float32)
        s, m = x.shape
        n = packed.shape[0]
        assert packed.shape[1] == rowstride_u16(m, G, scale)
        y = np.empty((s, n), dtype=np.float32)
        self.lib.q8o_linear_f32(self._p(packed), self._p(x), s, m, n, G,
                                scale_kind(scale), self._p(y))
        return y

    def embed_gather(self, packed, ids, d, G=64, scale="f16") -> np.ndarray:
        packed = np.ascontiguousarray(packed, dtype=np.uint16)
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        y = np.empty((ids.shape[0], d), dtype=np.float32)
        self.lib.q8o_embed_gather(self._p(packed), self._p(ids), ids.shape[0], d,
                                  G, scale_kind(scale), self._p(y))
        return y


_COR = None


def c_oracle() -> COracle:
    """Process-wide COracle instance."""
    global _COR
    if _COR is None:
        _COR = COracle()
    return _COR


def synth_weights_bf16(n: int, m: int, seed: int, std: float = 0.02) -> np.ndarray:
    """Synthetic weights: N(0, std) f32 rounded to bf16 (the reference's
    input domain, quantize.py:34).  Returns bf16 bit patterns [n, m]."""
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, m), dtype=np.float32) * np.float32(std))
    return f32_to_bf16_bits(w)


def synth_x(s: int, m: int, seed: int) -> np.ndarray:
    """Synthetic activations x ~ N(0, 1), float32 [s, m]."""
    rng = np.random.default_rng(seed)
    return rng.standard_normal((s, m), dtype=np.float32)
