"""Packed Q8 checkpoints: safetensors reading, writing and packing.

Mirrors the reference's file side of the Q8 path:

  * SafeTensors / TensorInfo -- the multi-shard reader (src/safetensors.mojo:
    17-95) over libq8hip's C++ parser (q8_st_*): tensor name -> shard path
    and absolute byte range, dtype and shape;
  * save_file -- a safetensors writer whose output is byte-identical to the
    safetensors library's for the same tensors (q8_stw_*);
  * pack_checkpoint -- qwen3_mojo/scripts/quantize.py:46-64 (main): every
    2-D tensor packed row-wise to [scales | int8 codes] (q8_quantize_pack on
    the GPU, bit-exact with pack_q8) and stored as an "F16" tensor
    [n, m/G * ss/2 + m/2]; every other tensor converted to bf16; written
    with the same layout as save_file, so the reference layout (G = 64,
    f16 scales) gives the bytes quantize.py writes.

Other layouts (G = 32 and/or f32 scales) are recorded in the file's
__metadata__ ("q8_group", "q8_scale") so a loader can tell them apart; the
reference layout writes no metadata, as quantize.py does not.
"""

from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass
from typing import Mapping, Sequence

import numpy as np

from . import q8hip
from .q8hip import Buffer, Context, Q8Error, lib

# numpy dtype -> safetensors dtype (bf16 has no numpy dtype: pass Raw)
_NP_TO_ST = {
    np.dtype(np.float64): "F64", np.dtype(np.float32): "F32", np.dtype(np.float16): "F16",
    np.dtype(np.int64): "I64", np.dtype(np.int32): "I32", np.dtype(np.int16): "I16",
    np.dtype(np.int8): "I8", np.dtype(np.uint64): "U64", np.dtype(np.uint32): "U32",
    np.dtype(np.uint16): "U16", np.dtype(np.uint8): "U8", np.dtype(np.bool_): "BOOL",
}
# safetensors dtype -> numpy dtype that holds its bytes
_ST_TO_NP = {"F64": np.float64, "F32": np.float32, "F16": np.float16, "BF16": np.uint16,
             "I64": np.int64, "I32": np.int32, "I16": np.int16, "I8": np.int8,
             "U64": np.uint64, "U32": np.uint32, "U16": np.uint16, "U8": np.uint8,
             "BOOL": np.bool_, "F8_E4M3": np.uint8, "F8_E5M2": np.uint8}

QUANT_GROUP_KEY, QUANT_SCALE_KEY = "q8_group", "q8_scale"


def _check_st(rc: int) -> None:
    if rc != q8hip.Q8_OK:
        raise Q8Error(rc, lib().q8_st_error().decode())


@dataclass
class TensorInfo:
    """One tensor of a safetensors model (src/safetensors.mojo:17-33)."""
    name: str
    dtype: str
    shape: list
    path: str      # shard file holding it
    begin: int     # absolute byte offset in that shard
    end: int

    def numel(self) -> int:
        return int(np.prod(self.shape, dtype=np.int64)) if self.shape else 1

    def nbytes(self) -> int:
        return self.end - self.begin


@dataclass
class Raw:
    """A tensor given as raw element bytes with an explicit safetensors dtype
    (for BF16, which numpy lacks: the u16 bit patterns)."""
    dtype: str
    data: np.ndarray


class SafeTensors:
    """A safetensors model: a file, or a directory with
    model.safetensors.index.json or model.safetensors (SafeTensors,
    src/safetensors.mojo:36-95).  infos lists the tensors shard by shard in
    header order."""

    def __init__(self, path: str):
        self._lib = lib()
        h = ctypes.c_void_p()
        _check_st(self._lib.q8_st_open(os.fsencode(path), ctypes.byref(h)))
        self.h = h
        self.infos: list[TensorInfo] = []
        for i in range(int(self._lib.q8_st_count(h))):
            name, dtype, spath = ctypes.c_char_p(), ctypes.c_char_p(), ctypes.c_char_p()
            ndim = ctypes.c_int()
            shape = ctypes.POINTER(ctypes.c_int64)()
            begin, nbytes = ctypes.c_uint64(), ctypes.c_uint64()
            _check_st(self._lib.q8_st_info(h, i, ctypes.byref(name), ctypes.byref(dtype),
                                           ctypes.byref(ndim), ctypes.byref(shape),
                                           ctypes.byref(spath), ctypes.byref(begin),
                                           ctypes.byref(nbytes)))
            self.infos.append(TensorInfo(name.value.decode(), dtype.value.decode(),
                                         [int(shape[d]) for d in range(ndim.value)],
                                         spath.value.decode(), int(begin.value),
                                         int(begin.value) + int(nbytes.value)))
        self.index = {t.name: i for i, t in enumerate(self.infos)}
        self.metadata = {}
        for i in range(int(self._lib.q8_st_metadata_count(h))):
            k, v = ctypes.c_char_p(), ctypes.c_char_p()
            _check_st(self._lib.q8_st_metadata(h, i, ctypes.byref(k), ctypes.byref(v)))
            self.metadata[k.value.decode()] = v.value.decode()

    def num_tensors(self) -> int:
        return len(self.infos)

    def has(self, name: str) -> bool:
        return name in self.index

    def get(self, name: str) -> TensorInfo:
        if name not in self.index:
            raise KeyError(name)
        return self.infos[self.index[name]]

    def read(self, name: str) -> np.ndarray:
        """The tensor's bytes as a numpy array of its shape (BF16 and F8 as
        their unsigned-integer bit patterns)."""
        t = self.get(name)
        out = np.empty(t.shape, dtype=_ST_TO_NP[t.dtype])
        _check_st(self._lib.q8_st_read(self.h, self.index[name], 0,
                                       out.ctypes.data_as(ctypes.c_void_p), out.nbytes))
        return out

    def upload(self, ctx: Context, name: str, buf: Buffer, byte_off: int) -> int:
        """Copy the tensor's bytes straight from the file to byte offset
        byte_off of a device buffer; returns the byte count."""
        t = self.get(name)
        ctx.check(self._lib.q8_st_upload(ctx.h, self.h, self.index[name], 0, t.nbytes(),
                                         buf.h, int(byte_off)))
        return t.nbytes()

    def close(self) -> None:
        if getattr(self, "h", None):
            self._lib.q8_st_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _spec(value) -> tuple[str, np.ndarray]:
    if isinstance(value, Raw):
        return value.dtype, np.ascontiguousarray(value.data)
    arr = np.ascontiguousarray(value)
    if arr.dtype not in _NP_TO_ST:
        raise ValueError(f"no safetensors dtype for numpy {arr.dtype}")
    return _NP_TO_ST[arr.dtype], arr


class Writer:
    """A safetensors file whose header is fixed at open: put() each tensor
    (any order), then close()."""

    def __init__(self, path: str, specs: Sequence[tuple[str, str, Sequence[int]]],
                 metadata: Mapping[str, str] | None = None):
        self._lib = lib()
        n = len(specs)
        names = (ctypes.c_char_p * n)(*[s[0].encode() for s in specs])
        dtypes = (ctypes.c_char_p * n)(*[s[1].encode() for s in specs])
        ndims = (ctypes.c_int * n)(*[len(s[2]) for s in specs])
        flat = [int(d) for s in specs for d in s[2]]
        shapes = (ctypes.c_int64 * max(1, len(flat)))(*flat)
        meta = list((metadata or {}).items())
        keys = (ctypes.c_char_p * max(1, len(meta)))(*[k.encode() for k, _ in meta])
        vals = (ctypes.c_char_p * max(1, len(meta)))(*[v.encode() for _, v in meta])
        h = ctypes.c_void_p()
        _check_st(self._lib.q8_stw_open(os.fsencode(path), n, names, dtypes, ndims, shapes,
                                        len(meta), keys, vals, ctypes.byref(h)))
        self.h = h
        self.index = {s[0]: i for i, s in enumerate(specs)}

    def put(self, name: str, data: np.ndarray) -> None:
        data = np.ascontiguousarray(data)
        _check_st(self._lib.q8_stw_put(self.h, self.index[name],
                                       data.ctypes.data_as(ctypes.c_void_p), data.nbytes))

    def close(self) -> None:
        if self.h:
            h, self.h = self.h, None
            _check_st(self._lib.q8_stw_close(h))


def save_file(tensors: Mapping[str, object], path: str,
              metadata: Mapping[str, str] | None = None) -> None:
    """Write tensors (numpy arrays, or Raw for BF16) as a safetensors file
    laid out byte for byte as the safetensors library writes it."""
    specs, datas = [], {}
    for name, value in tensors.items():
        dt, arr = _spec(value)
        specs.append((name, dt, list(arr.shape)))
        datas[name] = arr
    w = Writer(path, specs, metadata)
    try:
        for name, arr in datas.items():
            w.put(name, arr)
    finally:
        w.close()


def _to_bf16_bits(t: TensorInfo, raw: np.ndarray) -> np.ndarray:
    """A 1-D (or any non-2-D) tensor as bf16 bit patterns (torch .to(bfloat16):
    round to nearest even)."""
    if t.dtype == "BF16":
        return raw.view(np.uint16)
    if t.dtype in ("F32", "F16", "F64"):
        f = raw.astype(np.float32)
        b = f.view(np.uint32).astype(np.uint64)
        nan = np.isnan(f)
        r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
        r[nan] = 0x7FC0                                      # torch's NaN
        return r
    raise ValueError(f"{t.name}: dtype {t.dtype} cannot be converted to bf16")


def pack_checkpoint(ctx: Context, src: str, out_path: str, G: int = 64, scale: str = "f16",
                    names: Sequence[str] | None = None) -> dict:
    """quantize.py's main (qwen3_mojo/scripts/quantize.py:46-64) on the GPU:
    read the model at `src`, pack every 2-D tensor (bf16, f16 or f32 source;
    m % G == 0) with q8_quantize_pack, convert the rest to bf16, and write
    out_path.  Returns {"raw_bytes", "q8_bytes"} as quantize.py prints."""
    st = SafeTensors(src)
    try:
        infos = [st.get(n) for n in names] if names is not None else list(st.infos)
        specs = []
        for t in infos:
            if len(t.shape) == 2:
                n, m = t.shape
                if m % G:
                    raise ValueError(f"{t.name}: m={m} is not a multiple of G={G}")
                specs.append((t.name, "F16", [n, q8hip.rowstride_u16(m, G, scale)]))
            else:
                specs.append((t.name, "BF16", list(t.shape)))
        meta = None if (G, scale) == (64, "f16") else {QUANT_GROUP_KEY: str(G),
                                                         QUANT_SCALE_KEY: scale}
        w = Writer(out_path, specs, meta)
        raw_bytes = q_bytes = 0
        try:
            for t, spec in zip(infos, specs):
                raw_bytes += t.numel() * 2
                if len(t.shape) != 2:
                    bits = _to_bf16_bits(t, st.read(t.name))
                    w.put(t.name, bits)
                    q_bytes += bits.nbytes
                    continue
                n, m = t.shape
                rs = spec[2][1]
                if t.dtype in ("BF16", "F32"):
                    src_buf = Buffer.alloc(ctx, t.nbytes())
                    st.upload(ctx, t.name, src_buf, 0)
                    kind = q8hip.Q8_SRC_BF16 if t.dtype == "BF16" else q8hip.Q8_SRC_F32
                elif t.dtype == "F16":
                    # w.float() of an f16 tensor is exact: pack its f32 values
                    f = st.read(t.name).astype(np.float32)
                    src_buf = Buffer.alloc(ctx, f.nbytes)
                    src_buf.upload(f)
                    kind = q8hip.Q8_SRC_F32
                else:
                    raise ValueError(f"{t.name}: cannot pack dtype {t.dtype}")
                dst = Buffer.alloc(ctx, 2 * n * rs)
                try:
                    q8hip.quantize_pack(ctx, src_buf, 0, kind, n, m, dst, 0, G, scale)
                    packed = dst.download((n, rs), np.uint16)
                finally:
                    src_buf.free()
                    dst.free()
                w.put(t.name, packed)
                q_bytes += packed.nbytes
        finally:
            w.close()
        return {"raw_bytes": raw_bytes, "q8_bytes": q_bytes}
    finally:
        st.close()


def checkpoint_layout(st: SafeTensors) -> tuple[int, str]:
    """(G, scale) of a packed file: the metadata written by pack_checkpoint,
    else the reference layout (64, "f16")."""
    g = int(st.metadata.get(QUANT_GROUP_KEY, "64"))
    sc = st.metadata.get(QUANT_SCALE_KEY, "f16")
    return g, sc


def main(argv: Sequence[str] | None = None) -> int:
    """python -m lama32_mojo_amd.checkpoint SRC OUT [--group 64] [--scale f16]

    quantize.py's command (qwen3_mojo/scripts/quantize.py:46-64): pack the
    bf16 model at SRC (file, or directory with shards) into OUT on GPU 0."""
    import argparse

    p = argparse.ArgumentParser(description="pack a safetensors model to Q8 rows")
    p.add_argument("src")
    p.add_argument("out")
    p.add_argument("--group", type=int, default=64, choices=[32, 64])
    p.add_argument("--scale", default="f16", choices=["f16", "f32"])
    p.add_argument("--device", type=int, default=0)
    a = p.parse_args(argv)
    ctx = Context(a.device)
    try:
        sizes = pack_checkpoint(ctx, a.src, a.out, a.group, a.scale)
    finally:
        ctx.close()
    print(f"wrote {a.out}")
    print(f"bf16 {sizes['raw_bytes'] / 1e9:.2f} GB -> q8 {sizes['q8_bytes'] / 1e9:.2f} GB "
          f"({sizes['raw_bytes'] / max(1, sizes['q8_bytes']):.2f}x)")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
