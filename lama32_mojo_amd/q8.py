"""Host-side mirror of the reference's Q8 linear-layer interface, on libq8hip.

The names, argument meaning and error behaviour follow the reference so a
caller of its Q8 path finds the same API:

  QG, PAD, q8_rowstride       src/llama_q8.mojo:23,26-28; src/llama_common.mojo:22
  Weights (u16 arena)         src/resident.mojo:15-58
  Acts (f32 bump arena)       src/llama_common.mojo:578-606
  Q8Kernels                   src/llama_q8.mojo:115-121
  mm_q8_op                    src/llama_q8.mojo:124-141
  embed_q8                    qwen3_mojo/src/qwen_q8.mojo:110-124 (k_embed_gather_q8)
  pack_q8                     qwen3_mojo/scripts/quantize.py:31-43 (runs on the GPU)

Every compute call goes through the C ABI (libq8hip.so); nothing here falls
back to the CPU.
"""

from __future__ import annotations

from typing import Mapping, Sequence

import numpy as np

from . import q8hip
from .q8hip import Buffer, Context

QG = 64                  # quantization group (src/llama_q8.mojo:23)
PAD = 32                 # reserved head elements per arena (src/llama_common.mojo:22)
BLOCK = 256              # (src/llama_common.mojo:19)
TG_MM = 32               # (src/llama_common.mojo:21)
MM_CHUNK_MACS = 1 << 30  # (src/llama_common.mojo:23)


def q8_rowstride(m: int, G: int = QG, scale: str = "f16") -> int:
    """Packed row length in u16 elements: m/G scales + m/2 byte pairs."""
    return q8hip.rowstride_u16(m, G, scale)


class Weights:
    """u16 weight arena: PAD head, then tensors contiguous in `names` order.

    upload_all copies every tensor into one host staging array and uploads it
    with a single copy (the reference's single map_to_host, resident.mojo:30-58).
    Tensors are given as arrays whose raw bytes are the stored values (u16
    bit patterns of packed Q8 rows or bf16 norms)."""

    def __init__(self, ctx: Context, cap: int):
        self.ctx = ctx
        self.buf = Buffer.alloc(ctx, 2 * int(cap))
        self.offs: dict[str, int] = {}
        self.top = PAD
        self.cap = int(cap)

    def o(self, name: str) -> int:
        return self.offs[name]

    def upload_all(self, tensors: Mapping[str, np.ndarray], names: Sequence[str]) -> None:
        host = np.zeros(self.cap, dtype=np.uint16)
        top = self.top
        offs = {}
        for name in names:
            t = np.ascontiguousarray(tensors[name])
            count = t.nbytes // 2
            if top + count > self.cap:
                raise RuntimeError("weight arena overflow at " + name)
            host[top:top + count] = t.reshape(-1).view(np.uint16)
            offs[name] = top
            top += count
        self.buf.upload(host[: top])
        self.offs.update(offs)
        self.top = top

    def upload_file(self, st, names: Sequence[str]) -> None:
        """Tensors straight from a safetensors model (checkpoint.SafeTensors)
        into the arena, in `names` order, each copied file -> device through
        pinned staging (resident.mojo:30-58 reads each tensor's byte range
        and copies it into the mapped arena)."""
        top = self.top
        for name in names:
            if not st.has(name):
                raise KeyError(f"{name} is not in the checkpoint")
            info = st.get(name)
            if info.dtype not in ("F16", "BF16", "U16", "I16"):
                raise ValueError(f"{name}: dtype {info.dtype} is not 2 bytes per element")
            count = info.nbytes() // 2
            if top + count > self.cap:
                raise RuntimeError("weight arena overflow at " + name)
            st.upload(self.ctx, name, self.buf, 2 * top)
            self.offs[name] = top
            top += count
        self.top = top


class Acts:
    """f32 activation arena with bump allocation and a resettable mark."""

    def __init__(self, ctx: Context, cap: int):
        self.ctx = ctx
        self.buf = Buffer.alloc(ctx, 4 * int(cap))
        self.top = PAD
        self.cap = int(cap)

    def alloc(self, n: int) -> int:
        off = self.top
        self.top += int(n)
        if self.top > self.cap:
            raise RuntimeError("acts arena overflow")
        return off

    def align(self, k: int) -> None:
        """Round the next allocation's offset up to a multiple of k floats."""
        self.top = (self.top + k - 1) // k * k
        if self.top > self.cap:
            raise RuntimeError("acts arena overflow")

    def mark(self) -> int:
        return self.top

    def reset(self, m: int) -> None:
        self.top = m

    def write(self, off: int, values: np.ndarray) -> None:
        self.buf.upload(np.ascontiguousarray(values, dtype=np.float32), 4 * int(off))

    def read(self, off: int, count: int) -> np.ndarray:
        return self.buf.download((int(count),), np.float32, 4 * int(off))


class Q8Kernels:
    """The reference compiles its two Q8 kernels once per process; here they
    are compiled ahead of time into libq8hip.so, so this only records the
    layout the caller's packed weights use."""

    def __init__(self, ctx: Context, G: int = QG, scale: str = "f16"):
        self.ctx = ctx
        self.G = G
        self.scale = scale


def mm_q8_op(ctx: Context, w: Weights, a: Acts, qk: Q8Kernels, ox: int, s: int, m: int,
             owt: int, n: int) -> int:
    """y (s, n) = x (s, m) @ Wq8 (n, m)^T; returns y's f32 offset in `a`.

    Same contract as the reference host op: allocate y from the activation
    arena, enqueue, return the offset.  One launch replaces the reference's
    watchdog chunking."""
    oy = a.alloc(s * n)
    q8hip.linear(ctx, w.buf, owt, a.buf, ox, oy, s, m, n, qk.G, qk.scale)
    return oy


def embed_q8(ctx: Context, w: Weights, a: Acts, qk: Q8Kernels, oemb: int, ids: Sequence[int],
             d: int, vocab: int, idbuf: Buffer | None = None) -> int:
    """Gather embedding rows for `ids` from the packed table at `oemb`;
    returns the f32 offset of the (s, d) result (QwenQ8.embed)."""
    s = len(ids)
    ox = a.alloc(s * d)
    own = idbuf is None
    if own:
        idbuf = Buffer.alloc(ctx, 4 * max(s, 1))
    idbuf.upload(np.asarray(ids, dtype=np.int32))
    q8hip.embed_gather(ctx, w.buf, oemb, idbuf, 0, a.buf, ox, s, d, vocab, qk.G, qk.scale)
    if own:
        ctx.sync()
        idbuf.free()
    return ox


_DEFAULT_CTX: Context | None = None


def default_context() -> Context:
    global _DEFAULT_CTX
    if _DEFAULT_CTX is None:
        _DEFAULT_CTX = Context(0)
    return _DEFAULT_CTX


def pack_q8_bits(wbits: np.ndarray, G: int = QG, scale: str = "f16",
                 ctx: Context | None = None, src_dtype: str = "bf16") -> np.ndarray:
    """GPU quantize+pack of host weights; returns packed u16 rows [n, rowstride].

    wbits: bf16 bit patterns (uint16 [n, m]) or, with src_dtype="f32",
    float32 [n, m]."""
    ctx = ctx or default_context()
    w = np.ascontiguousarray(wbits)
    n, m = w.shape
    rs = q8_rowstride(m, G, scale)
    src = Buffer.alloc(ctx, max(w.nbytes, 1))
    dst = Buffer.alloc(ctx, max(2 * n * rs, 1))
    try:
        src.upload(w)
        sd = q8hip.Q8_SRC_F32 if src_dtype == "f32" else q8hip.Q8_SRC_BF16
        q8hip.quantize_pack(ctx, src, 0, sd, n, m, dst, 0, G, scale)
        out = dst.download((n, rs), np.uint16)
    finally:
        src.free()
        dst.free()
    return out


def pack_q8(w, G: int = QG, scale: str = "f16", ctx: Context | None = None):
    """pack_q8 with the reference's signature: bf16 torch tensor [n, m] ->
    float16 tensor [n, m/G + m/2] holding the packed rows (quantize.py:31-43).
    Quantization runs on the GPU; codes and scales are bit-identical."""
    import torch

    assert w.dim() == 2 and w.dtype == torch.bfloat16, (w.shape, w.dtype)
    bits = w.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
    packed = pack_q8_bits(bits, G, scale, ctx)
    return torch.from_numpy(packed.view(np.float16)).to(w.device)
