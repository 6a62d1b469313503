"""C ABI of libq8hip.so on the CPU: it loads, exports every symbol the header
declares, and validates every argument before touching a device (a host-only
context, Q8_DEVICE_NONE, returns Q8_ERR_NODEVICE only once the arguments are
valid)."""

import os
import re

import numpy as np
import pytest

from lama32_mojo_amd import q8, q8hip
from lama32_mojo_amd.q8hip import (Q8_ERR_ARG, Q8_ERR_NODEVICE, Q8_ERR_RANGE, Q8_ERR_SHAPE,
                                   Q8_SRC_BF16, Q8_SRC_F32, Q8Error)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "q8hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(q8_\w+)\s*\(", text)))


def test_header_symbols_exported():
    lib = q8hip.lib()
    names = declared_functions()
    assert len(names) >= 20
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(q8hip.SIGNATURES), set(names) ^ set(q8hip.SIGNATURES)


def test_only_the_c_abi_is_exported():
    """The dynamic symbol table holds the q8_* entry points and no internal
    launcher or helper (the link's version script)."""
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", q8hip.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    names = [line.split()[-1] for line in out.splitlines() if line.strip()]
    names = [n for n in names if not n.startswith("q8_")]
    assert names == [], names[:10]


def test_version_and_rowstride():
    lib = q8hip.lib()
    assert lib.q8_version() == 100
    assert q8hip.rowstride_u16(2048) == 1056          # src/llama_q8.mojo:26-28
    assert q8hip.rowstride_u16(14336) == 7392
    assert q8hip.rowstride_u16(2048, 32, "f32") == 1152
    assert lib.q8_rowstride_u16(100, 64, 1) == 0
    assert lib.q8_rowstride_u16(2048, 48, 1) == 0
    assert lib.q8_rowstride_u16(2048, 64, 3) == 0


@pytest.fixture
def hctx():
    c = q8hip.Context(q8hip.Q8_DEVICE_NONE)
    yield c
    c.close()


def code_of(fn, *args, **kw):
    try:
        fn(*args, **kw)
    except Q8Error as e:
        return e.code, e.msg
    return 0, ""


def test_linear_validation(hctx):
    rs = q8hip.rowstride_u16(2048)
    w = hctx.alloc(2 * (8 + 16 * rs))
    a = hctx.alloc(4 * 10000)
    L = q8hip.linear
    # valid -> reaches the device step
    assert code_of(L, hctx, w, 8, a, 0, 4096, 2, 2048, 16)[0] == Q8_ERR_NODEVICE
    # m not a multiple of G
    c, msg = code_of(L, hctx, w, 8, a, 0, 4096, 2, 2000, 16)
    assert c == Q8_ERR_SHAPE and "multiple of G" in msg
    # unsupported group size / scale dtype
    assert code_of(L, hctx, w, 8, a, 0, 4096, 2, 2048, 16, G=48)[0] == Q8_ERR_ARG
    assert code_of(L, hctx, w, 8, a, 0, 4096, 2, 2048, 16, scale=3)[0] == Q8_ERR_ARG
    # negative sizes
    assert code_of(L, hctx, w, 8, a, 0, 4096, -1, 2048, 16)[0] == Q8_ERR_SHAPE
    assert code_of(L, hctx, w, 8, a, 0, 4096, 1, 2048, -16)[0] == Q8_ERR_SHAPE
    # weights past the end of the weight buffer
    assert code_of(L, hctx, w, 9, a, 0, 4096, 2, 2048, 16)[0] == Q8_ERR_RANGE
    assert code_of(L, hctx, w, 8, a, 0, 4096, 2, 2048, 17)[0] == Q8_ERR_RANGE
    # x / y past the end of the activation arena
    assert code_of(L, hctx, w, 8, a, 6000, 0, 2, 2048, 16)[0] == Q8_ERR_RANGE
    assert code_of(L, hctx, w, 8, a, 0, 9990, 2, 2048, 16)[0] == Q8_ERR_RANGE
    # x and y overlap
    assert code_of(L, hctx, w, 8, a, 0, 2048, 2, 2048, 16)[0] == Q8_ERR_ARG
    # empty problems are valid no-ops
    assert code_of(L, hctx, w, 8, a, 0, 4096, 0, 2048, 16)[0] == Q8_ERR_NODEVICE


def test_linear_swiglu_validation(hctx):
    """q8_linear_swiglu: prompt rows only (s >= 32), gate / up / y in the
    arena and y apart from both inputs; valid calls reach the device step."""
    m, n, s = 2048, 64, 32
    rs = q8hip.rowstride_u16(m)
    w = hctx.alloc(2 * n * rs)
    a = hctx.alloc(4 * (2 * s * m + s * n))
    L = q8hip.linear_swiglu
    og, ou, oy = 0, s * m, 2 * s * m
    assert code_of(L, hctx, w, 0, a, og, ou, oy, s, m, n)[0] == Q8_ERR_NODEVICE
    assert code_of(L, hctx, w, 0, a, og, ou, oy, 31, m, n)[0] == q8hip.Q8_ERR_UNSUPPORTED
    assert code_of(L, hctx, w, 0, a, og, ou, ou, s, m, n)[0] == Q8_ERR_ARG      # y on up
    assert code_of(L, hctx, w, 0, a, og, ou, og + 8, s, m, n)[0] == Q8_ERR_ARG  # y on gate
    assert code_of(L, hctx, w, 0, a, og, ou, oy + 8, s, m, n)[0] == Q8_ERR_RANGE
    assert code_of(L, hctx, w, 0, a, og + 1, ou, oy, s, m, n)[0] == q8hip.Q8_ERR_UNSUPPORTED
    assert code_of(L, hctx, w, 8, a, og, ou, oy, s, m, n)[0] == Q8_ERR_RANGE    # rows past w
    # gate|up stacked in rows of ld >= 2m (ou = og + m); y after s rows of 2m + 8
    a2 = hctx.alloc(4 * (s * (2 * m + 8) + s * n))
    oy2 = s * (2 * m + 8)
    for og2, ld, want in ((0, 2 * m, Q8_ERR_NODEVICE), (0, m - 4, Q8_ERR_SHAPE),
                          (0, 2 * m + 2, q8hip.Q8_ERR_UNSUPPORTED),   # rows not 16-byte aligned
                          (8, 2 * m + 8, Q8_ERR_NODEVICE),            # the last up row ends at y
                          (12, 2 * m + 8, Q8_ERR_ARG)):               # ... and one past it
        assert code_of(L, hctx, w, 0, a2, og2, og2 + m, oy2, s, m, n, ld=ld)[0] == want, ld
    w.free()
    a.free()
    a2.free()


def test_head_rmsnorm_validation(hctx):
    """q8_head_rmsnorm: heads of head_dim inside rows of ld >= heads *
    head_dim, in place or apart from x, norm weights inside w; valid calls
    reach the device step."""
    tokens, heads, hd, ld = 5, 4, 128, 1024
    w = hctx.alloc(2 * hd)
    a = hctx.alloc(4 * (2 * tokens * ld))
    H = q8hip.head_rmsnorm

    def code(ox, oy, t=tokens, h=heads, d=hd, l=ld, wbuf=w, owt=0):
        return code_of(H, hctx, wbuf, owt, a, ox, oy, t, h, d, l, 1e-6)[0]

    assert code(0, 0) == Q8_ERR_NODEVICE                       # in place
    assert code(0, tokens * ld) == Q8_ERR_NODEVICE             # apart
    assert code(512, 512) == Q8_ERR_NODEVICE                   # k heads after 4 q heads
    assert code(0, 8) == Q8_ERR_ARG                            # shifted copy of x
    assert code(0, 0, l=heads * hd - 1) == Q8_ERR_SHAPE       # rows narrower than the heads
    assert code(0, 0, l=0) == Q8_ERR_NODEVICE                  # dense
    span = (tokens - 1) * ld + heads * hd
    assert code(0, 2 * tokens * ld - span) == Q8_ERR_NODEVICE  # y ends at the arena's end
    assert code(0, 2 * tokens * ld - span + 4) == Q8_ERR_RANGE # ... and past it
    assert code(0, 0, h=0) == Q8_ERR_SHAPE
    assert code(0, 0, owt=1) == Q8_ERR_RANGE                   # norm weights past w
    assert code(0, 0, t=0) == Q8_ERR_NODEVICE
    w.free()
    a.free()


def test_linear_rmsnorm_validation(hctx):
    """q8_linear_rmsnorm: prompt rows only (s >= 32) and rows of at most
    16384; norm weights inside w; x, res, h and y in the arena, h equal to x
    or res or apart from both, y apart from all three; valid calls reach the
    device step."""
    m, n, s = 2048, 64, 32
    rs = q8hip.rowstride_u16(m)
    w = hctx.alloc(2 * (n * rs + m))               # rows, then m bf16 norm weights
    norm = n * rs
    a = hctx.alloc(4 * (3 * s * m + s * n))
    L = q8hip.linear_rmsnorm
    ox, ores, oh, oy = 0, s * m, 2 * s * m, 3 * s * m

    def code(*args, **kw):
        return code_of(L, hctx, w, 0, norm, 1e-5, a, *args, **kw)[0]

    assert code(ox, oy, s, m, n) == Q8_ERR_NODEVICE
    assert code(ox, oy, s, m, n, ores_f32=ores, oh_f32=oh) == Q8_ERR_NODEVICE
    assert code(ox, oy, s, m, n, ores_f32=ores, oh_f32=ox) == Q8_ERR_NODEVICE     # h over x
    assert code(ox, oy, s, m, n, ores_f32=ores, oh_f32=ores) == Q8_ERR_NODEVICE   # h over res
    assert code(ox, oy, s, m, n, ores_f32=ores, oh_f32=ox + 8) == Q8_ERR_ARG      # shifted x
    assert code(ox, oy, s, m, n, ores_f32=ores, oh_f32=ores - 8) == Q8_ERR_ARG    # shifted res
    assert code(ox, ores, s, m, n, ores_f32=ores, oh_f32=oh) == Q8_ERR_ARG        # y on res
    assert code(ox, oh, s, m, n, ores_f32=ores, oh_f32=oh) == Q8_ERR_ARG          # y on h
    assert code(ox, ox + 8, s, m, n) == Q8_ERR_ARG                                # y on x
    assert code(ox, oy, 31, m, n) == q8hip.Q8_ERR_UNSUPPORTED
    assert code(ox + 1, oy, s, m, n) == q8hip.Q8_ERR_UNSUPPORTED                  # x misaligned
    assert code(ox, oy + 8, s, m, n) == Q8_ERR_RANGE
    assert code_of(L, hctx, w, 0, norm + 8, 1e-5, a, ox, oy, s, m, n)[0] == Q8_ERR_RANGE
    with pytest.raises(ValueError):
        L(hctx, w, 0, norm, 1e-5, a, ox, oy, s, m, n, ores_f32=ores)
    w.free()
    a.free()
    # rows longer than 16384
    m2 = 16384 + 64
    w2 = hctx.alloc(2 * (n * q8hip.rowstride_u16(m2) + m2))
    a2 = hctx.alloc(4 * (s * m2 + s * n))
    assert code_of(L, hctx, w2, 0, n * q8hip.rowstride_u16(m2), 1e-5, a2, 0, s * m2, s, m2,
                   n)[0] == q8hip.Q8_ERR_UNSUPPORTED
    w2.free()
    a2.free()


def test_linear_fused_validation(hctx):
    m, n = 2048, 64
    rs = q8hip.rowstride_u16(m)
    w = hctx.alloc(2 * (n * rs + m + 4))          # rows, then m bf16 norm weights
    a = hctx.alloc(4 * 16384)
    F = q8hip.linear_fused
    P, Q = q8hip, q8hip
    norm = n * rs
    # valid calls reach the device step
    assert code_of(F, hctx, w, 0, a, 0, 4096, m, n, pre=P.PRE_RMSNORM, onorm_u16=norm,
                   eps=1e-5)[0] == Q8_ERR_NODEVICE
    assert code_of(F, hctx, w, 0, a, 0, 4096, m, n, post=Q.POST_RESIDUAL,
                   ores_f32=4096)[0] == Q8_ERR_NODEVICE
    assert code_of(F, hctx, w, 0, a, 0, 4096, m // 2, n, pre=P.PRE_SWIGLU, post=Q.POST_RESIDUAL,
                   ores_f32=8192)[0] == Q8_ERR_NODEVICE
    assert code_of(F, hctx, w, 0, a, 0, 4096, m, n, post=Q.POST_SWIGLU)[0] == Q8_ERR_NODEVICE
    # unknown prologue / epilogue; odd row count for the swiglu epilogue
    assert code_of(F, hctx, w, 0, a, 0, 4096, m, n, pre=3)[0] == Q8_ERR_ARG
    assert code_of(F, hctx, w, 0, a, 0, 4096, m, n, post=3)[0] == Q8_ERR_ARG
    assert code_of(F, hctx, w, 0, a, 0, 4096, m, n - 1, post=Q.POST_SWIGLU)[0] == Q8_ERR_SHAPE
    # x overlaps y (swiglu reads 2m floats; the swiglu epilogue stores n/2)
    assert code_of(F, hctx, w, 0, a, 0, 2000, m, n)[0] == Q8_ERR_ARG
    assert code_of(F, hctx, w, 0, a, 0, 2000, m // 2, n, pre=P.PRE_SWIGLU)[0] == Q8_ERR_ARG
    assert code_of(F, hctx, w, 0, a, 0, 16384 - n // 2, m, n,
                   post=Q.POST_SWIGLU)[0] == Q8_ERR_NODEVICE
    assert code_of(F, hctx, w, 0, a, 0, 16384 - n // 2, m, n)[0] == Q8_ERR_RANGE
    # residual partly overlapping y; past the arena
    assert code_of(F, hctx, w, 0, a, 0, 4096, m, n, post=Q.POST_RESIDUAL,
                   ores_f32=4100)[0] == Q8_ERR_ARG
    assert code_of(F, hctx, w, 0, a, 0, 4096, m, n, post=Q.POST_RESIDUAL,
                   ores_f32=16380)[0] == Q8_ERR_RANGE
    # norm weights past the weight buffer, or not 8-byte aligned
    assert code_of(F, hctx, w, 0, a, 0, 4096, m, n, pre=P.PRE_RMSNORM,
                   onorm_u16=norm + 5)[0] == Q8_ERR_RANGE
    assert code_of(F, hctx, w, 0, a, 0, 4096, m, n, pre=P.PRE_RMSNORM,
                   onorm_u16=norm + 2)[0] == q8hip.Q8_ERR_UNSUPPORTED
    # x past the arena (swiglu: 2m floats)
    assert code_of(F, hctx, w, 0, a, 14000, 0, m, n, pre=P.PRE_SWIGLU)[0] == Q8_ERR_RANGE
    # rows too long to stage a normalised x on chip (a plain x is read from L2)
    big = 32768
    rsb = q8hip.rowstride_u16(big)
    wb = hctx.alloc(2 * (rsb + big))
    ab = hctx.alloc(4 * (big + 16))
    assert code_of(F, hctx, wb, 0, ab, 0, big, big, 1, pre=P.PRE_RMSNORM,
                   onorm_u16=rsb)[0] == q8hip.Q8_ERR_UNSUPPORTED
    assert code_of(F, hctx, wb, 0, ab, 0, big, big, 1)[0] == Q8_ERR_NODEVICE


def test_head_argmax_validation(hctx):
    m, n = 2048, 64
    rs = q8hip.rowstride_u16(m)
    w = hctx.alloc(2 * (2 * n * rs + m))
    a = hctx.alloc(4 * 16384)
    ids, pb = hctx.alloc(8), hctx.alloc(8)
    H = q8hip.head_argmax
    norm, emb = 2 * n * rs, n * rs
    ok = dict(oemb_u16=emb, onext_f32=8192)
    assert code_of(H, hctx, w, 0, norm, 1e-5, a, 0, 4096, m, n, 64, "f16", ids, 0, pb, 0, 1,
                   **ok)[0] == Q8_ERR_NODEVICE
    # logits overlap x; next row overlaps the logits
    assert code_of(H, hctx, w, 0, norm, 1e-5, a, 0, 2000, m, n, 64, "f16", ids)[0] == Q8_ERR_ARG
    assert code_of(H, hctx, w, 0, norm, 1e-5, a, 0, 4096, m, n, 64, "f16", ids, 0, pb, 0, 1,
                   oemb_u16=emb, onext_f32=4100)[0] == Q8_ERR_ARG
    # id / position slots, norm weights and embedding table out of range
    assert code_of(H, hctx, w, 0, norm, 1e-5, a, 0, 4096, m, n, 64, "f16", ids, 2)[0] == Q8_ERR_RANGE
    assert code_of(H, hctx, w, 0, norm, 1e-5, a, 0, 4096, m, n, 64, "f16", ids, 0, pb,
                   2)[0] == Q8_ERR_RANGE
    assert code_of(H, hctx, w, 0, norm + 1, 1e-5, a, 0, 4096, m, n, 64, "f16",
                   ids)[0] == Q8_ERR_RANGE
    assert code_of(H, hctx, w, 0, norm, 1e-5, a, 0, 4096, m, n, 64, "f16", ids,
                   oemb_u16=emb + n * rs, onext_f32=8192)[0] == Q8_ERR_RANGE
    # x or logits past the arena
    assert code_of(H, hctx, w, 0, norm, 1e-5, a, 0, 16380, m, n, 64, "f16",
                   ids)[0] == Q8_ERR_RANGE


def test_linear_bf16act_validation(hctx):
    rs = q8hip.rowstride_u16(1024, 32, "f32")
    w = hctx.alloc(2 * 64 * rs)
    x = hctx.alloc(2 * 512 * 1024)
    y = hctx.alloc(4 * 512 * 64)
    L = q8hip.linear_bf16act
    assert code_of(L, hctx, w, 0, x, 0, y, 0, 512, 1024, 64, 32, "f32")[0] == Q8_ERR_NODEVICE
    assert code_of(L, hctx, w, 0, x, 1, y, 0, 512, 1024, 64, 32, "f32")[0] == Q8_ERR_RANGE
    assert code_of(L, hctx, w, 0, x, 0, y, 1, 512, 1024, 64, 32, "f32")[0] == Q8_ERR_RANGE
    assert code_of(L, hctx, w, 0, x, 0, y, 0, 512, 1000, 64, 32, "f32")[0] == Q8_ERR_SHAPE


def test_pack_validation(hctx):
    n, m = 8, 256
    rs = q8hip.rowstride_u16(m)
    src = hctx.alloc(4 * n * m)
    dst = hctx.alloc(2 * n * rs)
    P = q8hip.quantize_pack
    assert code_of(P, hctx, src, 0, Q8_SRC_F32, n, m, dst, 0)[0] == Q8_ERR_NODEVICE
    assert code_of(P, hctx, src, 0, Q8_SRC_BF16, n, m, dst, 0)[0] == Q8_ERR_NODEVICE
    assert code_of(P, hctx, src, 1, Q8_SRC_F32, n, m, dst, 0)[0] == Q8_ERR_RANGE
    assert code_of(P, hctx, src, 0, Q8_SRC_F32, n, m, dst, 1)[0] == Q8_ERR_RANGE
    assert code_of(P, hctx, src, 0, 7, n, m, dst, 0)[0] == Q8_ERR_ARG
    assert code_of(P, hctx, src, 0, Q8_SRC_F32, n, 200, dst, 0)[0] == Q8_ERR_SHAPE
    assert code_of(P, hctx, src, 0, Q8_SRC_F32, -1, m, dst, 0)[0] == Q8_ERR_SHAPE
    # in-place packing would overwrite its own input
    assert code_of(P, hctx, src, 0, Q8_SRC_F32, 2, m, src, 0)[0] == Q8_ERR_ARG


def test_embed_validation(hctx):
    d, vocab = 2048, 10
    rs = q8hip.rowstride_u16(d)
    w = hctx.alloc(2 * vocab * rs)
    ids = hctx.alloc(4 * 4)
    a = hctx.alloc(4 * 4 * d)
    E = q8hip.embed_gather
    assert code_of(E, hctx, w, 0, ids, 0, a, 0, 4, d, vocab)[0] == Q8_ERR_NODEVICE
    assert code_of(E, hctx, w, 0, ids, 0, a, 0, 4, d, vocab + 1)[0] == Q8_ERR_RANGE
    assert code_of(E, hctx, w, 0, ids, 1, a, 0, 4, d, vocab)[0] == Q8_ERR_RANGE
    assert code_of(E, hctx, w, 0, ids, 0, a, 1, 4, d, vocab)[0] == Q8_ERR_RANGE
    assert code_of(E, hctx, w, 0, ids, 0, a, 0, 4, 100, vocab)[0] == Q8_ERR_SHAPE


def test_null_handles():
    lib = q8hip.lib()
    assert lib.q8_linear(None, None, 0, None, 0, 0, 1, 64, 1, 64, 1) == Q8_ERR_ARG
    assert lib.q8_sync(None) == Q8_ERR_ARG
    assert lib.q8_last_error(None) is not None


def test_buffer_ranges(hctx):
    b = hctx.alloc(64)
    assert b.ptr == 0                      # host-only: sizes only
    c, _ = code_of(b.upload, np.zeros(80, dtype=np.uint8))
    assert c == Q8_ERR_RANGE
    c, _ = code_of(b.upload, np.zeros(16, dtype=np.uint8), 60)
    assert c == Q8_ERR_RANGE
    c, _ = code_of(b.upload, np.zeros(16, dtype=np.uint8), 0)
    assert c == Q8_ERR_NODEVICE


def test_no_device_context_fails_cleanly():
    import torch
    if torch.cuda.device_count() > 0:
        pytest.skip("a GPU is present")
    with pytest.raises(Q8Error) as ei:
        q8hip.Context(0)
    assert ei.value.code == q8hip.Q8_ERR_HIP


def test_acts_arena_semantics(hctx):
    a = q8.Acts(hctx, 1000)
    assert a.top == q8.PAD
    o1 = a.alloc(100)
    assert o1 == q8.PAD
    mark = a.mark()
    a.alloc(800)
    with pytest.raises(RuntimeError, match="acts arena overflow"):
        a.alloc(100)
    a.reset(mark)
    assert a.alloc(10) == mark


def test_weights_arena_overflow(hctx):
    w = q8.Weights(hctx, 100)
    with pytest.raises(RuntimeError, match="weight arena overflow at big"):
        w.upload_all({"big": np.zeros(80, dtype=np.uint16)}, ["big"])


def test_mm_q8_op_allocates_output_then_validates(hctx):
    rs = q8.q8_rowstride(2048)
    w = q8.Weights(hctx, q8.PAD + 4 * rs)
    a = q8.Acts(hctx, q8.PAD + 2048 + 4)
    qk = q8.Q8Kernels(hctx)
    ox = a.alloc(2048)
    with pytest.raises(Q8Error) as ei:
        q8.mm_q8_op(hctx, w, a, qk, ox, 1, 2048, q8.PAD, 4)
    assert ei.value.code == Q8_ERR_NODEVICE
    assert a.top == q8.PAD + 2048 + 4   # y was allocated, as mm_q8_op does


def test_gemm_activation_buffer_limit(hctx):
    """From 32 rows q8_linear runs the dequant-GEMM through the context's
    64 MiB binary16 activation buffer, which must hold at least one row
    (2 m + 4 bytes) plus n weight-row exponents: larger shapes are
    rejected before any launch (a zero-row chunk would never advance)."""
    big = 1 << 26
    w = hctx.alloc(1 << 44)                # host-only: sizes only
    a = hctx.alloc(1 << 44)
    L = q8hip.linear
    # m = 2^24: 2 m + 4 bytes per row no longer fit with the exponents
    m = 1 << 25
    c, msg = code_of(L, hctx, w, 0, a, 0, 32 * m, 32, m, 64)
    assert c == Q8_ERR_SHAPE and "activation buffer" in msg
    # one row fewer than the GEMM threshold takes the small-batch path: no limit
    assert code_of(L, hctx, w, 0, a, 0, 31 * m, 31, m, 64)[0] == Q8_ERR_NODEVICE
    # n weight-row exponents alone fill the buffer
    c, msg = code_of(L, hctx, w, 0, a, 0, 32 * 64, 32, 64, big // 4)
    assert c == Q8_ERR_SHAPE and "activation buffer" in msg
    assert code_of(L, hctx, w, 0, a, 0, 32 * 64, 32, 64, big // 8)[0] == Q8_ERR_NODEVICE
    B = q8hip.linear_bf16act
    c, msg = code_of(B, hctx, w, 0, a, 0, a, 1 << 40, 1, m, 64)
    assert c == Q8_ERR_SHAPE and "activation buffer" in msg


def test_qkv_row_stride_validation(hctx):
    """Row strides of q8_rope_kv / q8_attention: 0 or at least each row
    width; k's columns may not meet q's at the stride; the q rows' span,
    not s * qd, must fit the arena."""
    nh, nkv, hd, s, maxlen = 8, 2, 64, 16, 64
    qd, kvd = nh * hd, nkv * hd
    ld = qd + 2 * kvd
    a = hctx.alloc(4 * (s * ld + hd + 2 * s * qd))
    kv = hctx.alloc(2 * 2 * maxlen * kvd)
    blk = maxlen * kvd
    oinv = s * ld

    def rope(oq, ok, ov, ld_):
        return code_of(q8hip.rope_kv, hctx, a, oq, ok, ov, oinv, kv, 0, blk, maxlen, s, 0, nh,
                       nkv, hd, ld=ld_)

    assert rope(0, qd, qd + kvd, ld)[0] == Q8_ERR_NODEVICE
    assert rope(0, qd, qd + kvd, 0)[0] == Q8_ERR_ARG           # dense spans overlap
    assert rope(0, qd, qd + kvd, qd - 1)[0] == Q8_ERR_SHAPE
    assert rope(0, qd, qd + kvd, -ld)[0] == Q8_ERR_SHAPE
    c, msg = rope(0, qd - 1, qd + kvd, ld)                     # k's first column is q's last
    assert c == Q8_ERR_ARG and "stride" in msg
    assert rope(0, ld - kvd + 1, qd + kvd, ld)[0] == Q8_ERR_ARG   # k wraps into the next q row
    # q rows wrap into the next row's v columns (and the last one into
    # inv_freq): q is rotated in place while v is read
    c, msg = rope(qd + kvd, 2 * qd + kvd, 0, ld)
    assert c == Q8_ERR_ARG and "v rows" in msg
    assert rope(2 * kvd, 0, kvd, ld)[0] == Q8_ERR_NODEVICE    # rotated: k, v, then q
    assert rope(kvd, 0, qd + kvd, ld)[0] == Q8_ERR_NODEVICE   # k before q in each row
    assert rope(0, qd, qd + kvd - 1, ld)[0] == Q8_ERR_ARG     # v's first column is k's last
    assert rope(0, qd, qd - 1, ld)[0] == Q8_ERR_ARG           # v's first column is q's last
    # dense rows (one row each): v must meet neither q nor k, inv_freq
    # neither q nor k (v and inv_freq are only read, they may meet)
    s1 = 1
    dense = lambda oq, ok, ov, oi: code_of(q8hip.rope_kv, hctx, a, oq, ok, ov, oi, kv, 0, blk,
                                           maxlen, s1, 0, nh, nkv, hd)[0]
    assert dense(0, qd, qd + kvd, qd + 2 * kvd) == Q8_ERR_NODEVICE
    assert dense(0, qd, qd + kvd, qd + kvd) == Q8_ERR_NODEVICE    # inv_freq inside v
    assert dense(0, qd, qd + kvd - 1, qd + 2 * kvd) == Q8_ERR_ARG   # v meets k
    assert dense(0, qd, qd - 1, qd + 2 * kvd) == Q8_ERR_ARG         # v meets q
    assert dense(0, qd, qd + kvd, qd - 1) == Q8_ERR_ARG             # inv_freq meets q
    assert dense(0, qd, qd + kvd, qd + kvd - 1) == Q8_ERR_ARG       # inv_freq meets k
    na = s * ld + hd + 2 * s * qd                               # arena floats
    assert rope(na - (s - 1) * ld - qd, 0, 0, ld)[0] != Q8_ERR_RANGE
    assert rope(na - (s - 1) * ld - qd + 1, 0, 0, ld)[0] == Q8_ERR_RANGE   # last q row past it

    def attn(oq, ldq):
        return code_of(q8hip.attention, hctx, a, oq, kv, 0, blk, maxlen, oinv + hd, 0, s, 0,
                       nh, nkv, hd, ldq=ldq)

    assert attn(0, ld)[0] == Q8_ERR_NODEVICE
    assert attn(0, qd - 1)[0] == Q8_ERR_SHAPE
    assert attn(2 * kvd, ld)[0] == Q8_ERR_NODEVICE
    # a span that reaches the output
    assert attn(oinv + hd - (s - 1) * ld - qd + 1, ld)[0] == Q8_ERR_ARG
    # 16 rows take the one-pass kernel, which moves q and out in 16-byte vectors
    for oq, ldq, oy in ((1, ld, oinv + hd), (0, ld + 1, oinv + hd), (0, ld, oinv + hd + 2)):
        c, msg = code_of(q8hip.attention, hctx, a, oq, kv, 0, blk, maxlen, oy, 0, s, 0, nh, nkv,
                         hd, ldq=ldq)
        assert c == q8hip.Q8_ERR_UNSUPPORTED and "aligned" in msg, (oq, ldq, oy)
    for b in (a, kv):
        b.free()


@pytest.mark.parametrize("which", ["rope_kv", "attention"])
def test_kv_cache_block_under_2gib(hctx, which):
    """The attention kernels address a K or V block with 32-bit buffer
    offsets: maxlen * nkv * head_dim binary16 values must stay under 2 GiB
    (the same limit q8_decode_attention enforces)."""
    nh, nkv, hd = 32, 8, 128
    a = hctx.alloc(4 * 200000)
    kv = hctx.alloc(1 << 44)
    ok_len = (1 << 30) // (nkv * hd) - 1          # 2 GiB - 2 KiB per block
    bad_len = (1 << 30) // (nkv * hd)             # exactly 2 GiB per block
    for maxlen, want in ((ok_len, Q8_ERR_NODEVICE), (bad_len, Q8_ERR_SHAPE),
                         (4 * bad_len, Q8_ERR_SHAPE)):
        blk = maxlen * nkv * hd
        if which == "rope_kv":
            c, msg = code_of(q8hip.rope_kv, hctx, a, 0, 8192, 9216, 10240, kv, 0, blk, maxlen,
                             1, 0, nh, nkv, hd)
        else:
            # 16 query rows: the one-pass kernel, which needs no scratch
            c, msg = code_of(q8hip.attention, hctx, a, 0, kv, 0, blk, maxlen, 65536, 0, 16, 0,
                             nh, nkv, hd)
        assert c == want, (maxlen, msg)
        if want == Q8_ERR_SHAPE:
            assert "2 GiB" in msg


def test_noalloc_validation_without_a_device():
    """q8_linear_noalloc rejects misaligned pointers (w 2-byte, x and y
    4-byte: the alignment q8_linear's element offsets give), null pointers,
    overlapping x and y and bad shapes before any HIP call."""
    L = q8hip.linear_noalloc
    base = 1 << 20                                   # never dereferenced
    for wo, xo, yo in ((1, 0, 4096), (0, 2, 4096), (0, 0, 4098), (0, 1, 4096)):
        c, msg = code_of(L, None, base + wo, base + xo, base + yo, 1, 64, 4, 64, "f16")
        assert c == Q8_ERR_ARG and "aligned" in msg, (wo, xo, yo, msg)
    c, msg = code_of(L, None, 0, base, base + 4096, 1, 64, 4, 64, "f16")
    assert c == Q8_ERR_ARG and "null" in msg
    c, msg = code_of(L, None, base, base, base + 128, 1, 64, 4, 64, "f16")
    assert c == Q8_ERR_ARG and "overlap" in msg
    c, msg = code_of(L, None, base, base, base + 4096, 1, 100, 4, 64, "f16")
    assert c == Q8_ERR_SHAPE
    assert code_of(L, None, base + 1, base + 1, base + 3, 0, 64, 4, 64, "f16")[0] == 0   # empty
