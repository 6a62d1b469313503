"""q8_linear_noalloc (through the C ABI) against q8_linear.

The allocation-free entry point runs q8_linear's kernels with its scratch
in the library's fixed per-GPU array instead of a context's workspace, so
on every path -- the one-row GEMV, the f32 4x4-block kernel (2-4 rows),
the split-bf16 kernel with its cross-workgroup K split (partials in the
scratch), the dequant-GEMM with its binary16 buffer and split-K partials --
it must give q8_linear's bits.  Each case calls it twice in a row, the
second time with a smaller input, so a first call's leftovers in the shared
array (partials, exponents) would show.  A GEMM
whose rows overflow the 16 MiB activation buffer runs in row chunks and is
held to the 1e-3 contract against the float64 oracle instead.
"""

import os
import subprocess
import sys

import numpy as np
import pytest

from lama32_mojo_amd import q8hip
from lama32_mojo_amd.q8hip import Q8_ERR_ARG, Q8_ERR_SHAPE, Q8Error
from oracle.q8_oracle import max_rel_err, synth_weights_bf16, synth_x

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def case_buffers(ctx, cor, s, n, m, G, scale, seed):
    pk = cor.pack_bf16(synth_weights_bf16(n, m, seed=seed), G, scale)
    w = ctx.alloc(pk.nbytes)
    w.upload(pk)
    x = synth_x(s, m, seed=seed + 1)
    a = ctx.alloc(4 * (s * m + 2 * s * n))
    a.upload(x)
    return pk, w, x, a


def run_both(ctx, w, a, s, m, n, G, scale):
    """q8_linear into y1, q8_linear_noalloc (raw pointers, the context's
    stream) into y2; returns both."""
    oy1, oy2 = s * m, s * m + s * n
    q8hip.linear(ctx, w, 0, a, 0, oy1, s, m, n, G, scale)
    q8hip.linear_noalloc(ctx.stream, w.ptr, a.ptr, a.ptr + 4 * oy2, s, m, n, G, scale)
    ctx.sync()
    return a.download((s, n), np.float32, 4 * oy1), a.download((s, n), np.float32, 4 * oy2)


# (s, n, m) first call, then (s2, n2, m2) second (smaller) call, and the path
PAIRS = [((1, 3072, 2048), (1, 1000, 1536), "GEMV"),
         ((4, 4096, 4096), (3, 512, 2048), "f32 4x4 blocks"),
         ((16, 4096, 12288), (9, 2048, 8192), "split bf16, K split over workgroups"),
         ((512, 2048, 2048), (64, 1024, 2048), "GEMM, K split with a reduce launch"),
         ((512, 16384, 1024), (40, 24, 4096), "GEMM, 256-column tiles / one ragged tile")]


@pytest.mark.parametrize("G,scale", [(64, "f16"), (32, "f32")])
@pytest.mark.parametrize("first,second,path", PAIRS)
def test_noalloc_equals_q8_linear(ctx, cor, G, scale, first, second, path):
    say("noalloc", G, scale, first, second, path)
    for k, (s, n, m) in enumerate((first, second)):
        pk, w, x, a = case_buffers(ctx, cor, s, n, m, G, scale, seed=100 * k + s + n)
        y1, y2 = run_both(ctx, w, a, s, m, n, G, scale)
        assert np.array_equal(y1, y2), (path, k, np.abs(y1 - y2).max())
        assert max_rel_err(y2, cor.linear_f64(pk, x, G, scale)) <= (1e-5 if s < 32 else 1e-3)
        w.free()
        a.free()


def test_noalloc_gemm_in_row_chunks(ctx, cor):
    """1024 rows of 8192 binary16 values (16 MiB) do not fit the 16 MiB
    activation buffer with the weight exponents: two row chunks, each its
    own GEMM launch; then a small call reuses the array."""
    say("noalloc chunks")
    G, scale = 32, "f32"
    for s, n, m in ((1024, 1024, 8192), (48, 512, 1024)):
        pk, w, x, a = case_buffers(ctx, cor, s, n, m, G, scale, seed=s + 7)
        y1, y2 = run_both(ctx, w, a, s, m, n, G, scale)
        ref = cor.linear_f64(pk, x, G, scale)
        assert max_rel_err(y2, ref) <= 1e-3
        assert max_rel_err(y1, ref) <= 1e-3
        for r in (0, 511, 512, s - 1):
            if r < s:
                assert max_rel_err(y2[r], ref[r]) <= 1e-3, r
        w.free()
        a.free()


def test_noalloc_errors(ctx):
    """Argument errors come back as status codes with the calling thread's
    message, before any launch."""
    say("noalloc errors")
    w = ctx.alloc(1 << 20)
    a = ctx.alloc(1 << 20)
    L = q8hip.linear_noalloc
    with pytest.raises(Q8Error) as e:
        L(ctx.stream, 0, a.ptr, a.ptr + 4096, 1, 64, 4, 64, "f16")
    assert e.value.code == Q8_ERR_ARG and "null" in e.value.msg
    with pytest.raises(Q8Error) as e:
        L(ctx.stream, w.ptr, a.ptr, a.ptr + 128, 1, 64, 4, 64, "f16")      # y inside x
    assert e.value.code == Q8_ERR_ARG and "overlap" in e.value.msg
    with pytest.raises(Q8Error) as e:
        L(ctx.stream, w.ptr, a.ptr, a.ptr + 4096, 1, 100, 4, 64, "f16")
    assert e.value.code == Q8_ERR_SHAPE
    for wo, xo, yo in ((1, 0, 4096), (0, 2, 4096), (0, 0, 4097)):          # misaligned
        with pytest.raises(Q8Error) as e:
            L(ctx.stream, w.ptr + wo, a.ptr + xo, a.ptr + yo, 1, 64, 4, 64, "f16")
        assert e.value.code == Q8_ERR_ARG and "aligned" in e.value.msg, (wo, xo, yo)
    with pytest.raises(Q8Error) as e:                                      # one row too long
        L(ctx.stream, w.ptr, a.ptr, a.ptr + (1 << 40), 32, 1 << 23, 4, 64, "f16")
    assert e.value.code == Q8_ERR_SHAPE and "allocation-free" in e.value.msg
    L(ctx.stream, w.ptr, a.ptr, a.ptr + 4096, 0, 64, 4, 64, "f16")        # empty: no-op
    w.free()
    a.free()


# (s, n, m): the GEMV, the split-bf16 kernel with its cross-workgroup K split
# and reduce launch, the GEMM with split-K partials and its reduce launch
CAPTURED = [(1, 3072, 2048), (16, 4096, 12288), (512, 2048, 2048)]


@pytest.mark.parametrize("G,scale", [(64, "f16"), (32, "f32")])
def test_noalloc_captured_graph_replays(ctx, cor, G, scale):
    """q8_linear_noalloc captured into a HIP graph on the context's stream:
    every replay gives eager q8_linear's bits.  Between replays the output
    is overwritten with NaN and eager calls of other sizes reuse the
    shared scratch (and the eager reference runs), so a replay that read a
    leftover or skipped a write would show."""
    say("noalloc captured", G, scale)
    bufs = []
    for k, (s, n, m) in enumerate(CAPTURED):
        pk, w, x, a = case_buffers(ctx, cor, s, n, m, G, scale, seed=300 + 7 * k + s)
        bufs.append((s, n, m, w, a))
    ctx.graph_begin()
    try:
        for s, n, m, w, a in bufs:
            q8hip.linear_noalloc(ctx.stream, w.ptr, a.ptr, a.ptr + 4 * (s * m + s * n), s, m, n,
                                 G, scale)
    finally:
        g = ctx.graph_end()
    try:
        nan = {s: np.full((s, n), np.nan, np.float32) for s, n, m, w, a in bufs}
        for rep in range(3):
            for s, n, m, w, a in bufs:
                a.upload(nan[s], 4 * (s * m + s * n))
            ctx.sync()
            g.launch()
            ctx.sync()
            for s, n, m, w, a in reversed(bufs):        # other sizes, then the reference
                q8hip.linear_noalloc(ctx.stream, w.ptr, a.ptr, a.ptr + 4 * s * m, s, m, n, G,
                                     scale)
                q8hip.linear(ctx, w, 0, a, 0, s * m, s, m, n, G, scale)
            ctx.sync()
            for s, n, m, w, a in bufs:
                want = a.download((s, n), np.float32, 4 * s * m)
                got = a.download((s, n), np.float32, 4 * (s * m + s * n))
                assert np.array_equal(got, want), (rep, s, n, m)
    finally:
        g.destroy()
        for s, n, m, w, a in bufs:
            w.free()
            a.free()


_CHILD = r"""
import sys
import numpy as np
from lama32_mojo_amd import q8hip
from oracle.q8_oracle import c_oracle, synth_weights_bf16, synth_x
print("child: first q8_linear_noalloc inside a capture", flush=True)
cor = c_oracle()
ctx = q8hip.Context(0)
for (s, n, m, G, scale) in ((16, 4096, 12288, 32, "f32"), (1, 3072, 2048, 64, "f16")):
    pk = cor.pack_bf16(synth_weights_bf16(n, m, seed=s + n), G, scale)
    w = ctx.alloc(pk.nbytes)
    w.upload(pk)
    a = ctx.alloc(4 * (s * m + 2 * s * n))
    a.upload(synth_x(s, m, seed=s))
    oy1, oy2 = s * m, s * m + s * n
    ctx.graph_begin()
    try:
        q8hip.linear_noalloc(ctx.stream, w.ptr, a.ptr, a.ptr + 4 * oy2, s, m, n, G, scale)
    finally:
        g = ctx.graph_end()
    for rep in range(2):
        a.upload(np.full((s, n), np.nan, np.float32), 4 * oy2)
        g.launch()
        ctx.sync()
        q8hip.linear(ctx, w, 0, a, 0, oy1, s, m, n, G, scale)
        ctx.sync()
        y1 = a.download((s, n), np.float32, 4 * oy1)
        y2 = a.download((s, n), np.float32, 4 * oy2)
        if not np.array_equal(y1, y2):
            print("child: replay differs", s, n, m, rep, flush=True)
            sys.exit(3)
    g.destroy()
    w.free()
    a.free()
ctx.close()
print("child: ok", flush=True)
"""


def test_noalloc_first_call_inside_capture():
    """In a fresh process the very first q8_linear_noalloc call -- the one
    that resolves the device's scratch array -- happens inside a graph
    capture; the captured launch replays to q8_linear's bits."""
    say("noalloc first call in capture (child process)")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ)
    env["PYTHONPATH"] = root + os.pathsep + env.get("PYTHONPATH", "")
    r = subprocess.run([sys.executable, "-c", _CHILD], cwd=root, env=env, capture_output=True,
                       text=True, timeout=100)
    say(r.stdout.strip())
    assert r.returncode == 0 and "child: ok" in r.stdout, (r.returncode, r.stderr[-2000:])
