"""GPU parity at the widths of the 8B-class models (through the C ABI)
against the float64 oracle.

Shapes (m inputs -> n outputs):
  Qwen3-8B      q|k|v 4096 -> 6144, o 4096 -> 4096, gate|up 4096 -> 24576,
                down 12288 -> 4096, lm_head 4096 -> 151936
  Llama-3.1-8B  q|k|v 4096 -> 6144, o 4096 -> 4096, gate|up 4096 -> 28672,
                down 14336 -> 4096, untied lm_head 4096 -> 128256
                (llama31_mojo/src/llama_gpu.mojo:26-41,142-159)
  Qwen3-0.6B    q|k|v 1024 -> 4096 (qwen3_mojo/src/qwen_q8.mojo:212-224)
Each reaches a GEMV shape class the 1B shapes do not: one activation row
with 4096 .. 8191 outputs (2 rows per wave), rows longer than 8192 codes
(the K split over the waves with x read from L2), the fused 2-row class
and the vocabulary heads; the few-row and small-batch kernels at 4 and 16
rows; the dequant-GEMM's 256-column tiles and its K = 14336 pre-pass; the
prompt-row attention at 2048 rows.

Bars (written in each test): the f32 GEMV / few-row / small-batch paths
within 1e-5 normwise of float64 (f32 products on the GEMV and few-row
paths, x as bf16 hi + lo with a residual below 2^-17 |x| on the small-batch
path; f32 sums); the fused GEMV
within 1e-5 of float64 rmsnorm / swiglu / residual around the float64
linear; the f16-MFMA GEMM within 1e-3 (the product contract), also per
activation row, and per output column at 2e-3 for small weights; attention
within 1e-5.
"""

import sys

import numpy as np
import pytest

from lama32_mojo_amd import q8hip
from oracle import model_oracle as mo
from oracle.q8_oracle import (bf16_bits_to_f32, elementwise_err, f32_to_bf16_bits, max_rel_err,
                              synth_weights_bf16, synth_x)

pytestmark = pytest.mark.gpu
LAYOUTS = [(64, "f16"), (32, "f32")]

# (m, n): every s = 1 decode projection of the three models
DECODE_8B = [(4096, 6144), (4096, 4096), (1024, 4096), (4096, 24576), (4096, 28672),
             (12288, 4096), (14336, 4096), (4096, 128256), (4096, 151936)]
QWEN3_8B = [(4096, 6144), (4096, 4096), (4096, 24576), (12288, 4096), (4096, 151936)]


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


class Packed:
    """n x m random bf16 weights ~ N(0, std), generated and packed on the GPU
    (q8_quantize_pack, bit-exact against the oracle's packer in
    test_gpu_parity), with the packed rows downloaded for the oracle."""

    def __init__(self, ctx, n, m, G, scale, seed, std=0.02, extra_u16=0):
        import torch
        self.n, self.m, self.G, self.scale = n, m, G, scale
        self.rs = q8hip.rowstride_u16(m, G, scale)
        gen = torch.Generator(device="cuda")
        gen.manual_seed(seed)
        src = (torch.randn((n, m), device="cuda", generator=gen) * std).to(torch.bfloat16)
        torch.cuda.synchronize()
        sbuf = ctx.wrap(src.data_ptr(), src.numel() * 2)
        self.w = ctx.alloc(2 * (n * self.rs + extra_u16))
        q8hip.quantize_pack(ctx, sbuf, 0, q8hip.Q8_SRC_BF16, n, m, self.w, 0, G, scale)
        ctx.sync()
        sbuf.free()
        del src
        self.pk = self.w.download((n, self.rs), np.uint16)

    def free(self):
        self.w.free()


def run_linear(ctx, P, x):
    s = x.shape[0]
    a = ctx.alloc(4 * (s * P.m + s * P.n))
    a.upload(np.ascontiguousarray(x, dtype=np.float32))
    q8hip.linear(ctx, P.w, 0, a, 0, s * P.m, s, P.m, P.n, P.G, P.scale)
    y = a.download((s, P.n), np.float32, 4 * s * P.m)
    a.free()
    return y


@pytest.mark.parametrize("G,scale", LAYOUTS)
@pytest.mark.parametrize("m,n", DECODE_8B)
def test_gemv_one_row_8b_shapes(ctx, cor, G, scale, m, n):
    say("8B GEMV s=1", G, scale, m, n)
    P = Packed(ctx, n, m, G, scale, seed=m + n)
    x = synth_x(1, m, seed=7)
    y = run_linear(ctx, P, x)
    ref = cor.linear_f64(P.pk, x, G, scale)
    err = max_rel_err(y, ref)
    assert err <= 1e-5, err
    if n >= 65536:                       # the vocabulary heads pick the same token
        assert int(np.argmax(y[0])) == int(np.argmax(ref[0]))
    P.free()


@pytest.mark.parametrize("G,scale", LAYOUTS)
@pytest.mark.parametrize("m,n", QWEN3_8B)
@pytest.mark.parametrize("s", [4, 16])
def test_batched_decode_qwen3_8b_shapes(ctx, cor, G, scale, m, n, s):
    """Batches of 4 (f32 4x4-block MFMA, shared-x form from n = 16384) and
    16 rows (split-bf16 MFMA; the down projection splits K over workgroups)
    at every Qwen3-8B decode shape, row by row."""
    say("8B batched", G, scale, m, n, s)
    P = Packed(ctx, n, m, G, scale, seed=3 * m + n)
    x = synth_x(s, m, seed=11 + s)
    y = run_linear(ctx, P, x)
    ref = cor.linear_f64(P.pk, x, G, scale)
    for b in range(s):
        assert max_rel_err(y[b], ref[b]) <= 1e-5, b
    P.free()


# (m, n, pre, post): the fused launches of the 8B decode steps
FUSED_8B = [(4096, 6144, q8hip.PRE_RMSNORM, q8hip.POST_STORE),       # q|k|v
            (1024, 4096, q8hip.PRE_RMSNORM, q8hip.POST_STORE),       # Qwen3-0.6B q|k|v
            (4096, 4096, q8hip.PRE_NONE, q8hip.POST_RESIDUAL),       # o + residual
            (4096, 24576, q8hip.PRE_RMSNORM, q8hip.POST_SWIGLU),     # Qwen3-8B gate|up
            (4096, 28672, q8hip.PRE_RMSNORM, q8hip.POST_SWIGLU),     # Llama-3.1-8B gate|up
            (12288, 4096, q8hip.PRE_NONE, q8hip.POST_RESIDUAL),      # Qwen3-8B down
            (14336, 4096, q8hip.PRE_NONE, q8hip.POST_RESIDUAL),      # Llama-3.1-8B down
            (12288, 4096, q8hip.PRE_SWIGLU, q8hip.POST_RESIDUAL),    # swiglu read by down
            (4096, 128256, q8hip.PRE_RMSNORM, q8hip.POST_STORE)]     # untied lm_head


# (m, n, pre, post): the fused launches of the Llama-3.2-1B decode step (the
# headline workload) and the Qwen3-0.6B ones the 8B widths do not reach
FUSED_1B = [(2048, 3072, q8hip.PRE_RMSNORM, q8hip.POST_STORE),       # rmsnorm + q|k|v
            (2048, 2048, q8hip.PRE_NONE, q8hip.POST_RESIDUAL),       # o + residual
            (2048, 16384, q8hip.PRE_RMSNORM, q8hip.POST_SWIGLU),     # rmsnorm + gate|up + swiglu
            (8192, 2048, q8hip.PRE_NONE, q8hip.POST_RESIDUAL),       # down + residual
            (2048, 128256, q8hip.PRE_RMSNORM, q8hip.POST_STORE),     # final norm + tied lm_head
            (1024, 6144, q8hip.PRE_RMSNORM, q8hip.POST_SWIGLU),      # Qwen3-0.6B gate|up
            (2048, 1024, q8hip.PRE_NONE, q8hip.POST_RESIDUAL),       # Qwen3-0.6B o
            (3072, 1024, q8hip.PRE_NONE, q8hip.POST_RESIDUAL)]       # Qwen3-0.6B down


@pytest.mark.parametrize("G,scale", LAYOUTS)
@pytest.mark.parametrize("m,n,pre,post", FUSED_8B + FUSED_1B)
def test_fused_gemv_8b_shapes_against_float64(ctx, cor, G, scale, m, n, pre, post):
    """q8_linear_fused against float64 rmsnorm / swiglu of the input, the
    float64 linear of the oracle and float64 swiglu / residual of its
    outputs (the oracle's linear takes its input as f32: the normed or
    gated x is rounded once to f32, 2^-24 relative, far below the bar)."""
    say("8B fused", G, scale, m, n, pre, post)
    rng = np.random.default_rng(m + 7 * n + pre)
    P = Packed(ctx, n, m, G, scale, seed=5 * m + n, extra_u16=m)
    wn = f32_to_bf16_bits((1 + 0.1 * rng.standard_normal(m)).astype(np.float32))
    onorm = n * P.rs
    P.w.upload(wn, 2 * onorm)
    eps = 1e-5
    x2 = (2 * rng.standard_normal(2 * m)).astype(np.float32)      # x, or [gate | up]
    nout = n // 2 if post == q8hip.POST_SWIGLU else n
    res = rng.standard_normal(nout).astype(np.float32)
    ox, oy = 0, 2 * m
    a = ctx.alloc(4 * (2 * m + nout))
    a.upload(x2)
    if post == q8hip.POST_RESIDUAL:
        a.upload(res, 4 * oy)
    q8hip.linear_fused(ctx, P.w, 0, a, ox, oy, m, n, G, scale, pre, onorm, eps, post, oy)
    got = a.download((nout,), np.float32, 4 * oy)
    a.free()

    x = x2[:m].astype(np.float64)
    if pre == q8hip.PRE_RMSNORM:
        x = mo.rmsnorm(x[None, :], wn, eps)[0]
    elif pre == q8hip.PRE_SWIGLU:
        x = mo.swiglu(x2[:m], x2[m:].astype(np.float64))
    y = cor.linear_f64(P.pk, x[None, :].astype(np.float32), G, scale)[0]
    if post == q8hip.POST_SWIGLU:
        want = mo.swiglu(y[:n // 2], y[n // 2:])
    elif post == q8hip.POST_RESIDUAL:
        want = res.astype(np.float64) + y
    else:
        want = y
    assert np.all(np.isfinite(got))
    err = max_rel_err(got, want)
    assert err <= 1e-5, err
    P.free()


# (m, n): rows longer than 4096 codes at one activation row take the K split
# in workgroups of 16 waves (n >= 4096, 16 rows each, at most 256
# workgroups looping over the rest) or 8 waves (n >= 2048, 8 rows each) with
# x staged in LDS; ragged n leaves a partial last tile, and 8896 rows make
# every workgroup walk two or three tiles.
LONG_ROWS_RAGGED = [(8192, 4100), (8192, 2050), (5120, 8896), (12288, 2056)]


@pytest.mark.parametrize("G,scale", LAYOUTS)
@pytest.mark.parametrize("m,n", LONG_ROWS_RAGGED)
def test_long_rows_ragged_against_float64(ctx, cor, G, scale, m, n):
    """q8_linear and q8_linear_fused (residual in place) on the long-row
    K-split workgroups, ragged and multi-tile, within 1e-5 of float64."""
    say("long rows", G, scale, m, n)
    P = Packed(ctx, n, m, G, scale, seed=m + 3 * n)
    x = synth_x(1, m, seed=5)
    y = run_linear(ctx, P, x)
    ref = cor.linear_f64(P.pk, x, G, scale)
    assert max_rel_err(y, ref) <= 1e-5
    res = np.random.default_rng(n).standard_normal(n).astype(np.float32)
    a = ctx.alloc(4 * (m + n))
    a.upload(x)
    a.upload(res, 4 * m)
    q8hip.linear_fused(ctx, P.w, 0, a, 0, m, m, n, G, scale, post=q8hip.POST_RESIDUAL, ores_f32=m)
    got = a.download((n,), np.float32, 4 * m)
    a.free()
    assert max_rel_err(got, res.astype(np.float64) + ref[0]) <= 1e-5
    P.free()


@pytest.mark.parametrize("G,scale", LAYOUTS)
@pytest.mark.parametrize("m,n", [(4096, 128256), (2048, 128256), (1024, 151936)])
def test_head_argmax_untied_8b_head(ctx, cor, G, scale, m, n):
    """q8_head_argmax over the Llama-3.1-8B head (4096 -> 128256), the
    Llama-3.2-1B head of the headline step (2048 -> 128256) and the
    Qwen3-0.6B one (1024 -> 151936): the float64 model's token, logits
    within 1e-5."""
    say("head argmax", G, scale, m, n)
    rng = np.random.default_rng(17)
    P = Packed(ctx, n, m, G, scale, seed=99, extra_u16=m)
    wn = f32_to_bf16_bits((1 + 0.1 * rng.standard_normal(m)).astype(np.float32))
    onorm = n * P.rs
    P.w.upload(wn, 2 * onorm)
    x = rng.standard_normal(m).astype(np.float32)
    a = ctx.alloc(4 * (m + n))
    a.upload(x)
    ids = ctx.alloc(16)
    q8hip.head_argmax(ctx, P.w, 0, onorm, 1e-5, a, 0, m, m, n, G, scale, ids, 0)
    tok = int(ids.download((1,), np.int32)[0])
    y = a.download((n,), np.float32, 4 * m)
    xn = mo.rmsnorm(x[None, :].astype(np.float64), wn, 1e-5).astype(np.float32)
    ref = cor.linear_f64(P.pk, xn, G, scale)[0]
    assert max_rel_err(y, ref) <= 1e-5
    assert tok == int(np.argmax(y))
    top = np.sort(ref)[-2:]
    if top[1] - top[0] > 1e-5 * np.max(np.abs(ref)):
        assert tok == int(np.argmax(ref))
    for b in (a, ids):
        b.free()
    P.free()


# (s, n, m): the prefill GEMMs of the 1B bench (stacked gate|up) and of
# Llama-3.1-8B (2048-token prompt: gate 4096 -> 14336, down 14336 -> 4096)
GEMM_8B = [(512, 16384, 2048), (2048, 14336, 4096), (2048, 4096, 14336)]


def sample_rows(s):
    """Rows spread over every 128-row tile edge: the oracle runs on these."""
    rows = {0, 1, s - 1, s // 2 + 3}
    for t in range(0, s, 128):
        rows.update({t, min(s - 1, t + 127), min(s - 1, t + 64 + (t // 128) % 37)})
    return np.array(sorted(rows))


@pytest.mark.parametrize("G,scale", LAYOUTS)
@pytest.mark.parametrize("s,n,m", GEMM_8B)
@pytest.mark.parametrize("act", ["bf16", "f32"])
def test_gemm_large_shapes(ctx, cor, G, scale, s, n, m, act):
    """The dequant-GEMM at its 256-column tiles (all three shapes fill 256
    or more of them) and, at m = 14336, the K = 14336 binary16 pre-pass;
    every output row is computed, the oracle checks rows spread over every
    row tile: within 1e-3 normwise, and each of those rows on its own."""
    say("8B GEMM", G, scale, s, n, m, act)
    P = Packed(ctx, n, m, G, scale, seed=s + n + m)
    x = synth_x(s, m, seed=s + 1)
    if act == "bf16":
        xbits = f32_to_bf16_bits(x)
        xb = ctx.alloc(2 * s * m)
        xb.upload(xbits)
        yb = ctx.alloc(4 * s * n)
        q8hip.linear_bf16act(ctx, P.w, 0, xb, 0, yb, 0, s, m, n, G, scale)
        y = yb.download((s, n), np.float32)
        xb.free()
        yb.free()
        x = bf16_bits_to_f32(xbits)
    else:
        y = run_linear(ctx, P, x)
    rows = sample_rows(s)
    ref = cor.linear_f64(P.pk, np.ascontiguousarray(x[rows]), G, scale)
    got = y[rows]
    err = max_rel_err(got, ref)
    assert err <= 1e-3, err
    for i, r in enumerate(rows):
        assert max_rel_err(got[i], ref[i]) <= 1e-3, r
    ew = elementwise_err(got, ref, cor.linear_abs(P.pk, np.ascontiguousarray(x[rows]), G, scale))
    assert ew <= 1e-3, ew
    assert np.all(np.isfinite(y))
    P.free()


@pytest.mark.parametrize("G,scale", LAYOUTS)
def test_linear_swiglu_8b_prompt_against_float64(ctx, cor, G, scale):
    """The Llama-3.1-8B prompt path's down projection: q8_linear_swiglu over
    2048 stacked gate|up rows (row stride 2 x 14336, silu(g) * u formed in
    the binary16 pre-pass) -> 4096 outputs, against float64 swiglu and the
    float64 linear on rows spread over every row tile: within 1e-3
    normwise, per row and elementwise (each output against sum |x||w|)."""
    say("linear_swiglu 8B", G, scale)
    s, m, n = 2048, 14336, 4096
    P = Packed(ctx, n, m, G, scale, seed=77)
    rng = np.random.default_rng(78)
    gu = rng.standard_normal((s, 2 * m), dtype=np.float32)
    gu[:, :m] *= 2.0
    a = ctx.alloc(4 * (s * 2 * m + s * n))
    a.upload(gu)
    oy = s * 2 * m
    q8hip.linear_swiglu(ctx, P.w, 0, a, 0, m, oy, s, m, n, G, scale, ld=2 * m)
    y = a.download((s, n), np.float32, 4 * oy)
    a.free()
    rows = sample_rows(s)
    xs = mo.swiglu(gu[rows, :m], gu[rows, m:].astype(np.float64))
    ref = cor.linear_f64x(P.pk, xs, G, scale)
    got = y[rows]
    assert np.all(np.isfinite(y))
    assert max_rel_err(got, ref) <= 1e-3
    for i, r in enumerate(rows):
        assert max_rel_err(got[i], ref[i]) <= 1e-3, r
    ew = elementwise_err(got, ref, cor.linear_abs(P.pk, xs, G, scale))
    assert ew <= 1e-3, ew
    P.free()


def mixed_magnitude_weights(n, m, G, seed):
    """bf16 weights whose rows span five decades (row std 3e-2 .. 1e-5) and
    whose groups inside a row alternate between full size and 1/20."""
    rng = np.random.default_rng(seed)
    row = np.array([1e-2, 1e-3, 1e-4, 1e-5, 3e-2])[np.arange(n) % 5]
    grp = np.where((np.arange(m) // G) % 2 == 0, 1.0, 0.05)
    w = rng.standard_normal((n, m)) * row[:, None] * grp[None, :]
    return f32_to_bf16_bits(w.astype(np.float32))


@pytest.mark.parametrize("G,scale", LAYOUTS)
@pytest.mark.parametrize("act", ["bf16", "f32"])
@pytest.mark.parametrize("std", [1e-2, 1e-3, 1e-4, "mixed"])
def test_gemm_small_weights(ctx, cor, G, scale, act, std):
    """Small weights through the dequant-GEMM: with f32 scales each weight
    row's scales are brought to binary16 after a power-of-two shift of the
    row (without it a group absmax under 7.75e-3 gives a binary16-subnormal
    scale), so weight std 1e-2 .. 1e-4 and rows that mix magnitudes stay
    within 1e-3 normwise.  Each output column (one weight row) is also
    checked on its own against its largest value over the 64 activation
    rows, a weaker normaliser than the whole output, at 2e-3: the binary16
    roundings give about 3e-4 there, a subnormal binary16 scale of a
    1e-5-std row about 1e-1."""
    say("gemm small weights", G, scale, act, std)
    s, n, m = 64, 500, 2048
    if std == "mixed":
        wb = mixed_magnitude_weights(n, m, G, seed=71)
    else:
        wb = synth_weights_bf16(n, m, seed=72, std=std)
    pk = cor.pack_bf16(wb, G, scale)
    w = ctx.alloc(pk.nbytes)
    w.upload(pk)
    x = synth_x(s, m, seed=73)
    if act == "bf16":
        xbits = f32_to_bf16_bits(x)
        xb = ctx.alloc(2 * s * m)
        xb.upload(xbits)
        yb = ctx.alloc(4 * s * n)
        q8hip.linear_bf16act(ctx, w, 0, xb, 0, yb, 0, s, m, n, G, scale)
        y = yb.download((s, n), np.float32)
        for b in (xb, yb):
            b.free()
        x = bf16_bits_to_f32(xbits)
    else:
        a = ctx.alloc(4 * (s * m + s * n))
        a.upload(x)
        q8hip.linear(ctx, w, 0, a, 0, s * m, s, m, n, G, scale)
        y = a.download((s, n), np.float32, 4 * s * m)
        a.free()
    w.free()
    ref = cor.linear_f64(pk, x, G, scale)
    assert max_rel_err(y, ref) <= 1e-3
    col = np.abs(y - ref).max(axis=0) / np.abs(ref).max(axis=0)
    assert col.max() <= 2e-3, (int(col.argmax()), col.max())


@pytest.mark.parametrize("head_dim,nh,nkv,s,pos0,maxlen", [(128, 32, 8, 2048, 0, 2048),
                                                           (128, 32, 8, 1000, 1048, 2048),
                                                           (64, 32, 8, 2048, 0, 2048)])
def test_prompt_attention_long_prompt(ctx, head_dim, nh, nkv, s, pos0, maxlen):
    """The MFMA prompt-row attention over a whole 2048-token prompt (the
    Llama-3.1-8B prefill: 32 / 8 heads of 128) and over the second half of
    one whose first half is cached, within 1e-5 of float64."""
    say("prompt attention", head_dim, nh, nkv, s, pos0)
    rng = np.random.default_rng(8)
    qd, kvd = nh * head_dim, nkv * head_dim
    kc = (rng.standard_normal((maxlen, kvd)) * 0.7).astype(np.float16)
    vc = rng.standard_normal((maxlen, kvd)).astype(np.float16)
    q = rng.standard_normal((s, qd)).astype(np.float32)
    kv = ctx.alloc(2 * 2 * maxlen * kvd)
    kv.upload(np.concatenate([kc.reshape(-1), vc.reshape(-1)]))
    assert q8hip.attention_scratch_floats(s, nh, head_dim, maxlen) == 0
    a = ctx.alloc(4 * 2 * s * qd)
    a.upload(q)
    q8hip.attention(ctx, a, 0, kv, 0, maxlen * kvd, maxlen, s * qd, 0, s, pos0, nh, nkv,
                    head_dim)
    y = a.download((s, qd), np.float32, 4 * s * qd)
    ref = mo.attention(q.astype(np.float64), kc.astype(np.float64), vc.astype(np.float64), pos0,
                       nh, nkv, head_dim)
    assert max_rel_err(y, ref) <= 1e-5
    for r in (0, 1, s // 2, s - 1):
        assert max_rel_err(y[r], ref[r]) <= 1e-5, r
    for b in (a, kv):
        b.free()
