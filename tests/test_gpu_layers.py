"""GPU parity of the decode-step layer kernels and the Q8 model runner
(through the C ABI) against the CPU oracle (oracle/model_oracle.py).

Bars (written in each test):
  * rmsnorm / rope / attention / swiglu: max relative error <= 1e-5 against
    the float64 restatement (f32 arithmetic on the GPU);
  * residual adds and the binary16 cache rows of v: bit-exact; rotated k in
    the cache: within one binary16 ulp (the angle's cos/sin differ in the
    last f32 bits);
  * whole model: last-position logits within max-rel-err 1e-3 of the float64
    model (which rounds the cache to binary16 like the build), and the same
    greedy ids;
  * device-position calls and graph replays: bit-identical to the
    host-position eager calls.
"""

import sys

import numpy as np
import pytest

from lama32_mojo_amd import model as gm
from lama32_mojo_amd import q8hip
from oracle import model_oracle as mo
from oracle.q8_oracle import f32_to_bf16_bits, max_rel_err

sys.path.insert(0, __file__.rsplit("/", 1)[0])
from test_model_oracle import qwen_tiny, tiny_model  # noqa: E402

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def arena(ctx, floats):
    return ctx.alloc(4 * floats)


def put(buf, off_f32, x):
    buf.upload(np.ascontiguousarray(x, dtype=np.float32), 4 * off_f32)


def get(buf, off_f32, shape):
    return buf.download(shape, np.float32, 4 * off_f32)


@pytest.mark.parametrize("d", [64, 100, 1000, 2048, 4096, 5000, 8192, 9000])
def test_rmsnorm_and_add_rmsnorm(ctx, d):
    """Rows of 64 to 9000 elements (ragged ones too: fewer than 256, or not
    a multiple of 256) against float64; the residual form's h bit-exact, in
    place too."""
    say("rmsnorm", d)
    rng = np.random.default_rng(d)
    rows, eps = 3, 1e-5
    x = rng.standard_normal((rows, d)).astype(np.float32)
    o = rng.standard_normal((rows, d)).astype(np.float32)
    wbits = f32_to_bf16_bits((1 + 0.2 * rng.standard_normal(d)).astype(np.float32))
    w = ctx.alloc(2 * (16 + d))
    w.upload(wbits, 2 * 16)
    a = arena(ctx, 5 * rows * d)
    put(a, 0, x)
    put(a, rows * d, o)
    q8hip.rmsnorm(ctx, w, 16, a, 0, 2 * rows * d, rows, d, eps)
    y = get(a, 2 * rows * d, (rows, d))
    assert max_rel_err(y, mo.rmsnorm(x, wbits, eps)) <= 1e-5
    q8hip.add_rmsnorm(ctx, w, 16, a, 0, rows * d, 3 * rows * d, 4 * rows * d, rows, d, eps)
    h = get(a, 3 * rows * d, (rows, d))
    assert np.array_equal(h, x + o)
    y2 = get(a, 4 * rows * d, (rows, d))
    assert max_rel_err(y2, mo.rmsnorm(h, wbits, eps)) <= 1e-5
    # residual sum in place (h == x)
    put(a, 3 * rows * d, x)
    q8hip.add_rmsnorm(ctx, w, 16, a, 3 * rows * d, rows * d, 3 * rows * d, 4 * rows * d, rows, d,
                      eps)
    assert np.array_equal(get(a, 3 * rows * d, (rows, d)), h)
    assert np.array_equal(get(a, 4 * rows * d, (rows, d)), y2)
    # in place (y == x)
    q8hip.rmsnorm(ctx, w, 16, a, 0, 0, rows, d, eps)
    assert np.array_equal(get(a, 0, (rows, d)), y)
    w.free()
    a.free()


@pytest.mark.parametrize("head_dim", [64, 128])
def test_rope_kv_append(ctx, head_dim):
    say("rope_kv", head_dim)
    rng = np.random.default_rng(1)
    nh, nkv, s, pos0, maxlen = 8, 2, 3, 5, 16
    qd, kvd = nh * head_dim, nkv * head_dim
    inv = mo.llama3_inv_freq(head_dim, 500000.0, 32.0, 1.0, 4.0, 8192.0)
    q = rng.standard_normal((s, qd)).astype(np.float32)
    k = rng.standard_normal((s, kvd)).astype(np.float32)
    v = rng.standard_normal((s, kvd)).astype(np.float32)
    oq, ok, ov, oinv = 0, s * qd, s * qd + s * kvd, s * qd + 2 * s * kvd
    a = arena(ctx, oinv + head_dim)
    put(a, oq, q)
    put(a, ok, k)
    put(a, ov, v)
    put(a, oinv, inv)
    kv = ctx.alloc(2 * 2 * maxlen * kvd)
    kv.upload(np.zeros(2 * maxlen * kvd, np.float16))
    q8hip.rope_kv(ctx, a, oq, ok, ov, oinv, kv, 0, maxlen * kvd, maxlen, s, pos0, nh, nkv, head_dim)
    qr, kr = get(a, oq, (s, qd)), get(a, ok, (s, kvd))
    assert max_rel_err(qr, mo.rope(q, pos0, inv, nh, head_dim)) <= 1e-5
    kref = mo.rope(k, pos0, inv, nkv, head_dim)
    assert max_rel_err(kr, kref) <= 1e-5
    cache = kv.download((2, maxlen, kvd), np.float16)
    kc, vc = cache[0].astype(np.float64), cache[1]
    assert np.all(kc[:pos0] == 0) and np.all(kc[pos0 + s:] == 0)
    ulp = np.spacing(np.abs(kref).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(kc[pos0:pos0 + s] - mo.f16_round(kref)) <= ulp)
    assert np.array_equal(vc[pos0:pos0 + s], v.astype(np.float16))
    # device position: same bits
    pb = ctx.alloc(16)
    pb.upload(np.array([pos0, 0, 0, 0], np.int32))
    put(a, oq, q)
    put(a, ok, k)
    kv.upload(np.zeros(2 * maxlen * kvd, np.float16))
    q8hip.rope_kv(ctx, a, oq, ok, ov, oinv, kv, 0, maxlen * kvd, maxlen, s, 0, nh, nkv, head_dim,
                  posbuf=pb, opos_i32=0)
    assert np.array_equal(get(a, oq, (s, qd)), qr)
    assert np.array_equal(kv.download((2, maxlen, kvd), np.float16), cache)
    for b in (a, kv, pb):
        b.free()


@pytest.mark.parametrize("head_dim,nh,nkv", [(64, 32, 8), (128, 32, 8), (64, 8, 8), (128, 16, 2),
                                              (64, 16, 8)])
@pytest.mark.parametrize("s,pos0", [(1, 0), (1, 63), (1, 64), (1, 1023), (5, 100), (3, 1021),
                                     (15, 9), (16, 0), (37, 5), (200, 700), (130, 894),
                                     (300, 0)])
def test_attention(ctx, head_dim, nh, nkv, s, pos0):
    say("attention", head_dim, nh, nkv, s, pos0)
    rng = np.random.default_rng(2)
    maxlen = 1024
    qd, kvd = nh * head_dim, nkv * head_dim
    kc = (rng.standard_normal((maxlen, kvd)) * 0.7).astype(np.float16)
    vc = rng.standard_normal((maxlen, kvd)).astype(np.float16)
    q = rng.standard_normal((s, qd)).astype(np.float32)
    kv = ctx.alloc(2 * 2 * maxlen * kvd)
    kv.upload(np.concatenate([kc.reshape(-1), vc.reshape(-1)]))
    scr = q8hip.attention_scratch_floats(s, nh, head_dim, maxlen)
    oq, oy, osc = 0, s * qd, 2 * s * qd
    a = arena(ctx, osc + scr)
    put(a, oq, q)
    q8hip.attention(ctx, a, oq, kv, 0, maxlen * kvd, maxlen, oy, osc, s, pos0, nh, nkv, head_dim)
    y = get(a, oy, (s, qd))
    ref = mo.attention(q.astype(np.float64), kc.astype(np.float64), vc.astype(np.float64), pos0,
                       nh, nkv, head_dim)
    assert max_rel_err(y, ref) <= 1e-5
    pb = ctx.alloc(16)
    pb.upload(np.array([pos0, 0, 0, 0], np.int32))
    q8hip.attention(ctx, a, oq, kv, 0, maxlen * kvd, maxlen, oy, osc, s, 0, nh, nkv, head_dim,
                    posbuf=pb, opos_i32=0)
    assert np.array_equal(get(a, oy, (s, qd)), y)
    for b in (a, kv, pb):
        b.free()


@pytest.mark.parametrize("head_dim,nh,nkv,s", [(64, 8, 2, 3), (128, 32, 8, 48),
                                               (64, 32, 8, 130)])
def test_stacked_qkv_rows_equal_dense(ctx, head_dim, nh, nkv, s):
    """q|k|v stacked in the rows of one linear output (row stride
    qd + 2*kvd): RoPE leaves the same q and k bits in place and writes the
    same cache bits as on dense q, k, v, and attention over the stacked q
    gives the same output bits as over the dense q (the few-row split path
    at 3 rows, the one-pass path at 48 and 130)."""
    say("stacked q|k|v", head_dim, nh, nkv, s)
    rng = np.random.default_rng(11)
    pos0, maxlen = 7, 256
    qd, kvd = nh * head_dim, nkv * head_dim
    ld = qd + 2 * kvd
    inv = mo.llama3_inv_freq(head_dim, 500000.0, 32.0, 1.0, 4.0, 8192.0)
    rows = rng.standard_normal((s, ld)).astype(np.float32)
    q, k, v = rows[:, :qd], rows[:, qd:qd + kvd], rows[:, qd + kvd:]
    od = s * ld                                 # dense q, k, v after the stacked rows
    oq, ok, ov = od, od + s * qd, od + s * qd + s * kvd
    oinv = ov + s * kvd
    scr = q8hip.attention_scratch_floats(s, nh, head_dim, maxlen)
    oy1, oy2 = oinv + head_dim, oinv + head_dim + s * qd
    osc = oy2 + s * qd
    a = arena(ctx, osc + scr)
    put(a, 0, rows)
    put(a, oq, np.ascontiguousarray(q))
    put(a, ok, np.ascontiguousarray(k))
    put(a, ov, np.ascontiguousarray(v))
    put(a, oinv, inv)
    kv = ctx.alloc(4 * 2 * maxlen * kvd)
    kv.upload(np.zeros(4 * maxlen * kvd, np.float16))
    blk = maxlen * kvd
    q8hip.rope_kv(ctx, a, 0, qd, qd + kvd, oinv, kv, 0, blk, maxlen, s, pos0, nh, nkv, head_dim,
                  ld=ld)
    q8hip.rope_kv(ctx, a, oq, ok, ov, oinv, kv, 2 * blk, 3 * blk, maxlen, s, pos0, nh, nkv,
                  head_dim)
    st = get(a, 0, (s, ld))
    assert np.array_equal(st[:, :qd], get(a, oq, (s, qd)))
    assert np.array_equal(st[:, qd:qd + kvd], get(a, ok, (s, kvd)))
    assert np.array_equal(st[:, qd + kvd:], v)               # v is only read
    c = kv.download((4, blk), np.float16)
    assert np.array_equal(c[0], c[2]) and np.array_equal(c[1], c[3])
    assert np.any(c[0] != 0)
    q8hip.attention(ctx, a, 0, kv, 0, blk, maxlen, oy1, osc, s, pos0, nh, nkv, head_dim, ldq=ld)
    q8hip.attention(ctx, a, oq, kv, 2 * blk, 3 * blk, maxlen, oy2, osc, s, pos0, nh, nkv,
                    head_dim)
    assert np.array_equal(get(a, oy1, (s, qd)), get(a, oy2, (s, qd)))
    for b in (a, kv):
        b.free()


@pytest.mark.parametrize("head_dim,nh,nkv", [(128, 32, 8), (64, 8, 8)])
def test_attention_prompt_rows_any_q_scale(ctx, head_dim, nh, nkv):
    """The multi-row (s >= 16) path splits q into binary16 hi + lo after a
    per-column power-of-two scaling: rows of q from 1e-30 to 30 in size
    (a sharply peaked softmax at the top; beyond that f32 scores themselves
    drift from float64) and an all-zero row (uniform weights) stay within
    max-rel-err 1e-5 of float64, row by row."""
    say("attention q scales", head_dim, nh, nkv)
    rng = np.random.default_rng(5)
    maxlen, s, pos0 = 512, 48, 40
    qd, kvd = nh * head_dim, nkv * head_dim
    kc = (rng.standard_normal((maxlen, kvd)) * 0.7).astype(np.float16)
    vc = rng.standard_normal((maxlen, kvd)).astype(np.float16)
    q = rng.standard_normal((s, qd))
    scales = np.array([1e-30, 1e-7, 1e-3, 0.05, 1.0, 7.0, 30.0, 0.0])
    q = (q * scales[np.arange(s) % len(scales)][:, None]).astype(np.float32)
    kv = ctx.alloc(2 * 2 * maxlen * kvd)
    kv.upload(np.concatenate([kc.reshape(-1), vc.reshape(-1)]))
    assert q8hip.attention_scratch_floats(s, nh, head_dim, maxlen) == 0
    a = arena(ctx, 2 * s * qd)
    put(a, 0, q)
    q8hip.attention(ctx, a, 0, kv, 0, maxlen * kvd, maxlen, s * qd, 0, s, pos0, nh, nkv, head_dim)
    y = get(a, s * qd, (s, qd))
    ref = mo.attention(q.astype(np.float64), kc.astype(np.float64), vc.astype(np.float64), pos0,
                       nh, nkv, head_dim)
    for i in range(s):
        assert max_rel_err(y[i], ref[i]) <= 1e-5, (i, scales[i % len(scales)])
    for b in (a, kv):
        b.free()


@pytest.mark.parametrize("head_dim,nh,nkv", [(64, 32, 8), (128, 32, 8), (64, 16, 16), (128, 8, 1)])
@pytest.mark.parametrize("pos0", [0, 1, 31, 32, 63, 64, 95, 96, 500, 1023, 1500])
def test_decode_attention_equals_rope_then_attention(ctx, head_dim, nh, nkv, pos0):
    """The one-launch token step writes the same cache bits as q8_rope_kv and
    matches q8_rope_kv + q8_attention within 2e-6 (it sums the splits in
    another order).  maxlen 1536 gives 24 splits of two 32-key chunks
    (head_dim 64 in groups of 4: 8 waves of one head each; of one 64-key
    chunk in the other groups, one head per wave) or, at head_dim 128, 12 splits of four
    32-key chunks (groups of 4: 8 waves, two per chunk with 2 heads each)
    or 24 of two (groups of 8: each wave one chunk for 4 heads): small pos0
    is served by one block per KV head,
    larger pos0 by several blocks whose records the merge launch combines;
    a second call must reproduce the first."""
    decode_attention_case(ctx, head_dim, nh, nkv, pos0, 1536)


@pytest.mark.parametrize("head_dim,nh,nkv", [(64, 32, 8), (128, 32, 8), (64, 8, 1)])
@pytest.mark.parametrize("pos0", [2100, 5000, 6143])
def test_decode_attention_long_context(ctx, head_dim, nh, nkv, pos0):
    """maxlen 6144 caps the splits at 32, so each block takes several chunks
    per wave (the first chunk guessed before the position is read is then
    reloaded), up to the last cache row."""
    decode_attention_case(ctx, head_dim, nh, nkv, pos0, 6144)


@pytest.mark.parametrize("head_dim,nh,nkv", [(128, 16, 8), (64, 32, 8), (128, 32, 8)])
@pytest.mark.parametrize("pos0", [0, 40, 127, 159])
def test_decode_attention_short_cache(ctx, head_dim, nh, nkv, pos0):
    """A cache of at most 4 chunks per wave (maxlen 160) is served by one
    block per KV head, which takes every chunk and writes the output, with
    no merge launch."""
    decode_attention_case(ctx, head_dim, nh, nkv, pos0, 160)


def decode_attention_case(ctx, head_dim, nh, nkv, pos0, maxlen):
    say("decode attention", head_dim, nh, nkv, pos0, maxlen)
    rng = np.random.default_rng(4)
    qd, kvd = nh * head_dim, nkv * head_dim
    inv = mo.llama3_inv_freq(head_dim, 500000.0, 32.0, 1.0, 4.0, 8192.0)
    cache = rng.standard_normal((2, maxlen, kvd)).astype(np.float16)
    q = rng.standard_normal(qd).astype(np.float32)
    k = rng.standard_normal(kvd).astype(np.float32)
    v = rng.standard_normal(kvd).astype(np.float32)
    oq, ok, ov, oinv, oy = 0, qd, qd + kvd, qd + 2 * kvd, qd + 2 * kvd + head_dim
    osc = oy + qd
    a = arena(ctx, osc + q8hip.attention_scratch_floats(1, nh, head_dim, maxlen))
    kv1, kv2 = ctx.alloc(cache.nbytes), ctx.alloc(cache.nbytes)
    kv1.upload(cache)
    kv2.upload(cache)
    for buf, x in [(oq, q), (ok, k), (ov, v), (oinv, inv)]:
        put(a, buf, x)
    q8hip.decode_attention(ctx, a, oq, ok, ov, oinv, kv1, 0, maxlen * kvd, maxlen, oy, pos0, nh,
                           nkv, head_dim)
    fused = get(a, oy, (qd,))
    put(a, oy, np.zeros(qd, np.float32))
    q8hip.decode_attention(ctx, a, oq, ok, ov, oinv, kv1, 0, maxlen * kvd, maxlen, oy, pos0, nh,
                           nkv, head_dim)
    assert np.array_equal(get(a, oy, (qd,)), fused)
    q8hip.rope_kv(ctx, a, oq, ok, ov, oinv, kv2, 0, maxlen * kvd, maxlen, 1, pos0, nh, nkv,
                  head_dim)
    q8hip.attention(ctx, a, oq, kv2, 0, maxlen * kvd, maxlen, oy, osc, 1, pos0, nh, nkv, head_dim)
    sep = get(a, oy, (qd,))
    c1 = kv1.download((2, maxlen, kvd), np.float16)
    assert np.array_equal(c1, kv2.download((2, maxlen, kvd), np.float16))
    assert np.all(np.isfinite(fused)) and max_rel_err(fused, sep) <= 2e-6
    ref = mo.attention(get(a, oq, (1, qd)).astype(np.float64), c1[0].astype(np.float64),
                       c1[1].astype(np.float64), pos0, nh, nkv, head_dim)
    assert max_rel_err(fused, ref[0]) <= 1e-5
    for b in (a, kv1, kv2):
        b.free()


def test_elementwise_and_argmax(ctx):
    say("elementwise")
    rng = np.random.default_rng(3)
    n = 10000
    g = (rng.standard_normal(n) * 4).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    a = arena(ctx, 4 * n)
    put(a, 0, g)
    put(a, n, u)
    q8hip.swiglu(ctx, a, 0, n, n)
    sw = get(a, 0, (n,))
    assert max_rel_err(sw, mo.swiglu(g.astype(np.float64), u.astype(np.float64))) <= 1e-5
    put(a, 0, g)
    q8hip.res_add(ctx, a, 0, n, 2 * n, n)
    assert np.array_equal(get(a, 2 * n, (n,)), g + u)
    q8hip.add(ctx, a, 0, 2 * n, n)
    assert np.array_equal(get(a, 2 * n, (n,)), (g + u) + g)
    ids = ctx.alloc(16)
    for case in ["random", "ties", "nan", "first", "vocab"]:
        v = rng.standard_normal(n).astype(np.float32)
        if case == "ties":
            v[[77, 5000, 9999]] = 50.0
            want = 77
        elif case == "nan":
            v[[10, 20]] = np.nan
            v[3000] = 40.0
            want = 3000
        elif case == "first":
            v[0] = 99.0
            want = 0
        elif case == "vocab":
            v = rng.standard_normal(128256).astype(np.float32)
            want = int(np.argmax(v))
        else:
            want = int(np.argmax(v))
        b = arena(ctx, len(v))
        put(b, 0, v)
        q8hip.argmax(ctx, b, 0, len(v), ids, 1)
        assert int(ids.download((2,), np.int32)[1]) == want, case
        b.free()
    pb = ctx.alloc(16)
    pb.upload(np.array([5, 0, 0, 0], np.int32))
    q8hip.pos_advance(ctx, pb, 0, 3)
    q8hip.pos_advance(ctx, pb, 0, 1)
    assert int(pb.download((1,), np.int32)[0]) == 9
    for b in (a, ids, pb):
        b.free()


def gpu_model(ctx, spec, tensors, maxlen, max_prefill=8, fuse=True):
    if spec.qk_norm:        # Qwen3-style: plain RoPE, theta 1e6 (as qwen_tiny's oracle)
        cfg = gm.Config(spec.hidden, spec.layers, spec.n_heads, spec.n_kv, spec.head_dim,
                        spec.inter, spec.vocab, spec.eps, 1000000.0, 1.0, 1.0, 4.0, 8192.0,
                        tied=spec.tied, name="tiny-qwen", qk_norm=True, rope="plain")
    else:
        cfg = gm.Config(spec.hidden, spec.layers, spec.n_heads, spec.n_kv, spec.head_dim,
                        spec.inter, spec.vocab, spec.eps, 500000.0, 32.0, 1.0, 4.0, 8192.0,
                        tied=spec.tied, name="tiny")
    return gm.Q8Llama(ctx, cfg, maxlen, spec.G, spec.scale, weights=tensors,
                      max_prefill=max_prefill, fuse=fuse)


# (m, n) of each GEMV shape class: 1 row per wave, 4 rows per wave, K split
# over the waves (m > 4096), vocabulary heads (n >= 65536, 2 rows per wave)
FUSED_SHAPES = [(2048, 3072), (2048, 16384), (8192, 2048), (512, 65600)]


FUSED_CASES = [(q8hip.PRE_RMSNORM, q8hip.POST_STORE), (q8hip.PRE_NONE, q8hip.POST_RESIDUAL),
               (q8hip.PRE_SWIGLU, q8hip.POST_RESIDUAL), (q8hip.PRE_SWIGLU, q8hip.POST_STORE),
               (q8hip.PRE_RMSNORM, q8hip.POST_RESIDUAL), (q8hip.PRE_NONE, q8hip.POST_SWIGLU),
               (q8hip.PRE_RMSNORM, q8hip.POST_SWIGLU)]


@pytest.mark.parametrize("G,scale", [(64, "f16"), (32, "f32")])
@pytest.mark.parametrize("m,n", FUSED_SHAPES)
def test_linear_fused_equals_separate_calls(ctx, G, scale, m, n):
    """q8_linear_fused against q8_rmsnorm or q8_swiglu, then q8_linear, then
    q8_add or q8_swiglu.  Bit-exact without the norm, while both sum each row
    in the same order; max-rel-err <= 1e-5 with the norm (its factor
    multiplies the output instead of each x) and for the swiglu epilogue at
    m > 4096 (whole rows per wave there, K split over the waves in
    q8_linear)."""
    say("linear_fused", G, scale, m, n)
    rng = np.random.default_rng(m + n)
    rs = q8hip.rowstride_u16(m, G, scale)
    wsrc = ctx.alloc(2 * n * m)
    wsrc.upload(f32_to_bf16_bits((0.02 * rng.standard_normal((n, m))).astype(np.float32)))
    w = ctx.alloc(2 * (n * rs + m))
    q8hip.quantize_pack(ctx, wsrc, 0, q8hip.Q8_SRC_BF16, n, m, w, 0, G, scale)
    wsrc.free()
    onorm = n * rs
    w.upload(f32_to_bf16_bits((1 + 0.1 * rng.standard_normal(m)).astype(np.float32)), 2 * onorm)
    x2 = (2 * rng.standard_normal(2 * m)).astype(np.float32)    # x, or [gate | up]
    res = rng.standard_normal(n).astype(np.float32)
    ox, oxs, oy, oyf, ores = 0, 2 * m, 3 * m, 3 * m + n, 3 * m + 2 * n
    a = arena(ctx, 3 * m + 3 * n)
    put(a, ox, x2)
    eps = 1e-5

    def separate(pre, post):
        if pre == q8hip.PRE_RMSNORM:
            q8hip.rmsnorm(ctx, w, onorm, a, ox, oxs, 1, m, eps)
        else:
            put(a, oxs, x2[:m])
            if pre == q8hip.PRE_SWIGLU:
                q8hip.swiglu(ctx, a, oxs, ox + m, m)
        q8hip.linear(ctx, w, 0, a, oxs, oy, 1, m, n, G, scale)
        if post == q8hip.POST_RESIDUAL:
            put(a, ores, res)
            q8hip.add(ctx, a, ores, oy, n)
        if post == q8hip.POST_SWIGLU:
            q8hip.swiglu(ctx, a, oy, oy + n // 2, n // 2)
            return get(a, oy, (n // 2,))
        return get(a, oy, (n,))

    for pre, post in FUSED_CASES:
        want = separate(pre, post)
        assert np.all(np.isfinite(want)) and np.std(want) > 0
        put(a, ores, res)
        q8hip.linear_fused(ctx, w, 0, a, ox, oyf, m, n, G, scale, pre, onorm, eps, post, ores)
        got = get(a, oyf, want.shape)
        if pre == q8hip.PRE_RMSNORM or (post == q8hip.POST_SWIGLU and m > 4096):
            assert np.all(np.isfinite(got)) and max_rel_err(got, want) <= 1e-5, (pre, post)
        else:
            assert np.array_equal(got, want), (pre, post)
        if post == q8hip.POST_RESIDUAL:           # residual in place
            put(a, oyf, res)
            q8hip.linear_fused(ctx, w, 0, a, ox, oyf, m, n, G, scale, pre, onorm, eps, post, oyf)
            got2 = get(a, oyf, want.shape)
            assert np.array_equal(got2, got), (pre, post, "in place")
    for b in (a, w):
        b.free()


@pytest.mark.parametrize("G,scale", [(64, "f16"), (32, "f32")])
@pytest.mark.parametrize("s,m,n", [(32, 2048, 512), (100, 14336, 1000), (300, 4096, 4096),
                                   (33, 20480, 256)])
def test_linear_swiglu_equals_swiglu_then_linear(ctx, G, scale, s, m, n):
    """q8_linear_swiglu (silu(g) * u computed in the GEMM's binary16 pre-pass)
    gives the bits of q8_swiglu into g followed by q8_linear on g, and leaves
    g and u unchanged: 2048..20480-code rows (the pre-pass holding up to 8
    chunks per thread in registers, and past 16384 re-reading the row),
    ragged row counts.  Gate|up stacked in rows of 2m (one linear's output,
    read at a row stride) give the same bits."""
    say("linear_swiglu", G, scale, s, m, n)
    rng = np.random.default_rng(s + m)
    rs = q8hip.rowstride_u16(m, G, scale)
    wsrc = ctx.alloc(2 * n * m)
    wsrc.upload(f32_to_bf16_bits((0.02 * rng.standard_normal((n, m))).astype(np.float32)))
    w = ctx.alloc(2 * n * rs)
    q8hip.quantize_pack(ctx, wsrc, 0, q8hip.Q8_SRC_BF16, n, m, w, 0, G, scale)
    wsrc.free()
    g = (2 * rng.standard_normal((s, m))).astype(np.float32)
    u = rng.standard_normal((s, m)).astype(np.float32)
    og, ou, oy1, oy2 = 0, s * m, 2 * s * m, 2 * s * m + s * n
    ost = (2 * s * m + 2 * s * n + 3) // 4 * 4       # stacked rows [g | u]
    oy3 = ost + 2 * s * m
    a = arena(ctx, oy3 + s * n)
    try:
        put(a, og, g)
        put(a, ou, u)
        put(a, ost, np.concatenate([g, u], axis=1))
        q8hip.linear_swiglu(ctx, w, 0, a, og, ou, oy2, s, m, n, G, scale)
        got = get(a, oy2, (s, n))
        q8hip.linear_swiglu(ctx, w, 0, a, ost, ost + m, oy3, s, m, n, G, scale, ld=2 * m)
        assert np.array_equal(get(a, oy3, (s, n)), got)
        assert np.array_equal(get(a, og, (s, m)), g) and np.array_equal(get(a, ou, (s, m)), u)
        q8hip.swiglu(ctx, a, og, ou, s * m)
        q8hip.linear(ctx, w, 0, a, og, oy1, s, m, n, G, scale)
        want = get(a, oy1, (s, n))
        assert np.all(np.isfinite(want)) and np.array_equal(got, want), \
            max_rel_err(got, want)
    finally:
        a.free()
        w.free()


@pytest.mark.parametrize("G,scale", [(64, "f16"), (32, "f32")])
@pytest.mark.parametrize("s,m,n,res", [(32, 2048, 512, False), (77, 1024, 3072, True),
                                       (300, 4096, 1000, True), (40, 16384, 256, True),
                                       (64, 5120, 512, False), (2100, 16384, 64, True)])
def test_linear_rmsnorm_equals_norm_then_linear(ctx, cor, G, scale, s, m, n, res):
    """q8_linear_rmsnorm (the RMSNorm, after the residual add, computed in
    the GEMM's binary16 pre-pass) gives the bits of q8_add_rmsnorm /
    q8_rmsnorm into a temporary followed by q8_linear on it, stores h = x +
    res with the bits of q8_add_rmsnorm (h over x in place too), and stays
    within the GEMM's 1e-3 of float64: rows of 1024..16384 codes (8 to 64
    values per thread), ragged row counts, and 2100 rows of 16384 codes (the
    call runs in two row chunks of the activation buffer)."""
    say("linear_rmsnorm", G, scale, s, m, n, res)
    rng = np.random.default_rng(s + m + n)
    rs = q8hip.rowstride_u16(m, G, scale)
    wsrc = ctx.alloc(2 * n * m)
    wsrc.upload(f32_to_bf16_bits((0.02 * rng.standard_normal((n, m))).astype(np.float32)))
    w = ctx.alloc(2 * (n * rs + m))
    q8hip.quantize_pack(ctx, wsrc, 0, q8hip.Q8_SRC_BF16, n, m, w, 0, G, scale)
    wsrc.free()
    onorm = n * rs
    wbits = f32_to_bf16_bits((1 + 0.2 * rng.standard_normal(m)).astype(np.float32))
    w.upload(wbits, 2 * onorm)
    eps = 1e-5
    x = (3 * rng.standard_normal((s, m))).astype(np.float32)
    r = rng.standard_normal((s, m)).astype(np.float32)
    sm, sn = s * m, s * n
    ox, ores, oh, oz, ox2, oy1, oy2, oy3 = (0, sm, 2 * sm, 3 * sm, 4 * sm, 5 * sm, 5 * sm + sn,
                                          5 * sm + 2 * sn)
    a = arena(ctx, 5 * sm + 3 * sn)
    try:
        put(a, ox, x)
        put(a, ores, r)
        put(a, ox2, x)
        kw = dict(ores_f32=ores, oh_f32=oh) if res else {}
        q8hip.linear_rmsnorm(ctx, w, 0, onorm, eps, a, ox, oy2, s, m, n, G, scale, **kw)
        got = get(a, oy2, (s, n))
        if res:
            h = get(a, oh, (s, m))
            q8hip.add_rmsnorm(ctx, w, onorm, a, ox, ores, oh, oz, s, m, eps)
            assert np.array_equal(get(a, oh, (s, m)), h)
            # h stored over x
            q8hip.linear_rmsnorm(ctx, w, 0, onorm, eps, a, ox2, oy3, s, m, n, G, scale,
                                 ores_f32=ores, oh_f32=ox2)
            assert np.array_equal(get(a, oy3, (s, n)), got)
            assert np.array_equal(get(a, ox2, (s, m)), h)
        else:
            h = x
            q8hip.rmsnorm(ctx, w, onorm, a, ox, oz, s, m, eps)
            assert np.array_equal(get(a, ox, (s, m)), x)
        q8hip.linear(ctx, w, 0, a, oz, oy1, s, m, n, G, scale)
        want = get(a, oy1, (s, n))
        assert np.all(np.isfinite(want)) and np.array_equal(got, want), \
            max_rel_err(got, want)
        if s * m * n <= 300 * 4096 * 1000:
            rows = np.arange(0, s, max(1, s // 16))
            pk = w.download((n, rs), np.uint16)
            ref = cor.linear_f64x(pk, mo.rmsnorm(h[rows], wbits, eps), G, scale)
            assert max_rel_err(got[rows], ref) <= 1e-3
    finally:
        a.free()
        w.free()


def test_model_prompt_folds_equal_separate_launches(ctx):
    """A prompt whose norms run in the GEMM pre-passes and whose residual adds
    run in the next block's norm gives the logits bits of the separate
    rmsnorm / add / linear launches, and the same cache."""
    say("prompt folds")
    spec, t, inv = tiny_model(seed=11)
    maxlen = 64
    prompt = [int(v) for v in np.random.default_rng(12).integers(0, spec.vocab, size=40)]
    a = gpu_model(ctx, spec, t, maxlen, max_prefill=40)
    b = gpu_model(ctx, spec, t, maxlen, max_prefill=40)
    b.fold_norm = b.fold_residual = False
    calls = []
    real = q8hip.linear_rmsnorm

    def counted(*args, **kw):
        calls.append(1)
        return real(*args, **kw)

    try:
        q8hip.linear_rmsnorm = counted
        la = a.forward(prompt)
        q8hip.linear_rmsnorm = real
        assert len(calls) == 2 * spec.layers          # q|k|v and gate|up of every block
        lb = b.forward(prompt)
        assert np.all(np.isfinite(la)) and np.array_equal(la, lb)
        la, lb = a.forward([3]), b.forward([3])
        assert np.array_equal(la, lb)
    finally:
        q8hip.linear_rmsnorm = real
        a.close()
        b.close()


def test_fused_model_equals_unfused(ctx):
    """One-row steps with the folded launches give the logits of the
    separate rmsnorm / swiglu / add launches within max-rel-err 1e-5 (the
    norm factor is applied after the GEMV) and the same greedy ids."""
    say("fused model")
    spec, t, inv = tiny_model(seed=7)
    maxlen = 24
    a = gpu_model(ctx, spec, t, maxlen, fuse=True)
    b = gpu_model(ctx, spec, t, maxlen, fuse=False)
    try:
        la, lb = a.forward([5, 6, 7]), b.forward([5, 6, 7])
        assert max_rel_err(la, lb) <= 1e-5
        tok = int(np.argmax(lb))
        for _ in range(5):
            la, lb = a.forward([tok]), b.forward([tok])
            assert np.all(np.isfinite(la)) and max_rel_err(la, lb) <= 1e-5
            assert int(np.argmax(la)) == int(np.argmax(lb))
            tok = int(np.argmax(lb))
    finally:
        a.close()
        b.close()


@pytest.mark.parametrize("G,scale", [(64, "f16"), (32, "f32")])
def test_model_forward_and_greedy_decode(ctx, G, scale):
    say("model", G, scale)
    spec, t, inv = tiny_model(G=G, scale=scale)
    maxlen = 32
    prompt = [3, 14, 15, 92, 65, 35, 89]
    ref = mo.OracleModel(spec, t, inv, maxlen)
    m = gpu_model(ctx, spec, t, maxlen)
    try:
        lg = m.forward(prompt)
        lr = ref.forward(prompt)
        assert max_rel_err(lg, lr) <= 1e-3, max_rel_err(lg, lr)
        # greedy continuation: eager steps, then captured-graph steps
        nxt = int(np.argmax(lg))
        assert nxt == int(np.argmax(lr))
        ids_ref = []
        cur = nxt
        for _ in range(6):
            l = ref.forward([cur])
            cur = int(np.argmax(l))
            ids_ref.append(cur)
        got = [m.forward_argmax([nxt])]
        got += [m.forward_argmax([got[-1]])]
        got += m.decode_steps(got[-1], 4)
        assert got == ids_ref, (got, ids_ref)
    finally:
        m.close()


@pytest.mark.parametrize("G,scale", [(64, "f16"), (32, "f32")])
def test_model_untied_head(ctx, G, scale):
    """A separate lm_head (the Llama-3.1-8B and Qwen3-8B layout,
    llama31_mojo/src/llama_gpu.mojo:142-159): logits within 1e-3 of the
    float64 model, which reads lm_head.weight, not the embedding table, and
    the same greedy ids over eager and captured-graph steps."""
    say("model untied", G, scale)
    spec, t, inv = tiny_model(G=G, scale=scale, seed=11, tied=False)
    assert not np.array_equal(t["lm_head.weight"], t["model.embed_tokens.weight"])
    maxlen = 32
    prompt = [5, 90, 1, 44, 13]
    ref = mo.OracleModel(spec, t, inv, maxlen)
    m = gpu_model(ctx, spec, t, maxlen)
    try:
        lg = m.forward(prompt)
        lr = ref.forward(prompt)
        assert max_rel_err(lg, lr) <= 1e-3, max_rel_err(lg, lr)
        nxt = int(np.argmax(lr))
        assert int(np.argmax(lg)) == nxt
        ids_ref = []
        cur = nxt
        for _ in range(5):
            cur = int(np.argmax(ref.forward([cur])))
            ids_ref.append(cur)
        got = [m.forward_argmax([nxt])]
        got += m.decode_steps(got[-1], 4)
        assert got == ids_ref, (got, ids_ref)
    finally:
        m.close()


@pytest.mark.parametrize("G,scale", [(64, "f16"), (32, "f32")])
def test_model_long_prompt(ctx, G, scale):
    """A 48-token prompt takes the prefill paths (the f16-MFMA dequant-GEMM
    for the linears, the MFMA prompt-row attention): logits within 3e-3 of
    the float64 model (binary16 activations and weights in the GEMM, each
    rounding below 2^-11, compounded over two layers), the same greedy id,
    and the following decode steps (exact f32 GEMVs) on the same ids."""
    say("model long prompt", G, scale)
    spec, t, inv = tiny_model(G=G, scale=scale, seed=9)
    maxlen = 64
    prompt = [int(v) for v in np.random.default_rng(4).integers(0, spec.vocab, size=48)]
    ref = mo.OracleModel(spec, t, inv, maxlen)
    m = gpu_model(ctx, spec, t, maxlen, max_prefill=48)
    try:
        lg = m.forward(prompt)
        lr = ref.forward(prompt)
        err = max_rel_err(lg, lr)
        assert err <= 3e-3, err
        top = np.sort(lr)[-2:]
        if top[1] - top[0] > 1e-2 * np.max(np.abs(lr)):
            assert int(np.argmax(lg)) == int(np.argmax(lr))
    finally:
        m.close()


def test_graph_replay_equals_eager(ctx):
    """The captured step (device position and id) gives the same ids and the
    same logits bits as eager host-position steps."""
    say("graph replay")
    spec, t, inv = tiny_model(seed=5)
    maxlen = 40
    prompt = [1, 2, 3, 4]
    a = gpu_model(ctx, spec, t, maxlen)
    b = gpu_model(ctx, spec, t, maxlen)
    try:
        first = a.forward_argmax(prompt)
        assert b.forward_argmax(prompt) == first
        eager = []
        cur = first
        for _ in range(8):
            cur = a.forward_argmax([cur])
            eager.append(cur)
        graph = b.decode_steps(first, 8)
        assert graph == eager
        # a second replay burst continues from the device position
        more = []
        cur = eager[-1]
        for _ in range(3):
            cur = a.forward_argmax([cur])
            more.append(cur)
        assert b.decode_steps(graph[-1], 3) == more
    finally:
        a.close()
        b.close()



@pytest.mark.parametrize("head_dim,nh,nkv", [(128, 16, 8), (64, 8, 2), (128, 32, 8)])
@pytest.mark.parametrize("pos0", [0, 100, 700])
def test_decode_attention_qk_norm_equals_rmsnorm_rope_attention(ctx, head_dim, nh, nkv, pos0):
    """With q/k norm weights the one-token step writes the cache bits of
    q8_rmsnorm over the head rows + q8_rope_kv, and its output is within
    2e-6 of q8_rmsnorm + q8_rope_kv + q8_attention (1e-5 of float64)."""
    say("decode attention qk-norm", head_dim, nh, nkv, pos0)
    rng = np.random.default_rng(8)
    maxlen, eps = 1024, 1e-6
    qd, kvd = nh * head_dim, nkv * head_dim
    inv = mo.rope_inv_freq(head_dim, 1000000.0)
    cache = rng.standard_normal((2, maxlen, kvd)).astype(np.float16)
    q = (3 * rng.standard_normal(qd)).astype(np.float32)
    k = (3 * rng.standard_normal(kvd)).astype(np.float32)
    v = rng.standard_normal(kvd).astype(np.float32)
    qnw = f32_to_bf16_bits((1 + 0.2 * rng.standard_normal(head_dim)).astype(np.float32))
    knw = f32_to_bf16_bits((1 + 0.2 * rng.standard_normal(head_dim)).astype(np.float32))
    w = ctx.alloc(2 * (64 + 2 * head_dim))
    w.upload(qnw, 2 * 64)
    w.upload(knw, 2 * (64 + head_dim))
    oq, ok, ov, oinv, oy = 0, qd, qd + kvd, qd + 2 * kvd, qd + 2 * kvd + head_dim
    oqn, okn = oy + qd, oy + 2 * qd
    osc = okn + kvd
    a = arena(ctx, osc + q8hip.attention_scratch_floats(1, nh, head_dim, maxlen))
    kv1, kv2 = ctx.alloc(cache.nbytes), ctx.alloc(cache.nbytes)
    kv1.upload(cache)
    kv2.upload(cache)
    for buf, x in [(oq, q), (ok, k), (ov, v), (oinv, inv)]:
        put(a, buf, x)
    q8hip.decode_attention(ctx, a, oq, ok, ov, oinv, kv1, 0, maxlen * kvd, maxlen, oy, pos0, nh,
                           nkv, head_dim, wn=w, oqnorm_u16=64, oknorm_u16=64 + head_dim, eps=eps)
    fused = get(a, oy, (qd,))
    q8hip.rmsnorm(ctx, w, 64, a, oq, oqn, nh, head_dim, eps)
    q8hip.rmsnorm(ctx, w, 64 + head_dim, a, ok, okn, nkv, head_dim, eps)
    qn = get(a, oqn, (1, qd))
    q8hip.rope_kv(ctx, a, oqn, okn, ov, oinv, kv2, 0, maxlen * kvd, maxlen, 1, pos0, nh, nkv,
                  head_dim)
    q8hip.attention(ctx, a, oqn, kv2, 0, maxlen * kvd, maxlen, oy, osc, 1, pos0, nh, nkv,
                    head_dim)
    sep = get(a, oy, (qd,))
    c1 = kv1.download((2, maxlen, kvd), np.float16)
    assert np.array_equal(c1, kv2.download((2, maxlen, kvd), np.float16))
    assert np.all(np.isfinite(fused)) and max_rel_err(fused, sep) <= 2e-6
    qr = mo.rope(mo.head_rmsnorm(q[None].astype(np.float64), qnw, nh, head_dim, eps), pos0, inv,
                 nh, head_dim)
    ref = mo.attention(qr, c1[0].astype(np.float64), c1[1].astype(np.float64), pos0, nh, nkv,
                       head_dim)
    assert max_rel_err(fused, ref[0]) <= 1e-5
    assert max_rel_err(qn[0], mo.head_rmsnorm(q[None].astype(np.float64), qnw, nh, head_dim,
                                               eps)[0]) <= 1e-6
    for b in (a, w, kv1, kv2):
        b.free()


@pytest.mark.parametrize("tokens,heads,hd,ld", [(3, 16, 128, 4096), (40, 8, 128, 2048),
                                                (7, 32, 64, 3072), (5, 4, 128, 0)])
def test_head_rmsnorm_equals_dense_rows(ctx, tokens, heads, hd, ld):
    """q8_head_rmsnorm over the heads inside strided rows (q or k of stacked
    q|k|v) gives each head row the bits q8_rmsnorm gives it as a dense row,
    in place and into another buffer, and leaves the rest of the rows alone."""
    say("head_rmsnorm", tokens, heads, hd, ld)
    rng = np.random.default_rng(tokens * heads)
    width = heads * hd
    L = ld or width
    rows = rng.standard_normal((tokens, L)).astype(np.float32)
    wbits = f32_to_bf16_bits((1 + 0.3 * rng.standard_normal(hd)).astype(np.float32))
    w = ctx.alloc(2 * hd)
    w.upload(wbits)
    dense = np.ascontiguousarray(rows[:, :width]).reshape(tokens * heads, hd)
    od, ody, ox, oy = 0, tokens * width, 2 * tokens * width, 2 * tokens * width + tokens * L
    a = arena(ctx, oy + tokens * L)
    try:
        put(a, od, dense)
        q8hip.rmsnorm(ctx, w, 0, a, od, ody, tokens * heads, hd, 1e-6)
        want = get(a, ody, (tokens, width))
        assert max_rel_err(want, mo.head_rmsnorm(rows[:, :width], wbits, heads, hd, 1e-6)) <= 1e-5
        put(a, ox, rows)
        put(a, oy, np.zeros_like(rows))
        q8hip.head_rmsnorm(ctx, w, 0, a, ox, oy, tokens, heads, hd, ld, 1e-6)
        got = get(a, oy, (tokens, L))
        assert np.array_equal(got[:, :width], want)
        assert not got[:, width:].any()
        q8hip.head_rmsnorm(ctx, w, 0, a, ox, ox, tokens, heads, hd, ld, 1e-6)
        got = get(a, ox, (tokens, L))
        assert np.array_equal(got[:, :width], want)
        assert np.array_equal(got[:, width:], rows[:, width:])
    finally:
        a.free()
        w.free()


def test_qwen_style_model_long_prompt(ctx):
    """A 40-token prompt through a Qwen3-style tiny model (q/k head norms):
    q|k|v as one stacked GEMM whose q and k heads are normalised in place at
    the row stride, the norms in the GEMM pre-passes; logits within 3e-3 of
    the float64 model, and the same bits with the separate norm and add
    launches."""
    say("qwen-style long prompt")
    spec, t, inv = qwen_tiny(seed=13)
    maxlen = 64
    prompt = [int(v) for v in np.random.default_rng(14).integers(0, spec.vocab, size=40)]
    ref = mo.OracleModel(spec, t, inv, maxlen)
    m = gpu_model(ctx, spec, t, maxlen, max_prefill=40)
    u = gpu_model(ctx, spec, t, maxlen, max_prefill=40)
    u.fold_norm = u.fold_residual = False
    try:
        lg, lr = m.forward(prompt), ref.forward(prompt)
        assert max_rel_err(lg, lr) <= 3e-3, max_rel_err(lg, lr)
        assert np.array_equal(u.forward(prompt), lg)
    finally:
        m.close()
        u.close()


def test_qwen_style_model_forward_and_greedy_decode(ctx):
    """Qwen3-style tiny model (q/k head norms, plain RoPE, head_dim 128):
    logits within 1e-3 of the float64 model, the same greedy ids through
    eager steps and graph replays, fused layers within 1e-5 of unfused."""
    say("qwen-style model")
    spec, t, inv = qwen_tiny(seed=6)
    maxlen = 32
    prompt = [7, 1, 8, 2, 8]
    ref = mo.OracleModel(spec, t, inv, maxlen)
    m = gpu_model(ctx, spec, t, maxlen)
    u = gpu_model(ctx, spec, t, maxlen, fuse=False)
    try:
        lg, lr = m.forward(prompt), ref.forward(prompt)
        assert max_rel_err(lg, lr) <= 1e-3, max_rel_err(lg, lr)
        assert max_rel_err(u.forward(prompt), lg) <= 1e-5
        nxt = int(np.argmax(lg))
        assert nxt == int(np.argmax(lr))
        ids_ref, cur = [], nxt
        for _ in range(6):
            cur = int(np.argmax(ref.forward([cur])))
            ids_ref.append(cur)
        got = [m.forward_argmax([nxt])]
        lu = u.forward([nxt])
        got += m.decode_steps(got[-1], 5)
        assert got == ids_ref, (got, ids_ref)
        assert int(np.argmax(lu)) == ids_ref[0]
    finally:
        m.close()
        u.close()


@pytest.mark.parametrize("G,scale", [(64, "f16"), (32, "f32")])
@pytest.mark.parametrize("m,n", [(2048, 128256), (1024, 151936), (512, 5000)])
def test_head_argmax_equals_linear_then_argmax(ctx, G, scale, m, n):
    """q8_head_argmax: the logits of q8_linear_fused (rmsnorm prologue), the
    argmax of q8_argmax on them (also with a tied maximum: the lower index
    wins; and NaN logits give 0), the position step, and the next
    embedding row exactly as q8_embed_gather gives it."""
    say("head_argmax", G, scale, m, n)
    rng = np.random.default_rng(n)
    rs = q8hip.rowstride_u16(m, G, scale)
    wsrc = ctx.alloc(2 * n * m)
    wsrc.upload(f32_to_bf16_bits((0.05 * rng.standard_normal((n, m))).astype(np.float32)))
    emb = n * rs                                     # a second table (the untied case)
    onorm = 2 * n * rs
    w = ctx.alloc(2 * (2 * n * rs + m))
    q8hip.quantize_pack(ctx, wsrc, 0, q8hip.Q8_SRC_BF16, n, m, w, 0, G, scale)
    q8hip.quantize_pack(ctx, wsrc, 0, q8hip.Q8_SRC_BF16, n, m, w, emb, G, scale)
    wsrc.free()
    w.upload(f32_to_bf16_bits((1 + 0.1 * rng.standard_normal(m)).astype(np.float32)), 2 * onorm)
    ox, oy, oy2, onext, oref = 0, m, m + n, m + 2 * n, 2 * m + 2 * n
    a = arena(ctx, 3 * m + 2 * n)
    x = rng.standard_normal(m).astype(np.float32)
    put(a, ox, x)
    ids, pb = ctx.alloc(16), ctx.alloc(16)
    pb.upload(np.array([41, 0, 0, 0], np.int32))
    q8hip.head_argmax(ctx, w, 0, onorm, 1e-5, a, ox, oy, m, n, G, scale, ids, 0, pb, 0, 3, emb,
                      onext)
    got = int(ids.download((1,), np.int32)[0])
    q8hip.linear_fused(ctx, w, 0, a, ox, oy2, m, n, G, scale, q8hip.PRE_RMSNORM, onorm, 1e-5)
    lg = get(a, oy2, (n,))
    assert np.array_equal(get(a, oy, (n,)), lg)
    q8hip.argmax(ctx, a, oy2, n, ids, 1)
    want = int(ids.download((2,), np.int32)[1])
    assert got == want == int(np.argmax(lg))
    assert int(pb.download((1,), np.int32)[0]) == 44
    q8hip.embed_gather(ctx, w, emb, ids, 0, a, oref, 1, m, n, G, scale)
    assert np.array_equal(get(a, onext, (m,)), get(a, oref, (m,)))
    # a tie: copy the winning row to a lower index -> the lower index wins
    if got > 0:
        lo = got // 2
        row = w.download((rs,), np.uint16, 2 * got * rs)
        w.upload(row, 2 * lo * rs)
        q8hip.head_argmax(ctx, w, 0, onorm, 1e-5, a, ox, oy, m, n, G, scale, ids, 0)
        assert int(ids.download((1,), np.int32)[0]) == lo
    # NaN logits (a NaN in x): index 0, as the reference's scan from v[0]
    x[3] = np.nan
    put(a, ox, x)
    q8hip.head_argmax(ctx, w, 0, onorm, 1e-5, a, ox, oy, m, n, G, scale, ids, 0)
    assert int(ids.download((1,), np.int32)[0]) == 0
    for b in (a, w, ids, pb):
        b.free()


def test_fused_graph_decode_equals_unfused_graph(ctx):
    """The captured fused step (lm_head + argmax + position + next embedding
    in two launches) gives the greedy ids of the unfused captured step."""
    say("fused graph")
    spec, t, inv = tiny_model(seed=12)
    a = gpu_model(ctx, spec, t, 32, fuse=True)
    b = gpu_model(ctx, spec, t, 32, fuse=False)
    try:
        first = a.forward_argmax([9, 8, 7])
        assert b.forward_argmax([9, 8, 7]) == first
        assert a.decode_steps(first, 10) == b.decode_steps(first, 10)
        assert int(a.posbuf.download((1,), np.int32)[0]) == 13
    finally:
        a.close()
        b.close()
