"""GPU parity: libq8hip.so (through its C ABI) against the CPU oracle.

Bars (written in each test):
  * pack: codes and scales bit-exact (reference golden vectors and oracle);
  * linear / GEMM: normwise max relative error  max|y - y*| / max|y*|
    <= 1e-3 against the float64 closed form over the same codes, scales and
    (bf16-rounded, for bf16 activations) inputs; elementwise, each output
    against its own scale sum_k |x_k||w_k| (elementwise_err), <= 1e-5 on the
    f32 paths (s < 32) and <= 1e-3 on the f16-MFMA GEMM;
  * one-hot inputs, fused-vs-separate calls and embedding gathers: bit-exact.
"""

import sys

import numpy as np
import pytest

from lama32_mojo_amd import q8, q8hip
from oracle.q8_oracle import (bf16_bits_to_f32, elementwise_err, f32_to_bf16_bits, max_rel_err,
                              rowstride_u16, synth_weights_bf16, synth_x, unpack_q8_np)

pytestmark = pytest.mark.gpu
TOL = 1e-3
LAYOUTS = [(64, "f16"), (32, "f32")]


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def upload(ctx, arr):
    arr = np.ascontiguousarray(arr)
    b = ctx.alloc(max(arr.nbytes, 16))
    b.upload(arr)
    return b


def gpu_linear(ctx, pk, x, G, scale, owt=0, pad_x=0):
    """Run q8_linear on packed rows pk [n, rs] and x [s, m]; returns y [s, n]."""
    n, rs = pk.shape
    s, m = x.shape
    wbuf = np.zeros(owt + n * rs, dtype=np.uint16)
    wbuf[owt:] = pk.reshape(-1)
    w = upload(ctx, wbuf)
    ox = pad_x
    oy = ox + s * m
    a = ctx.alloc(4 * (oy + s * n))
    a.upload(np.ascontiguousarray(x, dtype=np.float32), 4 * ox)
    q8hip.linear(ctx, w, owt, a, ox, oy, s, m, n, G, scale)
    y = a.download((s, n), np.float32, 4 * oy)
    w.free()
    a.free()
    return y


def gpu_linear_bf16(ctx, pk, xbits, G, scale):
    n, rs = pk.shape
    s, m = xbits.shape
    w = upload(ctx, pk)
    xb = upload(ctx, xbits)
    yb = ctx.alloc(4 * s * n)
    q8hip.linear_bf16act(ctx, w, 0, xb, 0, yb, 0, s, m, n, G, scale)
    y = yb.download((s, n), np.float32)
    for b in (w, xb, yb):
        b.free()
    return y


# ---------------------------------------------------------------------------
# quantize / pack
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("case", ["normal", "sweep", "edge", "tiny", "odd"])
def test_pack_matches_reference_golden(ctx, golden, case):
    say("pack golden", case)
    wi, wo = golden[case + "_in"], golden[case + "_out"]
    got = q8.pack_q8_bits(wi, 64, "f16", ctx)
    assert np.array_equal(got, wo), np.argwhere(got != wo)[:5]


@pytest.mark.parametrize("G,scale", LAYOUTS + [(32, "f16"), (64, "f32")])
@pytest.mark.parametrize("src", ["bf16", "f32"])
def test_pack_matches_oracle_llama_up_proj(ctx, cor, G, scale, src):
    say("pack 8192x2048", G, scale, src)
    wb = synth_weights_bf16(8192, 2048, seed=0)
    if src == "bf16":
        got = q8.pack_q8_bits(wb, G, scale, ctx)
    else:
        got = q8.pack_q8_bits(bf16_bits_to_f32(wb), G, scale, ctx, src_dtype="f32")
    want = cor.pack_bf16(wb, G, scale)
    assert np.array_equal(got, want)


def test_pack_f32_wide_dynamic_range(ctx, cor):
    """f32 inputs that are not bf16 values, spanning many binades."""
    say("pack f32 wide range")
    rng = np.random.default_rng(21)
    w = (rng.standard_normal((257, 512)).astype(np.float32)
         * np.exp(rng.uniform(-20, 12, (257, 1))).astype(np.float32))
    for G, scale in LAYOUTS:
        got = q8.pack_q8_bits(w, G, scale, ctx, src_dtype="f32")
        assert np.array_equal(got, cor.pack_f32(w, G, scale))


def test_pack_unaligned_offsets(ctx, cor):
    """Odd source / destination offsets take the scalar load paths."""
    say("pack unaligned")
    n, m = 33, 192
    wb = synth_weights_bf16(n, m, seed=22)
    rs = rowstride_u16(m)
    src = upload(ctx, np.concatenate([np.zeros(3, np.uint16), wb.reshape(-1)]))
    dst = ctx.alloc(2 * (5 + n * rs))
    q8hip.quantize_pack(ctx, src, 3, q8hip.Q8_SRC_BF16, n, m, dst, 5, 64, "f16")
    got = dst.download((n, rs), np.uint16, 10)
    assert np.array_equal(got, cor.pack_bf16(wb))
    src.free()
    dst.free()


# ---------------------------------------------------------------------------
# decode GEMV (q8_linear, small s)
# ---------------------------------------------------------------------------

# (n, m): the Llama-3.2-1B decode projections (gate|up 16384, up 8192,
# q|k|v 3072, o 2048, down 2048 x 8192) and ragged ones
SHAPES = [(8192, 2048), (3072, 2048), (2048, 2048), (16384, 2048), (2048, 8192), (1000, 1536),
          (1, 64), (7, 96)]


def layout_shapes(shapes, m_index):
    """(G, scale, *shape) for every layout whose group size divides the
    shape's m (a packed row holds whole groups)."""
    return [(G, scale, *sh) for sh in shapes for G, scale in LAYOUTS if sh[m_index] % G == 0]


@pytest.mark.parametrize("G,scale,n,m", layout_shapes(SHAPES, 1))
@pytest.mark.parametrize("s", [1, 2, 3, 4, 5, 8, 9, 16, 24])
def test_linear_matches_closed_form(ctx, cor, G, scale, n, m, s):
    say("linear", G, scale, n, m, s)
    wb = synth_weights_bf16(n, m, seed=n + m)
    pk = cor.pack_bf16(wb, G, scale)
    x = synth_x(s, m, seed=s)
    y = gpu_linear(ctx, pk, x, G, scale)
    ref = cor.linear_f64(pk, x, G, scale)
    err = max_rel_err(y, ref)
    assert err <= TOL, err
    assert err <= 1e-5, err      # fp32 accumulation is far inside the bar
    ew = elementwise_err(y, ref, cor.linear_abs(pk, x, G, scale))
    assert ew <= 1e-5, ew


@pytest.mark.parametrize("G,scale,n,m", [(32, "f32", 4099, 640), (32, "f32", 16386, 640),
                                         (64, "f16", 8195, 1536), (32, "f32", 24, 12288),
                                         (64, "f16", 16384, 512), (64, "f16", 16400, 1536),
                                         (32, "f32", 65600, 1024)])
@pytest.mark.parametrize("s", [2, 4, 6, 7, 8, 16, 23])
def test_few_rows_ragged(ctx, cor, G, scale, n, m, s):
    """2 <= s <= 23 rows (the f32 4x4-block kernels up to 4 rows, the split
    bf16 kernels above; K split over the waves below n = 16384, shared x
    from there): ragged weight-row blocks (n not a multiple of the block's
    rows, whole waves past n), K ending inside a 256-code slab, odd and even
    slab counts, long K; the error stays at f32 accumulation level."""
    say("few rows", G, scale, n, m, s)
    wb = synth_weights_bf16(n, m, seed=n + s)
    pk = cor.pack_bf16(wb, G, scale)
    x = synth_x(s, m, seed=40 + s)
    y = gpu_linear(ctx, pk, x, G, scale)
    ref = cor.linear_f64(pk, x, G, scale)
    err = max_rel_err(y, ref)
    assert err <= 1e-5, err
    # row-wise too: every batch row, not only the largest
    for b in range(s):
        assert max_rel_err(y[b], ref[b]) <= 1e-5, b


@pytest.mark.parametrize("G,scale", LAYOUTS)
def test_linear_one_hot_exact(ctx, cor, G, scale):
    say("linear one-hot", G, scale)
    n, m = 512, 2048
    pk = cor.pack_bf16(synth_weights_bf16(n, m, seed=31), G, scale)
    codes, sc = unpack_q8_np(pk, m, G, scale)
    for k in [0, 17, 1023, 1024, 2047]:
        x = np.zeros((1, m), dtype=np.float32)
        x[0, k] = 1.0
        y = gpu_linear(ctx, pk, x, G, scale)
        want = codes[:, k].astype(np.float32) * sc[:, k // G]
        assert np.array_equal(y[0], want)


def ones_packed(n, m, G, scale):
    """Packed rows whose codes are all 1 and whose scales are all 1.0."""
    ng = m // G
    if scale == "f16":
        sc = np.full((n, ng), 1.0, np.float16).view(np.uint16)
    else:
        sc = np.full((n, ng), 1.0, np.float32).view(np.uint16).reshape(n, 2 * ng)
    codes = np.ones((n, m), np.int8).view(np.uint16).reshape(n, m // 2)
    pk = np.concatenate([sc, codes], axis=1)
    assert pk.shape[1] == rowstride_u16(m, G, scale)
    return pk


@pytest.mark.parametrize("G,scale", LAYOUTS)
@pytest.mark.parametrize("s", [1, 3, 8, 40])
def test_linear_all_ones_gives_row_sums(ctx, cor, G, scale, s):
    """Codes all 1 with scales 1.0: every output is sum(x) of its row (the
    s = 1 GEMV, both small-batch kernels and the GEMM).  x >= 0, so the sum
    is well conditioned: the f32 paths stay within 1e-5 of it, the GEMM
    (binary16 copy of x, 2^-12 per element) within 3e-4.  Columns with
    equal weights take equal steps, so each row's outputs are all equal."""
    say("all ones", G, scale, s)
    n, m = 300, 4096
    pk = ones_packed(n, m, G, scale)
    codes, sc = unpack_q8_np(pk, m, G, scale)
    assert np.all(codes == 1) and np.all(sc == 1.0)
    x = np.random.default_rng(50 + s).random((s, m), dtype=np.float32)
    y = gpu_linear(ctx, pk, x, G, scale)
    want = x.astype(np.float64).sum(axis=1)
    tol = 1e-5 if s < 32 else 3e-4
    assert np.all(np.abs(y - want[:, None]) <= tol * want[:, None]), np.abs(y / want[:, None] - 1).max()
    assert np.all(y == y[:, :1])


@pytest.mark.parametrize("s,n,m", [(16, 4096, 12288), (8, 24, 12288), (6, 2000, 8192),
                                   (512, 2048, 2048), (64, 2048, 8192), (40, 24, 4096)])
def test_split_k_across_workgroups_repeats_bitwise(ctx, cor, s, n, m):
    """Long rows at 5..16 activation rows split K over workgroups, and GEMMs
    whose output tiles alone leave CUs idle (512x2048x2048: 4 K splits;
    64x2048x8192: 16; 40x24x4096: 8 splits of one ragged tile) split K too;
    both add the partials in a fixed order in a reduce launch: repeated
    calls give the same bits and match the closed form (1e-5 on the f32
    paths, 1e-3 through binary16 weights)."""
    say("split-K repeats", s, n, m)
    G, scale = 32, "f32"
    pk = cor.pack_bf16(synth_weights_bf16(n, m, seed=60 + s), G, scale)
    x = synth_x(s, m, seed=61)
    w = upload(ctx, pk)
    a = ctx.alloc(4 * (s * m + s * n))
    a.upload(np.ascontiguousarray(x, dtype=np.float32))
    ys = []
    for _ in range(4):
        q8hip.linear(ctx, w, 0, a, 0, s * m, s, m, n, G, scale)
        ys.append(a.download((s, n), np.float32, 4 * s * m))
    w.free()
    a.free()
    for y in ys[1:]:
        assert np.array_equal(y, ys[0])
    assert max_rel_err(ys[0], cor.linear_f64(pk, x, G, scale)) <= (1e-5 if s < 32 else 1e-3)


def test_linear_zero_input(ctx, cor):
    pk = cor.pack_bf16(synth_weights_bf16(300, 512, seed=32))
    y = gpu_linear(ctx, pk, np.zeros((2, 512), np.float32), 64, "f16")
    assert np.all(y == 0.0)


@pytest.mark.parametrize("G,scale", LAYOUTS)
def test_fused_qkv_equals_separate_calls(ctx, cor, G, scale):
    """run_layer_q8 fuses q|k|v into one call over contiguous rows
    (src/llama_q8.mojo:163-166); every output is independent, so the fused
    result equals the separate calls bit for bit."""
    say("fused qkv", G, scale)
    H, QD, KVD = 2048, 2048, 512
    rs = rowstride_u16(H, G, scale)
    pk = cor.pack_bf16(synth_weights_bf16(QD + 2 * KVD, H, seed=33), G, scale)
    w = upload(ctx, pk)
    x = synth_x(1, H, seed=34)
    a = ctx.alloc(4 * (H + 2 * (QD + 2 * KVD)))
    a.upload(x)
    q8hip.linear(ctx, w, 0, a, 0, H, 1, H, QD + 2 * KVD, G, scale)
    o = H + QD + 2 * KVD
    q8hip.linear(ctx, w, 0, a, 0, o, 1, H, QD, G, scale)
    q8hip.linear(ctx, w, QD * rs, a, 0, o + QD, 1, H, KVD, G, scale)
    q8hip.linear(ctx, w, (QD + KVD) * rs, a, 0, o + QD + KVD, 1, H, KVD, G, scale)
    fused = a.download((QD + 2 * KVD,), np.float32, 4 * H)
    sep = a.download((QD + 2 * KVD,), np.float32, 4 * o)
    assert np.array_equal(fused, sep)
    w.free()
    a.free()


@pytest.mark.parametrize("G,scale", LAYOUTS)
def test_linear_unaligned_weights(ctx, cor, G, scale):
    """A weight offset that is not 16-byte aligned takes the generic kernel."""
    say("linear unaligned", G, scale)
    n, m = 130, 512
    pk = cor.pack_bf16(synth_weights_bf16(n, m, seed=35), G, scale)
    x = synth_x(3, m, seed=36)
    y = gpu_linear(ctx, pk, x, G, scale, owt=3, pad_x=1)
    assert max_rel_err(y, cor.linear_f64(pk, x, G, scale)) <= TOL


def test_linear_lm_head_full_size(ctx, cor):
    """Llama-3.2-1B tied lm_head, 128256 x 2048, s = 1."""
    say("lm_head full size")
    n, m = 128256, 2048
    pk = cor.pack_bf16(synth_weights_bf16(n, m, seed=37))
    x = synth_x(1, m, seed=38)
    y = gpu_linear(ctx, pk, x, 64, "f16")
    ref = cor.linear_f64(pk, x)
    assert max_rel_err(y, ref) <= TOL
    assert np.argmax(y[0]) == np.argmax(ref[0])


# ---------------------------------------------------------------------------
# prefill GEMM (MFMA)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("G,scale,s,n,m", layout_shapes(
    [(512, 2048, 2048), (512, 512, 2048), (512, 8192, 2048), (512, 2048, 8192), (77, 200, 1024),
     (130, 96, 96), (1, 64, 64), (512, 3072, 2048), (200, 1000, 4096), (100, 200, 1056)], 2))
def test_gemm_bf16act_matches_closed_form(ctx, cor, G, scale, s, n, m):
    say("gemm bf16", G, scale, s, n, m)
    pk = cor.pack_bf16(synth_weights_bf16(n, m, seed=n + 3 * m), G, scale)
    xbits = f32_to_bf16_bits(synth_x(s, m, seed=s + 1))
    y = gpu_linear_bf16(ctx, pk, xbits, G, scale)
    ref = cor.linear_f64(pk, bf16_bits_to_f32(xbits), G, scale)
    err = max_rel_err(y, ref)
    assert err <= TOL, err
    ew = elementwise_err(y, ref, cor.linear_abs(pk, bf16_bits_to_f32(xbits), G, scale))
    assert ew <= TOL, ew


@pytest.mark.parametrize("G,scale", LAYOUTS)
@pytest.mark.parametrize("s", [32, 64, 512])
def test_gemm_f32act_matches_closed_form(ctx, cor, G, scale, s):
    """q8_linear with many activation rows runs the dequant-GEMM on f16
    MFMA: activations rounded once to binary16 after a power-of-two row
    scaling, weights q * s rounded to binary16 (s itself first when it is
    f32).  Each rounding is below 2^-11 relative and they do not add up
    coherently, so the normwise error stays near 2e-4, well inside 1e-3."""
    say("gemm f32", G, scale, s)
    n, m = 1024, 2048
    pk = cor.pack_bf16(synth_weights_bf16(n, m, seed=41), G, scale)
    x = synth_x(s, m, seed=42)
    y = gpu_linear(ctx, pk, x, G, scale)
    ref = cor.linear_f64(pk, x, G, scale)
    err = max_rel_err(y, ref)
    assert err <= TOL, err
    assert err <= 5e-4, err
    ew = elementwise_err(y, ref, cor.linear_abs(pk, x, G, scale))
    assert ew <= TOL, ew


@pytest.mark.parametrize("bf16", [False, True])
def test_gemm_rows_of_any_size(ctx, cor, bf16):
    """Each activation row enters binary16 after its own power-of-two
    scaling, so rows from 1e-30 to 1e30 in size (far outside binary16's
    range either way), an all-zero row and ordinary rows in one call are
    each within 5e-4 of float64, row by row."""
    say("gemm row scales", bf16)
    n, m, s = 192, 1024, 40
    pk = cor.pack_bf16(synth_weights_bf16(n, m, seed=44))
    x = synth_x(s, m, seed=45)
    sizes = np.array([1.0, 1e-30, 1e30, 1e-6, 3e4, 0.0, 1e6, 0.5])
    x = (x * sizes[np.arange(s) % len(sizes)][:, None]).astype(np.float32)
    if bf16:
        xbits = f32_to_bf16_bits(x)
        y = gpu_linear_bf16(ctx, pk, xbits, 64, "f16")
        x = bf16_bits_to_f32(xbits)
    else:
        y = gpu_linear(ctx, pk, x, 64, "f16")
    ref = cor.linear_f64(pk, x)
    for i in range(s):
        assert max_rel_err(y[i], ref[i]) <= 5e-4, (i, sizes[i % len(sizes)])


def test_gemm_bf16act_one_hot_exact(ctx, cor):
    n, m, s = 256, 512, 64
    pk = cor.pack_bf16(synth_weights_bf16(n, m, seed=43))
    codes, sc = unpack_q8_np(pk, m)
    ks = np.arange(s) * 7 % m
    x = np.zeros((s, m), dtype=np.float32)
    x[np.arange(s), ks] = 1.0
    y = gpu_linear_bf16(ctx, pk, f32_to_bf16_bits(x), 64, "f16")
    # a one-hot row reads back one dequantized weight: binary16 q * s, one
    # rounding (numpy's float16 product of two float16 values rounds once)
    w16 = codes[:, ks].astype(np.float16) * sc[:, ks // 64].astype(np.float16)
    assert np.array_equal(y, w16.astype(np.float32).T)


# ---------------------------------------------------------------------------
# embedding gather
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("G,scale", LAYOUTS)
def test_embed_gather_exact(ctx, cor, G, scale):
    say("embed", G, scale)
    vocab, d = 1000, 2048
    pk = cor.pack_bf16(synth_weights_bf16(vocab, d, seed=51), G, scale)
    w = upload(ctx, pk)
    ids = np.array([0, 999, 5, 5, 123, 7], dtype=np.int32)
    ib = upload(ctx, ids)
    a = ctx.alloc(4 * len(ids) * d)
    q8hip.embed_gather(ctx, w, 0, ib, 0, a, 0, len(ids), d, vocab, G, scale)
    got = a.download((len(ids), d), np.float32)
    assert np.array_equal(got, cor.embed_gather(pk, ids, d, G, scale))
    bad = upload(ctx, np.array([3, -1, vocab], dtype=np.int32))
    q8hip.embed_gather(ctx, w, 0, bad, 0, a, 0, 3, d, vocab, G, scale)
    got = a.download((3, d), np.float32)
    assert np.array_equal(got[0], cor.embed_gather(pk, np.array([3], np.int32), d, G, scale)[0])
    assert np.all(np.isnan(got[1:]))
    for b in (w, ib, a, bad):
        b.free()


# ---------------------------------------------------------------------------
# host mirror + graphs
# ---------------------------------------------------------------------------

def test_mm_q8_op_and_graph_replay(ctx, cor):
    """mm_q8_op through the arenas, captured in a HIP graph and replayed with
    new inputs written eagerly between replays; every replay matches the
    eager result."""
    say("graph replay")
    H, N = 2048, 3072
    pk = cor.pack_bf16(synth_weights_bf16(N, H, seed=61))
    w = q8.Weights(ctx, q8.PAD + pk.size)
    w.upload_all({"wq": pk}, ["wq"])
    a = q8.Acts(ctx, q8.PAD + H + 2 * N + 64)
    qk = q8.Q8Kernels(ctx)
    ox = a.alloc(H)
    ctx.graph_begin()
    oy = q8.mm_q8_op(ctx, w, a, qk, ox, 1, H, w.o("wq"), N)
    g = ctx.graph_end()
    for rep in range(4):
        x = synth_x(1, H, seed=70 + rep)
        a.write(ox, x)
        g.launch()
        ctx.sync()
        got = a.read(oy, N)
        emark = a.mark()
        oe = q8.mm_q8_op(ctx, w, a, qk, ox, 1, H, w.o("wq"), N)
        ctx.sync()
        eager = a.read(oe, N)
        a.reset(emark)
        assert oe != oy
        assert np.array_equal(got, eager)
        assert max_rel_err(got, cor.linear_f64(pk, x)[0]) <= TOL
    g.destroy()


def test_pack_q8_torch_signature(ctx, golden):
    import torch
    wi, wo = golden["normal_in"], golden["normal_out"]
    t = torch.from_numpy(wi.view(np.int16).copy()).view(torch.bfloat16)
    out = q8.pack_q8(t, ctx=ctx)
    assert out.dtype == torch.float16 and tuple(out.shape) == wo.shape
    assert np.array_equal(out.numpy().view(np.uint16), wo)
