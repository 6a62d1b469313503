"""Pins the CPU oracle (oracle/) before anything is compared against it.

Checks, each chosen so that a plausible mistake in the oracle fails it:
  * pack: byte-for-byte against golden vectors written by the reference's own
    pack_q8 (tests/golden/gen_pack_q8_golden.py), for both restatements;
  * f32 -> f16 conversion: against numpy's float16 cast on every rounding
    boundary of every exponent in range, and on random values;
  * pack invariants from the specification (|q| <= 127, a 127 code in every
    normal-scale group, |w - q s| <= s / 2 when not clipped, G32/f32 scale
    equal to max|w| / 127 in f32);
  * linear: float64 closed form against an independent dequantise-then-matmul
    restatement, one-hot inputs (exact), zero input, linearity, and the
    group-major fp32 restatement within f32 rounding;
  * planted mistakes (transposed operand, wrong group scale, dropped scale)
    are rejected by these comparisons.
"""

import numpy as np
import pytest

from oracle.q8_oracle import (abs_packed, bf16_bits_to_f32, elementwise_err, embed_gather_np,
                              linear_f64_np, max_rel_err,
                              pack_q8_np, rowstride_u16, synth_weights_bf16, synth_x,
                              unpack_q8_np)

CASES = ["normal", "sweep", "edge", "tiny", "odd"]


@pytest.mark.parametrize("case", CASES)
def test_numpy_pack_matches_reference_golden(golden, case):
    wi, wo = golden[case + "_in"], golden[case + "_out"]
    got = pack_q8_np(bf16_bits_to_f32(wi))
    assert got.shape == wo.shape
    assert np.array_equal(got, wo)


@pytest.mark.parametrize("case", CASES)
def test_c_pack_matches_reference_golden(golden, cor, case):
    wi, wo = golden[case + "_in"], golden[case + "_out"]
    assert np.array_equal(cor.pack_bf16(wi), wo)
    assert np.array_equal(cor.pack_f32(bf16_bits_to_f32(wi)), wo)


def test_golden_covers_scale_regimes(golden):
    """The fixture exercises zero scales, f16-subnormal scales, normal scales
    and scales that overflow to inf."""
    wo = golden["sweep_out"]
    s = wo[:, :8].reshape(-1)
    assert np.any(s == 0)                                  # scale 0
    assert np.any((s > 0) & (s < 0x0400))                  # subnormal
    assert np.any((s >= 0x0400) & (s < 0x7C00))            # normal
    assert np.any(s == 0x7C00)                             # inf


def _boundary_f32():
    hi = np.arange(2048, dtype=np.uint32) << 12
    lows = np.array([0x000, 0x001, 0x7FF, 0x800, 0x801, 0xFFF], dtype=np.uint32)
    mant = (hi[:, None] | lows[None, :]).reshape(-1)
    exps = np.arange(0x60, 0x91, dtype=np.uint32)
    bits = (exps[:, None] << 23 | mant[None, :]).reshape(-1)
    bits = np.concatenate([bits, bits | 0x80000000])
    extra = np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x477FE000, 0x477FEFFF,
                      0x477FF000, 0x477FF001, 0x33000000, 0x33000001, 0x32FFFFFF,
                      0x387FC000, 0x387FE000, 0x38800000, 0x00000001, 0x007FFFFF],
                     dtype=np.uint32)
    return np.concatenate([bits, extra]).view(np.float32)


def test_c_f16_conversion_matches_numpy_on_boundaries(cor):
    x = _boundary_f32()
    with np.errstate(over="ignore"):          # values past 65504 round to inf
        want = x.astype(np.float16).view(np.uint16)
    got = cor.f32_to_f16_array(x)
    assert np.array_equal(got, want)


def test_c_f16_conversion_matches_numpy_random(cor):
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2**32, size=4_000_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[~np.isnan(x)]
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(cor.f32_to_f16_array(x), want)


def test_c_f16_to_f32_exhaustive(cor):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = cor.f16_to_f32_array(h)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


@pytest.mark.parametrize("G,scale", [(64, "f16"), (32, "f32"), (32, "f16"), (64, "f32")])
def test_pack_invariants(cor, G, scale):
    rng = np.random.default_rng(11)
    w = (rng.standard_normal((64, 1024)).astype(np.float32)
         * np.exp(rng.uniform(-8, 4, (64, 1))).astype(np.float32))
    pk = cor.pack_f32(w, G, scale)
    assert np.array_equal(pk, pack_q8_np(w, G, scale))
    codes, s = unpack_q8_np(pk, 1024, G, scale)
    assert np.all(np.abs(codes.astype(np.int32)) <= 127)
    sg = np.repeat(s, G, axis=1)
    gmax = np.abs(codes.reshape(64, -1, G)).max(axis=2)
    if scale == "f16":
        normal = s >= np.float32(2.0 ** -14)
        assert np.all(gmax[normal] == 127)
    else:
        amax = np.abs(w.reshape(64, -1, G)).max(axis=2)
        want = np.maximum(amax / np.float32(127.0), np.float32(1e-8)).astype(np.float32)
        assert np.array_equal(s.view(np.uint32), want.view(np.uint32))
        assert np.all(gmax == 127)
    unclipped = np.abs(codes) < 127
    err = np.abs(w.astype(np.float64) - codes.astype(np.float64) * sg)
    assert np.all(err[unclipped] <= 0.5 * sg[unclipped] * (1 + 2.0 ** -22))


def test_rint_is_half_to_even(cor):
    # scale exactly 1.0 (absmax 127): x/1 = x, so codes are rint of the inputs.
    vals = np.array([127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, 126.5, -126.5],
                    dtype=np.float32)
    w = np.zeros((1, 64), dtype=np.float32)
    w[0, : vals.size] = vals
    codes, s = unpack_q8_np(cor.pack_f32(w), 64)
    assert s[0, 0] == 1.0
    assert list(codes[0, : vals.size]) == [127, 0, 2, 2, 0, -2, -2, 4, 126, -126]


def test_scale_zero_group_codes(cor):
    # absmax below ~3.78e-6 gives an f16 scale of 0: nonzero weights clip to
    # +-127 (x / 0 = +-inf) and zeros give 0 (0 / 0 = NaN -> 0).
    w = np.zeros((1, 64), dtype=np.float32)
    w[0, :3] = [2e-6, -1e-6, 0.0]
    codes, s = unpack_q8_np(cor.pack_f32(w), 64)
    assert s[0, 0] == 0.0
    assert list(codes[0, :4]) == [127, -127, 0, 0]


@pytest.mark.parametrize("G,scale", [(64, "f16"), (32, "f32")])
def test_linear_f64_closed_form(cor, G, scale):
    wb = synth_weights_bf16(96, 512, seed=3)
    pk = cor.pack_bf16(wb, G, scale)
    x = synth_x(5, 512, seed=4)
    y = cor.linear_f64(pk, x, G, scale)
    y2 = linear_f64_np(pk, x, 512, G, scale)
    assert max_rel_err(y, y2) < 1e-12


@pytest.mark.parametrize("G,scale", [(64, "f16"), (32, "f32")])
def test_linear_f64x_closed_form(cor, G, scale):
    """The float64-input closed form: the bits of the f32-input one on f32
    values (same float64 sums in the same order), and within 1e-12 of the
    dequantise-then-matmul form on inputs that need all 53 bits."""
    wb = synth_weights_bf16(96, 512, seed=3)
    pk = cor.pack_bf16(wb, G, scale)
    x = synth_x(5, 512, seed=4)
    assert np.array_equal(cor.linear_f64x(pk, x.astype(np.float64), G, scale),
                          cor.linear_f64(pk, x, G, scale))
    xd = np.random.default_rng(5).standard_normal((3, 512)) * np.pi
    assert not np.array_equal(xd, xd.astype(np.float32).astype(np.float64))
    assert max_rel_err(cor.linear_f64x(pk, xd, G, scale), linear_f64_np(pk, xd, 512, G, scale)) \
        < 1e-12


@pytest.mark.parametrize("G,scale", [(64, "f16"), (32, "f32")])
def test_abs_packed_and_elementwise_err(cor, G, scale):
    """abs_packed dequantises to |deq(W)| (every code and scale sign
    removed, nothing else changed), so linear_abs equals |x| . |deq(W)|^T;
    elementwise_err measures each output against that scale."""
    wb = synth_weights_bf16(64, 512, seed=31)
    pk = cor.pack_bf16(wb, G, scale)
    codes, s = unpack_q8_np(pk, 512, G, scale)
    assert (codes < 0).any() and (s >= 0).all()      # pack_q8's scales are absmax / 127
    ac, asc = unpack_q8_np(abs_packed(pk, 512, G, scale), 512, G, scale)
    assert np.array_equal(ac, np.abs(codes)) and np.array_equal(asc, np.abs(s))
    x = synth_x(3, 512, seed=32)
    want = np.abs(x).astype(np.float64) @ (np.abs(codes).astype(np.float64) *
                                           np.repeat(np.abs(s).astype(np.float64), G, axis=1)).T
    got = cor.linear_abs(pk, x, G, scale)
    assert max_rel_err(got, want) < 1e-12
    y = cor.linear_f64(pk, x, G, scale)
    assert np.all(got >= np.abs(y))
    assert elementwise_err(y, y, got) == 0.0
    bumped = y.copy()
    bumped[1, 7] += 1e-3 * got[1, 7]
    assert abs(elementwise_err(bumped, y, got) - 1e-3) < 1e-9


@pytest.mark.parametrize("G,scale", [(64, "f16"), (32, "f32")])
def test_linear_one_hot_is_exact(cor, G, scale):
    wb = synth_weights_bf16(40, 256, seed=5)
    pk = cor.pack_bf16(wb, G, scale)
    codes, s = unpack_q8_np(pk, 256, G, scale)
    ks = [0, 1, 63, 64, 130, 255]
    x = np.zeros((len(ks), 256), dtype=np.float32)
    for i, k in enumerate(ks):
        x[i, k] = 1.0
    y64 = cor.linear_f64(pk, x, G, scale)
    y32 = cor.linear_f32(pk, x, G, scale)
    for i, k in enumerate(ks):
        want = codes[:, k].astype(np.float32) * s[:, k // G]
        assert np.array_equal(y64[i].astype(np.float32), want)
        assert np.array_equal(y32[i], want)


def test_linear_zero_and_linearity(cor):
    wb = synth_weights_bf16(64, 512, seed=6)
    pk = cor.pack_bf16(wb)
    z = np.zeros((2, 512), dtype=np.float32)
    assert np.all(cor.linear_f64(pk, z) == 0.0)
    x1, x2 = synth_x(1, 512, 7), synth_x(1, 512, 8)
    a, b = np.float32(0.75), np.float32(-2.0)
    y = cor.linear_f64(pk, (a * x1 + b * x2).astype(np.float32))
    y12 = a * cor.linear_f64(pk, x1) + b * cor.linear_f64(pk, x2)
    assert max_rel_err(y, y12) < 1e-6


@pytest.mark.parametrize("G,scale", [(64, "f16"), (32, "f32")])
def test_group_major_f32_within_rounding(cor, G, scale):
    wb = synth_weights_bf16(128, 2048, seed=9)
    pk = cor.pack_bf16(wb, G, scale)
    x = synth_x(2, 2048, seed=10)
    assert max_rel_err(cor.linear_f32(pk, x, G, scale), cor.linear_f64(pk, x, G, scale)) < 1e-5


def test_embed_gather_oracle(cor):
    wb = synth_weights_bf16(50, 256, seed=12)
    for G, scale in [(64, "f16"), (32, "f32")]:
        pk = cor.pack_bf16(wb, G, scale)
        ids = np.array([0, 49, 7, 7, 23], dtype=np.int32)
        got = cor.embed_gather(pk, ids, 256, G, scale)
        want = embed_gather_np(pk, ids, 256, G, scale)
        assert np.array_equal(got, want)


def test_planted_mistakes_are_caught(cor):
    """Mistakes one could make in a restatement fail the closed-form check."""
    G, m, n = 64, 512, 64
    wb = synth_weights_bf16(n, m, seed=13)
    pk = cor.pack_bf16(wb)
    codes, s = unpack_q8_np(pk, m)
    x = synth_x(3, m, seed=14).astype(np.float64)
    ref = cor.linear_f64(pk, x.astype(np.float32))
    sg = np.repeat(s, G, axis=1).astype(np.float64)
    good = x @ (codes * sg).T
    assert max_rel_err(good, ref) < 1e-12
    wrong_group = x @ (codes * np.roll(sg, G, axis=1)).T          # scale of group g-1
    no_scale = x @ codes.astype(np.float64).T                     # dropped scale
    w_sq = (codes * sg)[:, :n]                                    # transposed operand
    transposed = x[:, :n] @ w_sq
    for bad in (wrong_group, no_scale / np.abs(no_scale).max() * np.abs(ref).max()):
        assert max_rel_err(bad, ref) > 1e-2
    assert max_rel_err(transposed, x[:, :n] @ w_sq.T) > 1e-2


def test_rowstride():
    assert rowstride_u16(2048) == 1056            # src/llama_q8.mojo:26-28
    assert rowstride_u16(8192) == 4224
    assert rowstride_u16(2048, 32, "f32") == 1152
