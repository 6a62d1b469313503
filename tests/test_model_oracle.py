"""Pins of the CPU model oracle (oracle/model_oracle.py) by closed forms and
invariants -- no GPU.  Each check is chosen so a plausible slip (a sign in
RoPE, a wrong GQA head map, a dropped causal mask, a missing eps) fails it."""

import numpy as np

from oracle import model_oracle as mo
from oracle.q8_oracle import bf16_bits_to_f32, f32_to_bf16_bits, pack_q8_np, synth_weights_bf16


def bf16_ones(d, scale=1.0):
    return f32_to_bf16_bits(np.full(d, scale, dtype=np.float32))


def test_rmsnorm_constant_rows_and_scale_invariance():
    d, eps = 64, 1e-5
    w = bf16_ones(d)
    for c in [3.0, -0.5]:
        y = mo.rmsnorm(np.full((1, d), c), w, eps)
        np.testing.assert_allclose(y, c / np.sqrt(c * c + float(np.float32(eps))), rtol=1e-12)
    x = np.random.default_rng(0).standard_normal((3, d))
    np.testing.assert_allclose(mo.rmsnorm(1e3 * x, w, 0.0), mo.rmsnorm(x, w, 0.0), rtol=1e-12)
    wd = f32_to_bf16_bits(np.linspace(0.5, 2.0, d).astype(np.float32))
    np.testing.assert_allclose(mo.rmsnorm(x, wd, 0.0),
                               mo.rmsnorm(x, w, 0.0) * np.linspace(0.5, 2.0, d).astype(np.float32),
                               rtol=1e-2)


def test_llama3_inv_freq_regimes():
    hd, theta, factor, low, high, orig = 128, 500000.0, 8.0, 1.0, 4.0, 8192.0
    inv = mo.llama3_inv_freq(hd, theta, factor, low, high, orig)
    base = np.array([1.0 / theta ** (2 * d / hd) for d in range(hd // 2)])
    wl = 2 * np.pi / base
    hi = wl < orig / high            # short wavelengths: unchanged
    lo = wl > orig / low             # long wavelengths: divided by the factor
    np.testing.assert_allclose(inv[hi], base[hi].astype(np.float32), rtol=1e-7)
    np.testing.assert_allclose(inv[lo], (base[lo] / factor).astype(np.float32), rtol=1e-7)
    mid = ~hi & ~lo
    assert np.all(inv[mid] <= base[mid] * (1 + 1e-6)) and np.all(inv[mid] >= base[mid] / factor * (1 - 1e-6))
    # factor 1 is plain RoPE
    np.testing.assert_allclose(mo.llama3_inv_freq(hd, theta, 1.0, low, high, orig),
                               base.astype(np.float32), rtol=1e-7)


def test_rope_identity_rotation_sign_and_composition():
    rng = np.random.default_rng(1)
    nh, hd = 3, 8
    x = rng.standard_normal((1, nh * hd))
    inv = np.linspace(0.1, 1.0, hd // 2).astype(np.float32)
    np.testing.assert_allclose(mo.rope(x, 0, inv, nh, hd), x, rtol=0, atol=0)
    # pairs keep their norm
    y = mo.rope(x, 7, inv, nh, hd).reshape(nh, hd)
    xr = x.reshape(nh, hd)
    h = hd // 2
    np.testing.assert_allclose(y[:, :h] ** 2 + y[:, h:] ** 2, xr[:, :h] ** 2 + xr[:, h:] ** 2,
                               rtol=1e-12)
    # angle pi/2 (inv = pi/2 at pos 1): (x0, x1) -> (-x1, x0)
    one = np.zeros((1, 2))
    one[0] = [1.0, 0.0]
    r = mo.rope(one, 1, np.array([np.float32(np.pi / 2)]), 1, 2)
    np.testing.assert_allclose(r, [[0.0, 1.0]], atol=1e-7)
    r = mo.rope(np.array([[0.0, 1.0]]), 1, np.array([np.float32(np.pi / 2)]), 1, 2)
    np.testing.assert_allclose(r, [[-1.0, 0.0]], atol=1e-7)
    # rotations compose: pos a then pos b equals pos a + b (exact angles)
    inv2 = np.array([0.25, 0.5], dtype=np.float32)
    a = mo.rope(mo.rope(x[:, :4], 2, inv2, 1, 4), 3, inv2, 1, 4)
    np.testing.assert_allclose(a, mo.rope(x[:, :4], 5, inv2, 1, 4), rtol=1e-10, atol=1e-12)


def test_attention_single_key_causal_and_gqa():
    rng = np.random.default_rng(2)
    nh, nkv, hd, n = 4, 2, 8, 6
    kc = rng.standard_normal((n, nkv * hd))
    vc = rng.standard_normal((n, nkv * hd))
    q = rng.standard_normal((1, nh * hd))
    out = mo.attention(q, kc, vc, 0, nh, nkv, hd)          # position 0: one key
    for h in range(nh):
        g = h // (nh // nkv)
        np.testing.assert_allclose(out[0, h * hd:(h + 1) * hd], vc[0, g * hd:(g + 1) * hd],
                                   rtol=1e-12)
    # causal: keys past the query's position do not matter
    q2 = rng.standard_normal((2, nh * hd))
    base = mo.attention(q2, kc, vc, 2, nh, nkv, hd)
    kc2, vc2 = kc.copy(), vc.copy()
    kc2[4:] = 99.0
    vc2[4:] = -99.0
    np.testing.assert_allclose(mo.attention(q2, kc2, vc2, 2, nh, nkv, hd), base, rtol=1e-12)
    # q = 0: uniform weights -> mean of the visible values
    z = mo.attention(np.zeros((1, nh * hd)), kc, vc, 3, nh, nkv, hd)
    np.testing.assert_allclose(z[0, :hd], vc[:4, :hd].mean(axis=0), rtol=1e-12)
    # heads of one group with equal q read the same KV head
    qs = np.tile(rng.standard_normal(hd), nh)[None, :]
    o = mo.attention(qs, kc, vc, 5, nh, nkv, hd)
    np.testing.assert_allclose(o[0, :hd], o[0, hd:2 * hd], rtol=1e-12)
    assert not np.allclose(o[0, :hd], o[0, 2 * hd:3 * hd])


def test_swiglu_values():
    g = np.array([0.0, 1.0, 30.0, -30.0])
    u = np.array([5.0, 2.0, 1.0, 1.0])
    np.testing.assert_allclose(mo.swiglu(g, u), [0.0, 2.0 / (1 + np.exp(-1.0)), 30.0, 0.0],
                               atol=1e-11)


def packed(n, m, seed, std, G, scale):
    return pack_q8_np(bf16_bits_to_f32(synth_weights_bf16(n, m, seed, std)), G, scale)


def tiny_model(maxlen=16, G=64, scale="f16", layers=2, seed=0, hidden=512, n_heads=8, n_kv=2,
               head_dim=64, inter=1024, vocab=97, qk_norm=False, tied=True):
    """A small Llama-style model (packed rows 16-byte aligned, head_dim 64);
    with qk_norm a Qwen3-style one (per-head q/k norms, plain RoPE); with
    tied=False a separate lm_head (Llama-3.1-8B, Qwen3-8B)."""
    spec = mo.ModelSpec(hidden=hidden, layers=layers, n_heads=n_heads, n_kv=n_kv,
                        head_dim=head_dim, inter=inter, vocab=vocab,
                        eps=1e-6 if qk_norm else 1e-5, G=G, scale=scale, qk_norm=qk_norm,
                        tied=tied)
    rng = np.random.default_rng(seed)
    H, QD, KVD, I = spec.hidden, spec.n_heads * spec.head_dim, spec.n_kv * spec.head_dim, spec.inter
    t = {"model.embed_tokens.weight": packed(spec.vocab, H, seed + 1, 0.5, G, scale),
         "model.norm.weight": f32_to_bf16_bits((1 + 0.1 * rng.standard_normal(H)).astype(np.float32))}
    if not tied:
        t["lm_head.weight"] = packed(spec.vocab, H, seed + 2, 1.5 / np.sqrt(H), G, scale)
    k = 10
    for L in range(layers):
        p = f"model.layers.{L}."
        for name, (n, m) in {"self_attn.q_proj.weight": (QD, H), "self_attn.k_proj.weight": (KVD, H),
                             "self_attn.v_proj.weight": (KVD, H), "self_attn.o_proj.weight": (H, QD),
                             "mlp.gate_proj.weight": (I, H), "mlp.up_proj.weight": (I, H),
                             "mlp.down_proj.weight": (H, I)}.items():
            k += 1
            t[p + name] = packed(n, m, seed + k, 1.5 / np.sqrt(m), G, scale)
        for name in ["input_layernorm.weight", "post_attention_layernorm.weight"]:
            t[p + name] = f32_to_bf16_bits((1 + 0.1 * rng.standard_normal(H)).astype(np.float32))
        if qk_norm:
            for name in ["self_attn.q_norm.weight", "self_attn.k_norm.weight"]:
                t[p + name] = f32_to_bf16_bits(
                    (1 + 0.1 * rng.standard_normal(head_dim)).astype(np.float32))
    inv = (mo.rope_inv_freq(spec.head_dim, 1000000.0) if qk_norm else
           mo.llama3_inv_freq(spec.head_dim, 500000.0, 32.0, 1.0, 4.0, 8192.0))
    return spec, t, inv


def qwen_tiny(**kw):
    """A small Qwen3-style model: head_dim 128, GQA 2, q/k head norms."""
    return tiny_model(hidden=512, n_heads=4, n_kv=2, head_dim=128, qk_norm=True, **kw)


def test_prefill_equals_token_by_token():
    """Appending the prompt at once or one token at a time gives the same
    last-position logits (KV cache, positions and causal mask agree)."""
    spec, t, inv = tiny_model()
    ids = [3, 14, 15, 92, 65]
    a = mo.OracleModel(spec, t, inv, 16)
    la = a.forward(ids)
    b = mo.OracleModel(spec, t, inv, 16)
    for i in ids:
        lb = b.forward([i])
    assert np.all(np.isfinite(la)) and np.std(la) > 0.1
    np.testing.assert_allclose(la, lb, rtol=1e-9, atol=1e-12, equal_nan=False)
    assert a.pos == b.pos == len(ids)


def test_head_rmsnorm_is_rowwise_and_heads_are_independent():
    rng = np.random.default_rng(3)
    nh, hd, eps = 3, 8, 1e-6
    x = rng.standard_normal((2, nh * hd))
    w = f32_to_bf16_bits((1 + 0.1 * rng.standard_normal(hd)).astype(np.float32))
    y = mo.head_rmsnorm(x, w, nh, hd, eps)
    for i in range(2):
        for h in range(nh):
            np.testing.assert_allclose(y[i, h * hd:(h + 1) * hd],
                                       mo.rmsnorm(x[i:i + 1, h * hd:(h + 1) * hd], w, eps)[0],
                                       rtol=1e-12)
    x2 = x.copy()
    x2[:, hd:2 * hd] *= 7.0                 # scale head 1 only
    y2 = mo.head_rmsnorm(x2, w, nh, hd, 0.0)
    y0 = mo.head_rmsnorm(x, w, nh, hd, 0.0)
    np.testing.assert_allclose(y2, y0, rtol=1e-12)


def test_rope_inv_freq_geometric():
    """Plain RoPE frequencies: 1 at d = 0, a constant ratio theta^(-2/hd)
    between neighbours (to f32 rounding), theta^(-(hd-2)/hd) at the end."""
    hd, theta = 128, 1000000.0
    inv = mo.rope_inv_freq(hd, theta).astype(np.float64)
    assert inv[0] == 1.0
    np.testing.assert_allclose(inv[1:] / inv[:-1], np.exp(-2.0 * np.log(theta) / hd), rtol=3e-7)
    np.testing.assert_allclose(inv[-1], np.exp(-(hd - 2) / hd * np.log(theta)), rtol=1e-7)


def test_qk_norm_removes_the_scale_of_q_and_k_projections():
    """With per-head q/k norms (eps = 0, which makes them scale-free),
    W_q -> 4 W_q and W_k -> 4 W_k (powers of two: only the f16 group scales
    change, exactly) leave the logits unchanged; without the norms they
    change them."""
    spec, t, inv = qwen_tiny(seed=4)
    spec = mo.ModelSpec(**{**spec.__dict__, "eps": 0.0})
    rs_h = t["model.layers.0.self_attn.q_proj.weight"].shape[1]
    groups = spec.hidden // spec.G

    def scaled(tensors):
        out = dict(tensors)
        for L in range(spec.layers):
            for name in ["self_attn.q_proj.weight", "self_attn.k_proj.weight"]:
                key = f"model.layers.{L}.{name}"
                w = out[key].copy()
                sc = w[:, :groups].view(np.float16).astype(np.float32) * 4.0
                w[:, :groups] = sc.astype(np.float16).view(np.uint16)
                out[key] = w
        return out

    assert rs_h == groups + spec.hidden // 2
    ids = [3, 1, 4, 1, 5]
    base = mo.OracleModel(spec, t, inv, 16).forward(ids)
    big = mo.OracleModel(spec, scaled(t), inv, 16).forward(ids)
    np.testing.assert_allclose(big, base, rtol=1e-9, atol=1e-9)
    plain = mo.ModelSpec(**{**spec.__dict__, "qk_norm": False})
    a = mo.OracleModel(plain, t, inv, 16).forward(ids)
    b = mo.OracleModel(plain, scaled(t), inv, 16).forward(ids)
    assert np.max(np.abs(a - b)) > 1e-3


def zero_rows(t, name):
    """Packed rows of zeros (scale 0, codes 0): the matrix dequantises to 0."""
    out = dict(t)
    out[name] = np.zeros_like(t[name])
    return out


def test_layer_with_zero_o_and_down_is_the_identity():
    """With W_o = W_down = 0 a pre-norm block adds nothing to its input: the
    layer returns x exactly (a dropped or doubled residual fails this), while
    the KV cache still receives the rotated k and v rows."""
    spec, t, inv = tiny_model(seed=21)
    for name in ["self_attn.o_proj.weight", "mlp.down_proj.weight"]:
        t = zero_rows(t, "model.layers.0." + name)
    m = mo.OracleModel(spec, t, inv, 16)
    x = np.random.default_rng(22).standard_normal((3, spec.hidden))
    y = m.layer(0, x)
    assert np.array_equal(y, x)
    assert np.abs(m.kc[0][:3]).max() > 0 and np.abs(m.vc[0][:3]).max() > 0
    # with either projection back the output moves off x
    spec2, t2, _ = tiny_model(seed=21)
    for keep in ["self_attn.o_proj.weight", "mlp.down_proj.weight"]:
        other = ({"self_attn.o_proj.weight", "mlp.down_proj.weight"} - {keep}).pop()
        m2 = mo.OracleModel(spec, zero_rows(t2, "model.layers.0." + other), inv, 16)
        assert np.abs(m2.layer(0, x) - x).max() > 1e-3, keep


def test_each_norm_weight_feeds_its_own_branch():
    """input_layernorm feeds only the attention branch and
    post_attention_layernorm only the MLP branch: with the MLP zeroed
    (W_down = 0) scaling the post-attention norm weights changes nothing and
    scaling the input norm weights changes the output; with the attention
    zeroed (W_o = 0) the other way round.  Swapped norm weights fail it."""
    spec, t, inv = tiny_model(seed=23)
    x = np.random.default_rng(24).standard_normal((2, spec.hidden))
    p = "model.layers.0."

    def run(tensors):
        return mo.OracleModel(spec, tensors, inv, 16).layer(0, x)

    def scaled_norm(tensors, name):
        out = dict(tensors)
        w = bf16_bits_to_f32(tensors[p + name]) * np.float32(1.5)
        out[p + name] = f32_to_bf16_bits(w.astype(np.float32))
        return out

    for zeroed, inert, live in (("mlp.down_proj.weight", "post_attention_layernorm.weight",
                                 "input_layernorm.weight"),
                                ("self_attn.o_proj.weight", "input_layernorm.weight",
                                 "post_attention_layernorm.weight")):
        tz = zero_rows(t, p + zeroed)
        base = run(tz)
        np.testing.assert_array_equal(run(scaled_norm(tz, inert)), base)
        assert np.abs(run(scaled_norm(tz, live)) - base).max() > 1e-3, live


def test_injected_linear_gives_the_same_model(cor):
    """The model oracle with the C float64 closed form as its linear gives
    the logits of its numpy dequantise-then-matmul form (1e-12)."""
    spec, t, inv = tiny_model(seed=25)
    ids = [7, 8, 9, 10]
    a = mo.OracleModel(spec, t, inv, 16).forward(ids)
    b = mo.OracleModel(spec, t, inv, 16, linear=cor.linear_f64x).forward(ids)
    assert np.max(np.abs(a - b)) <= 1e-12 * np.max(np.abs(a))
