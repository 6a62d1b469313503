"""Pins of the CPU model oracle (oracle/model_oracle.py) by closed forms and
invariants -- no GPU.  Each check is chosen so a plausible slip (a sign in
RoPE, a wrong GQA head map, a dropped causal mask, a missing eps) fails it."""

import numpy as np
import pytest

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
               head_dim=64, inter=1024, vocab=97):
    """A small Llama-style model (packed rows 16-byte aligned, head_dim 64)."""
    spec = mo.ModelSpec(hidden=hidden, layers=layers, n_heads=n_heads, n_kv=n_kv,
                        head_dim=head_dim, inter=inter, vocab=vocab, eps=1e-5, G=G, scale=scale)
    rng = np.random.default_rng(seed)
    H, QD, KVD, I = spec.hidden, spec.n_heads * spec.head_dim, spec.n_kv * spec.head_dim, spec.inter
    t = {"model.embed_tokens.weight": packed(spec.vocab, H, seed + 1, 0.5, G, scale),
         "model.norm.weight": f32_to_bf16_bits((1 + 0.1 * rng.standard_normal(H)).astype(np.float32))}
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
    inv = mo.llama3_inv_freq(spec.head_dim, 500000.0, 32.0, 1.0, 4.0, 8192.0)
    return spec, t, inv


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
