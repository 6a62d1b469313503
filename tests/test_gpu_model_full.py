"""Whole models at their real widths on the GPU (through the C ABI) against
the float64 model oracle -- the reference's own Q8 gate is a whole-model
check (prefill, greedy ids, a logit bound against an f32 oracle:
qwen3_mojo/src/qwen_q8.mojo:180-224) over the layer runner
src/llama_q8.mojo:144-230.

Models: Llama-3.2-1B (16 layers, hidden 2048, 32 / 8 heads of 64, MLP 8192,
tied 128256-row head -- the headline decode step), Qwen3-0.6B (28 layers,
hidden 1024, 16 / 8 heads of 128 with q/k head norms, MLP 3072, tied
151936-row head -- the reference's own Q8 model) and Llama-3.1-8B (32
layers, hidden 4096, MLP 14336, untied head), with random bf16 weights
packed on the GPU (G64 / binary16 scales, the reference layout) and
downloaded for the oracle, which runs every linear as the float64 closed
form over the same packed rows.

What is compared (bars written in each test):
  * a short prompt (the few-row linears and the split-KV attention):
    last-position logits within max-rel-err 1e-3 of float64;
  * then one eager fused step and graph-replayed steps (the decode step the
    bench times: fused GEMVs, the one-launch attention with its merge, the
    head with its argmax on the GPU): logits within 1e-3, and each step's
    token equal to the float64 model's unless the float64 model's two best
    logits lie within the bar of each other.
The oracle is fed the GPU's tokens, so both walk the same sequence.
"""

import sys

import numpy as np
import pytest

from lama32_mojo_amd import model as gm
from lama32_mojo_amd.q8 import q8_rowstride
from oracle import model_oracle as mo
from oracle.q8_oracle import max_rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def oracle_for(m: gm.Q8Llama, cor, maxlen: int) -> mo.OracleModel:
    """The GPU model's packed arena, downloaded tensor by tensor, as a
    float64 model oracle with the configuration's own RoPE frequencies
    (the oracle's restatement of them)."""
    cfg = m.cfg
    shapes = gm.tensor_shapes(cfg)
    tensors = {}
    for name in gm.weight_names(cfg):
        sh = shapes[name]
        off = m.w.offs[name]
        if len(sh) == 2:
            rs = q8_rowstride(sh[1], m.G, m.scale)
            tensors[name] = m.w.buf.download((sh[0], rs), np.uint16, 2 * off)
        else:
            tensors[name] = m.w.buf.download((sh[0],), np.uint16, 2 * off)
    spec = mo.ModelSpec(hidden=cfg.hidden, layers=cfg.layers, n_heads=cfg.n_heads,
                        n_kv=cfg.n_kv, head_dim=cfg.head_dim, inter=cfg.inter, vocab=cfg.vocab,
                        eps=cfg.eps, G=m.G, scale=m.scale, tied=cfg.tied, qk_norm=cfg.qk_norm)
    if cfg.rope == "plain":
        inv = mo.rope_inv_freq(cfg.head_dim, cfg.theta)
    else:
        inv = mo.llama3_inv_freq(cfg.head_dim, cfg.theta, cfg.rope_factor, cfg.low_ff,
                                 cfg.high_ff, cfg.orig_ctx)
    return mo.OracleModel(spec, tensors, inv, maxlen, linear=cor.linear_f64x)


def check_logits(lg, lr, what):
    """Logits within TOL of float64, and the same best token unless the
    float64 model's best two are within the bar of each other."""
    assert np.all(np.isfinite(lg)), what
    err = max_rel_err(lg, lr)
    say(f"  {what}: max-rel-err {err:.2e}")
    assert err <= TOL, (what, err)
    check_token(int(np.argmax(lg)), lr, what)


def check_token(tok, lr, what):
    best = int(np.argmax(lr))
    if tok != best:
        gap = float(lr[best] - lr[tok])
        assert gap <= 2 * TOL * float(np.max(np.abs(lr))), (what, tok, best, gap)


MODELS = {"llama-3.2-1b": gm.LLAMA_32_1B, "qwen3-0.6b": gm.QWEN3_06B,
          "llama-3.1-8b": gm.LLAMA_31_8B}


@pytest.mark.timeout(600)
@pytest.mark.parametrize("name", list(MODELS))
def test_full_width_model_against_float64(ctx, cor, name):
    cfg = MODELS[name]
    maxlen = 32
    say("full-width model", name)
    m = gm.Q8Llama(ctx, cfg, maxlen, 64, "f16", seed=3, max_prefill=8)
    try:
        ref = oracle_for(m, cor, maxlen)
        say("  weights packed and downloaded")
        prompt = [int(v) for v in np.random.default_rng(5).integers(0, cfg.vocab, size=6)]
        lg = m.forward(prompt)
        lr = ref.forward(prompt)
        check_logits(lg, lr, "prompt of 6")
        tok = int(np.argmax(lg))
        # one eager fused step (device argmax), the oracle fed the same token
        nxt = m.forward_argmax([tok])
        lr = ref.forward([tok])
        check_token(nxt, lr, "eager fused step")
        tok = nxt
        # graph-replayed steps: logits of each replay and its token
        for step in range(3):
            ids = m.decode_steps(tok, 1)
            lg = m.a.read(m.graph_logits, cfg.vocab)
            lr = ref.forward([tok])
            check_logits(lg, lr, f"graph step {step}")
            assert ids[0] == int(np.argmax(lg)), step
            tok = ids[0]
        assert ref.pos == m.n_cached == len(prompt) + 4
    finally:
        m.close()


PROMPT_MODELS = {"llama-3.2-1b": (gm.LLAMA_32_1B, 80), "qwen3-0.6b": (gm.QWEN3_06B, 80),
                 "llama-3.1-8b": (gm.LLAMA_31_8B, 40)}
# Prompt rows run every linear on the binary16 GEMM (activations and q*s
# rounded to binary16, 2^-11 each), and the rounding errors build up layer
# by layer: measured against float64, 1.6e-4 per layer on both Llama models
# (Llama-3.2-1B 2.6e-3 over 16 layers, Llama-3.1-8B 5.1e-3 over 32 at 40
# rows and 6.0e-3 at 80), Qwen3-0.6B 1.2e-3 over 28.  (The f32 paths of the
# short prompt above sit at 2e-4 - 7e-4 already: random-sign dot products
# of 2048 - 14336 terms lose about m times the f32 epsilon, relative to
# their sum, and the layers compound it.)  The bar is 3e-4 per layer; a
# wrong offset, stride or weight gives errors of order one.
TOL_PROMPT_PER_LAYER = 3e-4


@pytest.mark.timeout(600)
@pytest.mark.parametrize("name", list(PROMPT_MODELS))
def test_full_width_prompt_rows_against_float64(ctx, cor, name):
    """An 80-token prompt at the real widths (40 for Llama-3.1-8B, whose
    float64 model costs 7 GMAC per token): the dequant-GEMM path (64-row
    tiles and 128-code iterations on the narrower projections, q|k|v and
    gate|up stacked with the RMSNorms in their binary16 pre-passes, the
    residual folded into the next norm), the strided RoPE and the one-pass
    prompt attention.  Last-position logits within 3e-4 per layer of
    float64 (the GEMM rounds activations and q*s to binary16), then one
    graph-replayed
    decode step over the cache the prompt wrote, within the same bar and
    with the float64 model's token unless its best two logits lie within
    the bar."""
    cfg, s = PROMPT_MODELS[name]
    maxlen = 96
    tol = TOL_PROMPT_PER_LAYER * cfg.layers
    say("full-width prompt rows", name)
    m = gm.Q8Llama(ctx, cfg, maxlen, 64, "f16", seed=4, max_prefill=s)
    try:
        ref = oracle_for(m, cor, maxlen)
        prompt = [int(v) for v in np.random.default_rng(8).integers(0, cfg.vocab, size=s)]
        lg = m.forward(prompt)
        lr = ref.forward(prompt)
        assert np.all(np.isfinite(lg))
        err = max_rel_err(lg, lr)
        say(f"  prompt of {s}: max-rel-err {err:.2e}")
        assert err <= tol, err
        tok = int(np.argmax(lg))
        best = int(np.argmax(lr))
        if tok != best:
            assert float(lr[best] - lr[tok]) <= 2 * tol * float(np.max(np.abs(lr)))
        ids = m.decode_steps(tok, 1)
        lg = m.a.read(m.graph_logits, cfg.vocab)
        lr = ref.forward([tok])
        err = max_rel_err(lg, lr)
        say(f"  graph step after the prompt: max-rel-err {err:.2e}")
        assert err <= tol, err
        assert ids[0] == int(np.argmax(lg))
        assert ref.pos == m.n_cached == s + 1
    finally:
        m.close()
