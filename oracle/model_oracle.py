"""CPU oracle for the decode-step layer kernels and the Q8 transformer step.

TEST INFRASTRUCTURE ONLY.  This module is the checker.  It may be imported by
tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline leg, and by
nothing else; the product path (lama32_mojo_amd, libq8hip.so) never imports,
loads or calls it.

float64 numpy restatements of the reference's layer kernels and layer runner
(src/llama_common.mojo, src/llama_q8.mojo), over the same packed Q8 rows the
GPU reads:

  rmsnorm          k_rmsnorm_w              src/llama_common.mojo:197-225
  head_rmsnorm     k_rmsnorm2_w             src/llama_common.mojo:228-270
  rope_inv_freq    rope_inv_freq            src/llama_common.mojo:609-615
  llama3_inv_freq  llama3_inv_freq          src/llama_common.mojo:618-633
  rope             k_rope_qk_copy2          src/llama_common.mojo:299-342
  attention        k_scores, k_softmax_rows, k_att_out
                                            src/llama_common.mojo:402-473
  swiglu           k_swiglu_mul             src/llama_common.mojo:476-481
  run_layer        run_layer_q8             src/llama_q8.mojo:144-230
  forward          QwenQ8._run_forward      qwen3_mojo/src/qwen_q8.mojo:127-151

One deliberate difference of the build under test is modelled here: the KV
cache holds binary16 values (rounded to nearest) instead of f32, so the
oracle rounds cached k and v the same way.  Everything else is float64.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from .q8_oracle import bf16_bits_to_f32, linear_f64_np


def rmsnorm(x: np.ndarray, w_bits: np.ndarray, eps: float) -> np.ndarray:
    """y = w * x / sqrt(mean(x^2) + eps) per row (k_rmsnorm_w)."""
    x = np.asarray(x, dtype=np.float64)
    w = bf16_bits_to_f32(w_bits).astype(np.float64)
    inv = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + float(np.float32(eps)))
    return w * x * inv


def head_rmsnorm(x: np.ndarray, w_bits: np.ndarray, nheads: int, head_dim: int,
                 eps: float) -> np.ndarray:
    """Per-head RMSNorm of rows [s, nheads * head_dim] with one head_dim
    weight vector (k_rmsnorm2_w: every head row normalised on its own)."""
    s = x.shape[0]
    y = rmsnorm(np.asarray(x, dtype=np.float64).reshape(s * nheads, head_dim), w_bits, eps)
    return y.reshape(s, nheads * head_dim)


def rope_inv_freq(head_dim: int, theta: float) -> np.ndarray:
    """Plain RoPE inverse frequencies 1 / theta^(2d / head_dim), float64
    rounded to f32 (rope_inv_freq)."""
    return np.array([1.0 / (theta ** (2.0 * d / head_dim)) for d in range(head_dim // 2)],
                    dtype=np.float32)


def llama3_inv_freq(head_dim: int, theta: float, factor: float, low_ff: float, high_ff: float,
                    orig_ctx: float) -> np.ndarray:
    """Per-dim RoPE inverse frequencies with llama3 wavelength scaling,
    computed in float64 and rounded to f32 (llama3_inv_freq)."""
    half = head_dim // 2
    out = np.empty(half, dtype=np.float32)
    for d in range(half):
        inv = 1.0 / (theta ** (2.0 * d / head_dim))
        wavelen = 2.0 * 3.14159265358979323846 / inv
        scaled = inv
        if wavelen >= orig_ctx / high_ff:
            if wavelen > orig_ctx / low_ff:
                scaled = inv / factor
            else:
                smooth = (orig_ctx / wavelen - low_ff) / (high_ff - low_ff)
                scaled = (1.0 - smooth) * inv / factor + smooth * inv
        out[d] = np.float32(scaled)
    return out


def rope(x: np.ndarray, pos0: int, inv: np.ndarray, nheads: int, head_dim: int) -> np.ndarray:
    """HF rotate_half RoPE of rows at positions pos0 .. pos0 + s - 1: the
    angle is f32(pos) * f32(inv[d]) rounded to f32, as the kernel forms it."""
    s = x.shape[0]
    half = head_dim // 2
    y = np.array(x, dtype=np.float64).reshape(s, nheads, head_dim)
    pos = np.arange(pos0, pos0 + s, dtype=np.float32)[:, None]
    ang = (pos * inv[None, :].astype(np.float32)).astype(np.float64)       # [s, half]
    c, sn = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    x0, x1 = y[..., :half].copy(), y[..., half:].copy()
    y[..., :half] = x0 * c - x1 * sn
    y[..., half:] = x1 * c + x0 * sn
    return y.reshape(s, nheads * head_dim)


def f16_round(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=np.float64).astype(np.float16).astype(np.float64)


def attention(q: np.ndarray, kc: np.ndarray, vc: np.ndarray, pos0: int, nheads: int, nkv: int,
              head_dim: int) -> np.ndarray:
    """Causal GQA attention: query row i (position pos0 + i) attends cache
    rows 0 .. pos0 + i; head h reads KV head h // (nheads / nkv); scores are
    dot / sqrt(head_dim) (k_scores, k_softmax_rows, k_att_out)."""
    s = q.shape[0]
    grp = nheads // nkv
    n = pos0 + s                                  # keys the last row sees
    q = np.asarray(q, dtype=np.float64)
    out = np.zeros((s, nheads * head_dim))
    # key t is visible to row i iff t <= pos0 + i
    visible = np.arange(n)[None, :] <= (pos0 + np.arange(s))[:, None]
    for h in range(nheads):
        g = h // grp
        k = np.asarray(kc[:n, g * head_dim:(g + 1) * head_dim], dtype=np.float64)
        v = np.asarray(vc[:n, g * head_dim:(g + 1) * head_dim], dtype=np.float64)
        sc = q[:, h * head_dim:(h + 1) * head_dim] @ k.T / np.sqrt(head_dim)   # [s, n]
        sc = np.where(visible, sc, -np.inf)
        p = np.exp(sc - sc.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        out[:, h * head_dim:(h + 1) * head_dim] = p @ v
    return out


def swiglu(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g = np.asarray(g, dtype=np.float64)
    return g / (1.0 + np.exp(-g)) * u


@dataclass
class ModelSpec:
    hidden: int
    layers: int
    n_heads: int
    n_kv: int
    head_dim: int
    inter: int
    vocab: int
    eps: float
    G: int = 64
    scale: str = "f16"
    tied: bool = True
    qk_norm: bool = False    # per-head q / k RMSNorm before RoPE (Qwen3)


@dataclass
class OracleModel:
    """Packed Q8 weights (u16 rows) and bf16 norms of a Llama-style model,
    with a binary16 KV cache, run in float64."""
    spec: ModelSpec
    tensors: dict            # name -> packed u16 [n, rowstride] or bf16 bits [d]
    inv: np.ndarray          # f32 [head_dim / 2]
    maxlen: int
    kc: list = field(default_factory=list)
    vc: list = field(default_factory=list)
    pos: int = 0
    # the float64 linear y = x . deq(W)^T over packed rows:
    # linear(packed, x, G, scale); numpy's dequantise-then-matmul unless
    # given (a model at full width passes the C closed form, same values)
    linear: object = None

    def __post_init__(self):
        sp = self.spec
        kvd = sp.n_kv * sp.head_dim
        self.kc = [np.zeros((self.maxlen, kvd)) for _ in range(sp.layers)]
        self.vc = [np.zeros((self.maxlen, kvd)) for _ in range(sp.layers)]

    def lin(self, name: str, x: np.ndarray) -> np.ndarray:
        sp = self.spec
        if self.linear is not None:
            return self.linear(self.tensors[name], x, sp.G, sp.scale)
        return linear_f64_np(self.tensors[name], x, x.shape[1], sp.G, sp.scale)

    def layer(self, L: int, x: np.ndarray) -> np.ndarray:
        """One pre-norm GQA block with KV append (run_layer_q8,
        src/llama_q8.mojo:144-230, including the q/k head norms of :171-182)."""
        sp = self.spec
        p = f"model.layers.{L}."
        s = x.shape[0]
        xn = rmsnorm(x, self.tensors[p + "input_layernorm.weight"], sp.eps)
        q = self.lin(p + "self_attn.q_proj.weight", xn)
        k = self.lin(p + "self_attn.k_proj.weight", xn)
        v = self.lin(p + "self_attn.v_proj.weight", xn)
        if sp.qk_norm:
            q = head_rmsnorm(q, self.tensors[p + "self_attn.q_norm.weight"], sp.n_heads,
                             sp.head_dim, sp.eps)
            k = head_rmsnorm(k, self.tensors[p + "self_attn.k_norm.weight"], sp.n_kv,
                             sp.head_dim, sp.eps)
        q = rope(q, self.pos, self.inv, sp.n_heads, sp.head_dim)
        k = rope(k, self.pos, self.inv, sp.n_kv, sp.head_dim)
        self.kc[L][self.pos:self.pos + s] = f16_round(k)
        self.vc[L][self.pos:self.pos + s] = f16_round(v)
        ao = attention(q, self.kc[L], self.vc[L], self.pos, sp.n_heads, sp.n_kv, sp.head_dim)
        h = x + self.lin(p + "self_attn.o_proj.weight", ao)
        z = rmsnorm(h, self.tensors[p + "post_attention_layernorm.weight"], sp.eps)
        g = self.lin(p + "mlp.gate_proj.weight", z)
        u = self.lin(p + "mlp.up_proj.weight", z)
        return h + self.lin(p + "mlp.down_proj.weight", swiglu(g, u))

    def forward(self, ids) -> np.ndarray:
        """Logits of the last position (QwenQ8._run_forward) and KV append;
        the position advances by len(ids)."""
        sp = self.spec
        emb = self.tensors["model.embed_tokens.weight"]
        from .q8_oracle import embed_gather_np
        x = embed_gather_np(emb, np.asarray(ids, dtype=np.int64), sp.hidden, sp.G,
                            sp.scale).astype(np.float64)
        for L in range(sp.layers):
            x = self.layer(L, x)
        self.pos += len(ids)
        xn = rmsnorm(x[-1:], self.tensors["model.norm.weight"], sp.eps)
        head = "model.embed_tokens.weight" if sp.tied else "lm_head.weight"
        return self.lin(head, xn)[0]
