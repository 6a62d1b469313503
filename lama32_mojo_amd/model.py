"""Q8 Llama-family model runner on libq8hip (decode and prefill).

Host side of the reference's Q8 model: configuration, weight-arena layout,
the layer runner and the token loop, driving only libq8hip.so entry points:

  Config, make_config             src/llama_common.mojo:27-52, src/llama_gpu.mojo:29-31,
                                  qwen3_mojo/src/qwen_q8.mojo:30-32
  rope_inv_freq                   src/llama_common.mojo:609-615 (plain, Qwen3)
  llama3_inv_freq                 src/llama_common.mojo:618-633
  weight_names                    src/llama_gpu.mojo:33-47, qwen3_mojo/src/qwen_q8.mojo:35-52
  LayerOffs                       src/llama_common.mojo:55-67
  Q8Llama.layer (run_layer_q8)    src/llama_q8.mojo:144-230
  Q8Llama.forward / forward_argmax  qwen3_mojo/src/qwen_q8.mojo:127-162
  Q8Llama.embed                   qwen3_mojo/src/qwen_q8.mojo:110-124

Differences from the reference host, on purpose:
  * the KV cache is a binary16 buffer of its own (layers x {K, V} x maxlen x
    kv_dim) rather than f32 blocks of the activation arena;
  * residual add + post-attention RMSNorm run as one dispatch;
  * a decode step can be captured once as a HIP graph that reads the token id
    and the position from device memory and writes the argmax id and the next
    position back, so generation replays one graph per token.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Mapping, Sequence

import numpy as np

from . import q8hip
from .q8 import PAD, Acts, Q8Kernels, Weights, q8_rowstride
from .q8hip import Buffer, Context


@dataclass(frozen=True)
class Config:
    """Model dimensions (src/llama_common.mojo:27-52)."""
    hidden: int
    layers: int
    n_heads: int
    n_kv: int
    head_dim: int
    inter: int
    vocab: int
    eps: float
    theta: float
    rope_factor: float
    low_ff: float
    high_ff: float
    orig_ctx: float
    tied: bool = True          # lm_head = packed embed_tokens (Llama-3.2 / Qwen3 Q8 path)
    name: str = "llama"
    qk_norm: bool = False      # per-head RMSNorm of q and k before RoPE (Qwen3)
    rope: str = "llama3"       # "llama3" (wavelength scaling) or "plain" (Qwen3)

    def group(self) -> int:
        return self.n_heads // self.n_kv

    def q_dim(self) -> int:
        return self.n_heads * self.head_dim

    def kv_dim(self) -> int:
        return self.n_kv * self.head_dim

    def half(self) -> int:
        return self.head_dim // 2


# Llama-3.2-1B (src/llama_gpu.mojo:29-31)
LLAMA_32_1B = Config(2048, 16, 32, 8, 64, 8192, 128256, 1e-5, 500000.0, 32.0, 1.0, 4.0, 8192.0,
                     tied=True, name="Llama-3.2-1B")
# Llama-3.1-8B (llama31_mojo/src/llama_gpu.mojo:26-41: untied lm_head)
LLAMA_31_8B = Config(4096, 32, 32, 8, 128, 14336, 128256, 1e-5, 500000.0, 8.0, 1.0, 4.0, 8192.0,
                     tied=False, name="Llama-3.1-8B")
# Qwen3-0.6B, the reference's Q8 model (qwen3_mojo/src/qwen_q8.mojo:24-32)
QWEN3_06B = Config(1024, 28, 16, 8, 128, 3072, 151936, 1e-6, 1000000.0, 1.0, 1.0, 4.0, 8192.0,
                   tied=True, name="Qwen3-0.6B", qk_norm=True, rope="plain")
# Qwen3-8B (untied lm_head 4096 -> 151936)
QWEN3_8B = Config(4096, 36, 32, 8, 128, 12288, 151936, 1e-6, 1000000.0, 1.0, 1.0, 4.0, 8192.0,
                  tied=False, name="Qwen3-8B", qk_norm=True, rope="plain")


def rope_inv_freq(cfg: Config) -> np.ndarray:
    """RoPE inverse frequencies of the configuration: plain 1 / theta^(2d/hd)
    (rope_inv_freq) or with llama3 wavelength scaling (llama3_inv_freq),
    evaluated in float64 and stored as f32."""
    if cfg.rope == "plain":
        return np.array([1.0 / (cfg.theta ** (2.0 * d / cfg.head_dim)) for d in range(cfg.half())],
                        dtype=np.float32)
    return llama3_inv_freq(cfg)


def llama3_inv_freq(cfg: Config) -> np.ndarray:
    """Per-dim RoPE inverse frequencies with llama3 wavelength scaling,
    evaluated in float64 and stored as f32."""
    out = np.empty(cfg.half(), dtype=np.float32)
    for d in range(cfg.half()):
        inv = 1.0 / (cfg.theta ** (2.0 * d / cfg.head_dim))
        wavelen = 2.0 * 3.14159265358979323846 / inv
        scaled = inv
        if wavelen >= cfg.orig_ctx / cfg.high_ff:
            if wavelen > cfg.orig_ctx / cfg.low_ff:
                scaled = inv / cfg.rope_factor
            else:
                smooth = (cfg.orig_ctx / wavelen - cfg.low_ff) / (cfg.high_ff - cfg.low_ff)
                scaled = (1.0 - smooth) * inv / cfg.rope_factor + smooth * inv
        out[d] = np.float32(scaled)
    return out


def weight_names(cfg: Config) -> list[str]:
    """Arena order: embed, final norm, then per layer norms and projections
    (q|k|v and gate|up contiguous, which lets s == 1 fuse them)."""
    names = ["model.embed_tokens.weight", "model.norm.weight"]
    for L in range(cfg.layers):
        p = f"model.layers.{L}."
        names += [p + "input_layernorm.weight", p + "post_attention_layernorm.weight"]
        if cfg.qk_norm:
            names += [p + "self_attn.q_norm.weight", p + "self_attn.k_norm.weight"]
        names += [p + "self_attn.q_proj.weight", p + "self_attn.k_proj.weight",
                  p + "self_attn.v_proj.weight", p + "self_attn.o_proj.weight",
                  p + "mlp.gate_proj.weight", p + "mlp.up_proj.weight",
                  p + "mlp.down_proj.weight"]
    if not cfg.tied:
        names.append("lm_head.weight")
    return names


def tensor_shapes(cfg: Config) -> dict[str, tuple]:
    """name -> (n, m) for Q8 matrices, (d,) for bf16 norm vectors."""
    H, QD, KVD, I = cfg.hidden, cfg.q_dim(), cfg.kv_dim(), cfg.inter
    shapes = {"model.embed_tokens.weight": (cfg.vocab, H), "model.norm.weight": (H,)}
    for L in range(cfg.layers):
        p = f"model.layers.{L}."
        shapes.update({
            p + "input_layernorm.weight": (H,), p + "post_attention_layernorm.weight": (H,),
            p + "self_attn.q_proj.weight": (QD, H), p + "self_attn.k_proj.weight": (KVD, H),
            p + "self_attn.v_proj.weight": (KVD, H), p + "self_attn.o_proj.weight": (H, QD),
            p + "mlp.gate_proj.weight": (I, H), p + "mlp.up_proj.weight": (I, H),
            p + "mlp.down_proj.weight": (H, I)})
        if cfg.qk_norm:
            shapes[p + "self_attn.q_norm.weight"] = (cfg.head_dim,)
            shapes[p + "self_attn.k_norm.weight"] = (cfg.head_dim,)
    if not cfg.tied:
        shapes["lm_head.weight"] = (cfg.vocab, H)
    return shapes


def arena_elems(cfg: Config, G: int, scale: str) -> int:
    """u16 elements of the packed weight arena (PAD head included)."""
    total = PAD
    for name, sh in tensor_shapes(cfg).items():
        total += sh[0] * q8_rowstride(sh[1], G, scale) if len(sh) == 2 else sh[0]
    return total


@dataclass(frozen=True)
class LayerOffs:
    """u16 offsets of one layer's tensors in the weight arena."""
    q: int
    k: int
    v: int
    o: int
    gate: int
    up: int
    down: int
    in_norm: int
    post_norm: int
    q_norm: int = -1           # per-head q / k RMSNorm weights (Qwen3), -1 if none
    k_norm: int = -1


class Q8Llama:
    """A Llama-style model with Q8 linears resident on one GPU.

    weights: name -> array of raw stored values (packed u16 rows [n, rs] for
    matrices, bf16 bit patterns [d] for norms), or None to build random-init
    weights on the GPU (bf16 ~ N(0, std) packed in place, norms ~ 1)."""

    def __init__(self, ctx: Context, cfg: Config, maxlen: int, G: int = 64, scale: str = "f16",
                 weights: Mapping[str, np.ndarray] | None = None, seed: int = 0,
                 std: float = 0.02, act_floats: int | None = None, max_prefill: int = 1,
                 fuse: bool = True):
        self.ctx, self.cfg, self.maxlen = ctx, cfg, int(maxlen)
        # one-row steps fold rmsnorm, swiglu and the residual adds into the
        # GEMV launches
        self.fuse = bool(fuse)
        # prompt rows leave each block's down-projection output pending and
        # add it in the next block's input norm (one residual pass fewer per
        # block; the same bits as the separate add)
        self.fold_residual = True
        # prompt rows run the q|k|v and gate|up GEMMs with their norm (and
        # the residual add before it) in the GEMM's pre-pass (the same bits)
        self.fold_norm = True
        self.G, self.scale = G, scale
        self.qk = Q8Kernels(ctx, G, scale)
        names = weight_names(cfg)
        self.w = Weights(ctx, arena_elems(cfg, G, scale))
        if weights is None:
            self._random_weights(names, seed, std)
        elif hasattr(weights, "upload") and hasattr(weights, "infos"):
            self._check_checkpoint(weights, names)
            self.w.upload_file(weights, names)
        else:
            self.w.upload_all(weights, names)
        self.lo = []
        for L in range(cfg.layers):
            p = f"model.layers.{L}."
            o = self.w.o
            qn = (o(p + "self_attn.q_norm.weight"), o(p + "self_attn.k_norm.weight")) \
                if cfg.qk_norm else (-1, -1)
            self.lo.append(LayerOffs(o(p + "self_attn.q_proj.weight"), o(p + "self_attn.k_proj.weight"),
                                     o(p + "self_attn.v_proj.weight"), o(p + "self_attn.o_proj.weight"),
                                     o(p + "mlp.gate_proj.weight"), o(p + "mlp.up_proj.weight"),
                                     o(p + "mlp.down_proj.weight"), o(p + "input_layernorm.weight"),
                                     o(p + "post_attention_layernorm.weight"), *qn))
        H, QD, KVD, I = cfg.hidden, cfg.q_dim(), cfg.kv_dim(), cfg.inter
        if act_floats is None:
            # three residual row sets (two ping-pong, one pending down
            # output), one layer's temporaries (the arena is reset after every
            # layer), the head, and room for one captured decode step besides
            # a forward pass
            s = max(1, int(max_prefill))
            # (attention scratch grows with the rows up to 15 and is 0 from 16)
            att = q8hip.attention_scratch_floats(min(s, 15), cfg.n_heads, cfg.head_dim,
                                                 self.maxlen)
            layer = s * (4 * H + 3 * QD + 3 * KVD + 2 * I) + att    # incl. q/k norm outputs
            one = 3 * s * H + layer + H + cfg.vocab + 64
            act_floats = PAD + cfg.half() + one + (2 * H + (4 * H + 3 * QD + 3 * KVD + 2 * I)
                                                   + q8hip.attention_scratch_floats(
                                                       1, cfg.n_heads, cfg.head_dim, self.maxlen)
                                                   + H + cfg.vocab + 64)
        self.a = Acts(ctx, act_floats)
        self.oinv = self.a.alloc(cfg.half())
        self.a.write(self.oinv, rope_inv_freq(cfg))
        kvd = cfg.kv_dim()
        self.kv = Buffer.alloc(ctx, 2 * cfg.layers * 2 * self.maxlen * kvd)
        self.okc = [(2 * L) * self.maxlen * kvd for L in range(cfg.layers)]
        self.ovc = [(2 * L + 1) * self.maxlen * kvd for L in range(cfg.layers)]
        self.ids = Buffer.alloc(ctx, 4 * max(self.maxlen, 16))
        self.posbuf = Buffer.alloc(ctx, 16)
        self.posbuf.upload(np.zeros(4, dtype=np.int32))
        self.n_cached = 0
        self.graph = None
        self.graph_logits = None
        self.graph_x = None

    # ---- weights -------------------------------------------------------------
    def _check_checkpoint(self, st, names: Sequence[str]) -> None:
        """A packed file (checkpoint.pack_checkpoint / quantize.py) must hold
        this model's tensors in this layout: packed rows [n, rowstride(m)]
        as 2-byte elements, norms as bf16 vectors."""
        from .checkpoint import checkpoint_layout
        G, sc = checkpoint_layout(st)
        if (G, sc) != (self.G, self.scale):
            raise ValueError(f"checkpoint layout G={G} {sc}, model expects G={self.G} "
                             f"{self.scale}")
        shapes = tensor_shapes(self.cfg)
        for name in names:
            if not st.has(name):
                raise KeyError(f"{name} is not in the checkpoint")
            sh = shapes[name]
            want = ([sh[0], q8_rowstride(sh[1], self.G, self.scale)] if len(sh) == 2
                    else list(sh))
            info = st.get(name)
            if info.shape != want:
                raise ValueError(f"{name}: shape {info.shape} in the checkpoint, expected {want}")

    def _random_weights(self, names: Sequence[str], seed: int, std: float) -> None:
        import torch

        cfg, G, scale = self.cfg, self.G, self.scale
        shapes = tensor_shapes(cfg)
        top = self.w.top
        for i, name in enumerate(names):
            sh = shapes[name]
            self.w.offs[name] = top
            gen = torch.Generator(device="cuda")
            gen.manual_seed(seed * 100003 + i)
            if len(sh) == 1:
                t = (1.0 + 0.1 * torch.randn(sh, device="cuda", generator=gen)).to(torch.bfloat16)
                torch.cuda.synchronize()
                src = Buffer.wrap(self.ctx, t.data_ptr(), t.numel() * 2)
                self._upload_from_device(src, top, t.numel())
                top += sh[0]
            else:
                n, m = sh
                t = (torch.randn((n, m), device="cuda", generator=gen) * std).to(torch.bfloat16)
                torch.cuda.synchronize()
                src = Buffer.wrap(self.ctx, t.data_ptr(), t.numel() * 2)
                q8hip.quantize_pack(self.ctx, src, 0, q8hip.Q8_SRC_BF16, n, m, self.w.buf, top,
                                    G, scale)
                self.ctx.sync()
                src.free()
                top += n * q8_rowstride(m, G, scale)
            del t
        self.w.top = top

    def _upload_from_device(self, src: Buffer, off_u16: int, count: int) -> None:
        host = src.download((count,), np.uint16)
        src.free()
        self.w.buf.upload(host, 2 * off_u16)

    # ---- layer runner (run_layer_q8) ---------------------------------------
    def linear(self, ox: int, s: int, m: int, owt: int, n: int) -> int:
        self.a.align(4)                 # 16-byte rows for the vector kernels that read them
        oy = self.a.alloc(s * n)
        q8hip.linear(self.ctx, self.w.buf, owt, self.a.buf, ox, oy, s, m, n, self.G, self.scale)
        return oy

    def _norm_in_gemm(self, s: int, ox: int) -> bool:
        """Whether s rows at ox can take q8_linear_rmsnorm (GEMM rows, rows of
        at most 16384, 16-byte aligned)."""
        return self.fold_norm and s >= 32 and self.cfg.hidden <= 16384 and ox % 4 == 0

    def layer(self, L: int, ox: int, s: int, pos0: int, device_pos: bool = False,
              oh: int | None = None, pending: int | None = None,
              oout: int | None = None) -> int:
        """One block on the s rows at ox; the new residual rows go to oh
        (allocated here when None); returns oh.  With pending, the rows at
        pending (the previous block's down output) are first added to ox in
        place, in the input norm's launch; with oout, the down output is left
        at oout instead of being added to oh."""
        cfg, ctx, a, w = self.cfg, self.ctx, self.a, self.w
        lo = self.lo[L]
        H, QD, KVD, I = cfg.hidden, cfg.q_dim(), cfg.kv_dim(), cfg.inter
        rsH = q8_rowstride(H, self.G, self.scale)
        pb = self.posbuf if device_pos else None
        if (s == 1 and self.fuse and lo.k == lo.q + QD * rsH and lo.v == lo.k + KVD * rsH
                and lo.up == lo.gate + I * rsH):
            return self._layer_fused(L, ox, pos0, pb, oh)
        ld = 0                                            # q, k, v row stride
        qkv_stacked = lo.k == lo.q + QD * rsH and lo.v == lo.k + KVD * rsH
        if qkv_stacked and self._norm_in_gemm(s, ox):
            # prompt rows: the input norm (after the pending residual add,
            # stored over ox) in the stacked q|k|v GEMM's pre-pass
            a.align(4)
            oq = a.alloc(s * (QD + 2 * KVD))
            q8hip.linear_rmsnorm(ctx, w.buf, lo.q, lo.in_norm, cfg.eps, a.buf, ox, oq, s, H,
                                 QD + 2 * KVD, self.G, self.scale, ores_f32=pending,
                                 oh_f32=ox if pending is not None else None)
            okk, ov = oq + QD, oq + QD + KVD
            ld = QD + 2 * KVD
        else:
            xn = a.alloc(s * H)
            if pending is not None:
                q8hip.add_rmsnorm(ctx, w.buf, lo.in_norm, a.buf, ox, pending, ox, xn, s, H,
                                  cfg.eps)
            else:
                q8hip.rmsnorm(ctx, w.buf, lo.in_norm, a.buf, ox, xn, s, H, cfg.eps)
            if qkv_stacked:
                # one stacked q|k|v linear; prompt rows then carry the stride
                oq = self.linear(xn, s, H, lo.q, QD + 2 * KVD)
                okk, ov = oq + QD, oq + QD + KVD
                ld = QD + 2 * KVD if s > 1 else 0
            else:
                oq = self.linear(xn, s, H, lo.q, QD)
                okk = self.linear(xn, s, H, lo.k, KVD)
                ov = self.linear(xn, s, H, lo.v, KVD)
        if cfg.qk_norm and ld:                            # k_rmsnorm2_w
            # the q and k heads normalised in place inside the stacked rows
            q8hip.head_rmsnorm(ctx, w.buf, lo.q_norm, a.buf, oq, oq, s, cfg.n_heads,
                               cfg.head_dim, ld, cfg.eps)
            q8hip.head_rmsnorm(ctx, w.buf, lo.k_norm, a.buf, okk, okk, s, cfg.n_kv,
                               cfg.head_dim, ld, cfg.eps)
        elif cfg.qk_norm:
            a.align(4)
            oqn, okn = a.alloc(s * QD), a.alloc(s * KVD)
            q8hip.rmsnorm(ctx, w.buf, lo.q_norm, a.buf, oq, oqn, s * cfg.n_heads, cfg.head_dim,
                          cfg.eps)
            q8hip.rmsnorm(ctx, w.buf, lo.k_norm, a.buf, okk, okn, s * cfg.n_kv, cfg.head_dim,
                          cfg.eps)
            oq, okk = oqn, okn
        a.align(4)                      # q and out of the prompt attention: 16-byte aligned
        oao = a.alloc(s * QD)
        if s == 1:
            # (q and k are already normalised here when the model has q/k norms)
            q8hip.decode_attention(ctx, a.buf, oq, okk, ov, self.oinv, self.kv, self.okc[L],
                                   self.ovc[L], self.maxlen, oao, pos0, cfg.n_heads, cfg.n_kv,
                                   cfg.head_dim, pb, 0)
        else:
            q8hip.rope_kv(ctx, a.buf, oq, okk, ov, self.oinv, self.kv, self.okc[L], self.ovc[L],
                          self.maxlen, s, pos0, cfg.n_heads, cfg.n_kv, cfg.head_dim, pb, 0, ld)
            osc = a.alloc(q8hip.attention_scratch_floats(s, cfg.n_heads, cfg.head_dim,
                                                         self.maxlen))
            q8hip.attention(ctx, a.buf, oq, self.kv, self.okc[L], self.ovc[L], self.maxlen, oao,
                            osc, s, pos0, cfg.n_heads, cfg.n_kv, cfg.head_dim, pb, 0, ld)
        oo = self.linear(oao, s, QD, lo.o, H)
        if oh is None:
            oh = a.alloc(s * H)
        gu_stacked = lo.up == lo.gate + I * rsH and (s == 1 or (s >= 32 and I % 4 == 0))
        oz = None
        if not (gu_stacked and self._norm_in_gemm(s, ox)):
            oz = a.alloc(s * H)
            q8hip.add_rmsnorm(ctx, w.buf, lo.post_norm, a.buf, ox, oo, oh, oz, s, H, cfg.eps)
        if s >= 32:
            # 16-byte aligned gate rows: stacked rows then always take the
            # swiglu pre-pass below, the only path that reads them at their
            # 2I stride
            a.align(4)
        if oz is None:
            # prompt rows: residual add and post-attention norm in the stacked
            # gate|up GEMM's pre-pass
            og = a.alloc(s * 2 * I)
            q8hip.linear_rmsnorm(ctx, w.buf, lo.gate, lo.post_norm, cfg.eps, a.buf, ox, og, s,
                                 H, 2 * I, self.G, self.scale, ores_f32=oo, oh_f32=oh)
            ou = og + I
        elif gu_stacked:
            og = self.linear(oz, s, H, lo.gate, 2 * I)
            ou = og + I
        else:
            og = self.linear(oz, s, H, lo.gate, I)
            ou = self.linear(oz, s, H, lo.up, I)
        if s >= 32 and og % 4 == 0 and ou % 4 == 0:
            # prompt rows: the swiglu folded into the down GEMM's pre-pass,
            # gate|up rows read at their stride when stacked
            om = a.alloc(s * H) if oout is None else oout
            q8hip.linear_swiglu(ctx, w.buf, lo.down, a.buf, og, ou, om, s, I, H, self.G,
                                self.scale, ld=2 * I if gu_stacked else 0)
        else:
            assert not (gu_stacked and s > 1), "stacked gate|up rows need the strided pre-pass"
            q8hip.swiglu(ctx, a.buf, og, ou, s * I)
            om = a.alloc(s * H) if oout is None else oout
            q8hip.linear(ctx, w.buf, lo.down, a.buf, og, om, s, I, H, self.G, self.scale)
        if oout is None:
            q8hip.add(ctx, a.buf, om, oh, s * H)
        return oh

    def _layer_fused(self, L: int, ox: int, pos0: int, pb, oh: int | None) -> int:
        """One-row block in six launches: norm + q|k|v, attention (q/k head
        norms, RoPE, KV append, context splits) and its merge, o + residual,
        norm + gate|up + swiglu, down + residual (in place)."""
        cfg, ctx, a, w = self.cfg, self.ctx, self.a, self.w
        lo = self.lo[L]
        H, QD, KVD, I = cfg.hidden, cfg.q_dim(), cfg.kv_dim(), cfg.inter
        G, sc = self.G, self.scale
        oq = a.alloc(QD + 2 * KVD)
        q8hip.linear_fused(ctx, w.buf, lo.q, a.buf, ox, oq, H, QD + 2 * KVD, G, sc,
                           pre=q8hip.PRE_RMSNORM, onorm_u16=lo.in_norm, eps=cfg.eps)
        oao = a.alloc(QD)
        qk = dict(wn=w.buf, oqnorm_u16=lo.q_norm, oknorm_u16=lo.k_norm, eps=cfg.eps) \
            if cfg.qk_norm else {}
        q8hip.decode_attention(ctx, a.buf, oq, oq + QD, oq + QD + KVD, self.oinv, self.kv,
                               self.okc[L], self.ovc[L], self.maxlen, oao, pos0, cfg.n_heads,
                               cfg.n_kv, cfg.head_dim, pb, 0, **qk)
        if oh is None:
            oh = a.alloc(H)
        q8hip.linear_fused(ctx, w.buf, lo.o, a.buf, oao, oh, QD, H, G, sc,
                           post=q8hip.POST_RESIDUAL, ores_f32=ox)
        og = a.alloc(I)
        q8hip.linear_fused(ctx, w.buf, lo.gate, a.buf, oh, og, H, 2 * I, G, sc,
                           pre=q8hip.PRE_RMSNORM, onorm_u16=lo.post_norm, eps=cfg.eps,
                           post=q8hip.POST_SWIGLU)
        q8hip.linear_fused(ctx, w.buf, lo.down, a.buf, og, oh, I, H, G, sc,
                           post=q8hip.POST_RESIDUAL, ores_f32=oh)
        return oh

    # ---- token loop ----------------------------------------------------------
    def embed(self, s: int) -> int:
        """Gather s embedding rows for the ids already in self.ids."""
        cfg = self.cfg
        ox = self.a.alloc(s * cfg.hidden)
        q8hip.embed_gather(self.ctx, self.w.buf, self.w.o("model.embed_tokens.weight"), self.ids, 0,
                           self.a.buf, ox, s, cfg.hidden, cfg.vocab, self.G, self.scale)
        return ox

    def _head(self, oh: int, s: int) -> int:
        cfg = self.cfg
        head = "model.embed_tokens.weight" if cfg.tied else "lm_head.weight"
        if self.fuse:
            olg = self.a.alloc(cfg.vocab)
            q8hip.linear_fused(self.ctx, self.w.buf, self.w.o(head), self.a.buf,
                               oh + (s - 1) * cfg.hidden, olg, cfg.hidden, cfg.vocab, self.G,
                               self.scale, pre=q8hip.PRE_RMSNORM,
                               onorm_u16=self.w.o("model.norm.weight"), eps=cfg.eps)
            return olg
        onrm = self.a.alloc(cfg.hidden)
        q8hip.rmsnorm(self.ctx, self.w.buf, self.w.o("model.norm.weight"), self.a.buf,
                      oh + (s - 1) * cfg.hidden, onrm, 1, cfg.hidden, cfg.eps)
        return self.linear(onrm, 1, cfg.hidden, self.w.o(head), cfg.vocab)

    def _layers(self, cur: int, s: int, pos0: int, device_pos: bool) -> int:
        """Every layer over the s rows at cur (ping-pong residual buffers);
        returns the offset of the final residual rows."""
        H = self.cfg.hidden
        nxt = self.a.alloc(s * H)
        # (one-row steps fold the residual into the down GEMV instead)
        pend = self.a.alloc(s * H) if s > 1 and self.fold_residual else None
        for L in range(self.cfg.layers):
            mark = self.a.mark()
            self.layer(L, cur, s, pos0, device_pos, oh=nxt,
                       pending=pend if L > 0 else None, oout=pend)
            self.a.reset(mark)
            cur, nxt = nxt, cur
        if pend is not None:
            q8hip.add(self.ctx, self.a.buf, pend, cur, s * H)
        return cur

    def _run(self, s: int, pos0: int, device_pos: bool) -> int:
        return self._head(self._layers(self.embed(s), s, pos0, device_pos), s)

    def _head_name(self) -> str:
        return "model.embed_tokens.weight" if self.cfg.tied else "lm_head.weight"

    def _head_argmax(self, oh: int, posbuf=None, onext: int | None = None) -> int:
        """Final norm + lm_head + argmax -> ids[0] in two launches (position
        step and the next embedding row with posbuf / onext); returns the
        logits offset."""
        cfg = self.cfg
        olg = self.a.alloc(cfg.vocab)
        q8hip.head_argmax(self.ctx, self.w.buf, self.w.o(self._head_name()),
                          self.w.o("model.norm.weight"), cfg.eps, self.a.buf, oh, olg,
                          cfg.hidden, cfg.vocab, self.G, self.scale, self.ids, 0, posbuf, 0, 1,
                          self.w.o("model.embed_tokens.weight") if onext is not None else None,
                          onext or 0)
        return olg

    def _check_room(self, s: int) -> None:
        if self.n_cached + s > self.maxlen:
            raise RuntimeError("KV cache full")

    def forward(self, ids: Sequence[int]) -> np.ndarray:
        """Logits (f32 [vocab]) of the last of `ids`, appending them to the cache."""
        s = len(ids)
        self._check_room(s)
        self.ids.upload(np.asarray(ids, dtype=np.int32))
        mark = self.a.mark()
        olg = self._run(s, self.n_cached, False)
        logits = self.a.read(olg, self.cfg.vocab)
        self.a.reset(mark)
        self.n_cached += s
        self.posbuf.upload(np.array([self.n_cached], dtype=np.int32))
        return logits

    def forward_argmax(self, ids: Sequence[int]) -> int:
        """Greedy next id after `ids` (GPU argmax, 4-byte readback)."""
        s = len(ids)
        self._check_room(s)
        self.ids.upload(np.asarray(ids, dtype=np.int32))
        mark = self.a.mark()
        oh = self._layers(self.embed(s), s, self.n_cached, False)
        if self.fuse:
            self._head_argmax(oh + (s - 1) * self.cfg.hidden)
        else:
            olg = self._head(oh, s)
            q8hip.argmax(self.ctx, self.a.buf, olg, self.cfg.vocab, self.ids, 0)
        nxt = int(self.ids.download((1,), np.int32)[0])
        self.a.reset(mark)
        self.n_cached += s
        self.posbuf.upload(np.array([self.n_cached], dtype=np.int32))
        return nxt

    # ---- captured decode step -------------------------------------------------
    def capture_decode(self) -> None:
        """Capture one decode step as a HIP graph that reads the token's
        embedding row and the device position and ends by writing the argmax
        to ids[0], advancing the position and (fused) gathering the next
        token's embedding row into the step's input: every launch of a
        token in one graph, no host work between tokens."""
        if self.graph is not None:
            return
        ctx, H = self.ctx, self.cfg.hidden
        mark = self.a.mark()
        self.graph_x = self.a.alloc(H)          # the step's input row (persistent)
        self.ctx.graph_begin()
        try:
            if self.fuse:
                oh = self._layers(self.graph_x, 1, 0, True)
                olg = self._head_argmax(oh, posbuf=self.posbuf, onext=self.graph_x)
            else:
                olg = self._run(1, 0, True)
                q8hip.argmax(ctx, self.a.buf, olg, self.cfg.vocab, self.ids, 0)
                q8hip.pos_advance(ctx, self.posbuf, 0, 1)
        finally:
            self.graph = self.ctx.graph_end()
        self.graph_logits = olg
        self.graph_mark = mark
        # the captured step owns its arena slice for the model's lifetime

    def prime_decode(self, first_id: int) -> None:
        """Set up replays of the captured step: the token id, the device
        position (the cached length) and, for the fused step, the first
        token's embedding row in the step's input."""
        self.capture_decode()
        self.ids.upload(np.array([first_id], dtype=np.int32))
        self.posbuf.upload(np.array([self.n_cached], dtype=np.int32))
        if self.fuse:
            q8hip.embed_gather(self.ctx, self.w.buf, self.w.o("model.embed_tokens.weight"),
                               self.ids, 0, self.a.buf, self.graph_x, 1, self.cfg.hidden,
                               self.cfg.vocab, self.G, self.scale)

    def decode_steps(self, first_id: int, n: int) -> list[int]:
        """Greedy-decode n tokens starting from first_id at the current
        position by replaying the captured step; returns the n ids."""
        if self.n_cached + n > self.maxlen:
            raise RuntimeError("KV cache full")
        self.prime_decode(first_id)
        out = []
        for _ in range(n):
            self.graph.launch()
            out.append(int(self.ids.download((1,), np.int32)[0]))
        self.n_cached += n
        return out

    def decode_steps_nosync(self, first_id: int, n: int) -> None:
        """n replays of the captured step without host readback (timing)."""
        if self.n_cached + n > self.maxlen:
            raise RuntimeError("KV cache full")
        self.prime_decode(first_id)
        for _ in range(n):
            self.graph.launch()
        self.n_cached += n

    def reset(self) -> None:
        """Forget the cached context (positions restart at 0)."""
        self.n_cached = 0
        self.posbuf.upload(np.zeros(4, dtype=np.int32))

    def close(self) -> None:
        if self.graph is not None:
            self.graph.destroy()
            self.graph = None
        for b in (self.w.buf, self.a.buf, self.kv, self.ids, self.posbuf):
            b.free()
