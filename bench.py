#!/usr/bin/env python3
"""Benchmark of the Q8 (INT8 group-quantized, W8A32) path on one MI355X.

Default workload -- Llama-3.2-1B decode step, batch 1, at a KV context of
1024 tokens: the whole token step of the reference's Q8 model
(qwen3_mojo/src/qwen_q8.mojo:127-162 with run_layer_q8,
src/llama_q8.mojo:144-230) on libq8hip -- embedding gather, 16 layers of
[rmsnorm + fused q|k|v GEMV 2048->3072, RoPE + fp16 KV append + attention
(context splits, then their merge), o GEMV 2048->2048 + residual, rmsnorm +
fused gate|up GEMV 2048->16384 + swiglu, down GEMV 8192->2048 + residual],
final rmsnorm + tied lm_head GEMV 2048->128256, argmax: six launches per
layer, the norms, swiglu and residual adds folded into the GEMVs.  Weights
are random bf16 ~N(0, 0.02) per tensor, packed on the GPU by
q8_quantize_pack into one weight arena (G=64, f16 scales: the reference
layout); norms ~1; the 1024-token KV context is random fp16.

A step is one token: one replay of a HIP graph that reads the token id and
the position from device memory and writes the argmax id and the next
position back.  `value` is the step's streaming throughput in GB/s: packed
weight bytes (1.274 GB) plus the KV bytes read at the step's context length,
divided by the time per token (HIP events on the library's stream around K
replays); config.tok_s is tokens per second.

`roofline` is for the lm_head GEMV (the largest launch, 128256 x 2048):
its algorithmic bytes per launch divided by its average launch duration,
timed with HIP events around back-to-back launches that alternate between
two copies of the table (542 MB, more than the 256 MB Infinity Cache).

`cpu_baseline` runs the oracle's group-major fp32 restatement of k_mm_q8
(oracle/q8_oracle.c, OpenMP) over the same packed weights on the host cores.

Other workloads (--workload):
  decode-linears  only the 65 Q8 GEMVs of the Llama-3.2-1B step, one graph
  linear   one Q8 linear 8192x2048, x f32 [1, 2048], weights rotated over
           >= 64 copies (>= 1.1 GB) so no launch reads a cached matrix
  prefill  Llama-3.2-1B prefill linears, M = 512 bf16 activations, all 16
           layers x 7 projections (q|k|v and gate|up as one GEMM each over
           their adjacent rows) on the f16-MFMA dequant-GEMM (TFLOP/s), group 32
  qwen8b   Qwen3-8B decode linears, --batch 1 / 4 / 16, group 32
  e2e-8b   Llama-3.1-8B end to end: prefill of 2048 random ids (seed 3),
           then 256 greedy decode steps (one HIP graph per token); value is
           decode tok/s, config holds the prefill time
  qwen3-06b  the reference's own Q8 model, Qwen3-0.6B (q/k head norms, tied
           lm_head 1024 -> 151936), decode step at KV context 128; value is
           tok/s, vs_baseline against the reference's published 29 tok/s
           (Apple M4, QUANTIZATION.md:28)
  lmhead-pmc  the launches the HBM-traffic counter passes read: 3 copies of
           1 GiB by torch's copy kernel (the calibration of known size), then
           8 lm_head GEMVs 128256x2048 alternating over two tables

`roofline.traffic` (default workload) is the lm_head GEMV's HBM bytes per
launch measured by rocprofv3 FETCH_SIZE and WRITE_SIZE passes over
--workload lmhead-pmc, each scaled by the copy kernel's known bytes / its
counter reading; the figures are read from profiles/lm_head_gemv_pmc.md.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0

LLAMA_1B = dict(name="Llama-3.2-1B", hidden=2048, layers=16, heads=32, kv_heads=8,
                head_dim=64, inter=8192, vocab=128256)
QWEN3_8B = dict(name="Qwen3-8B", hidden=4096, layers=36, heads=32, kv_heads=8,
                head_dim=128, inter=12288, vocab=151936)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--workload", default="decode",
                   choices=["decode", "decode-linears", "linear", "prefill", "qwen8b",
                            "e2e-8b", "lmhead-pmc", "qwen3-06b"])
    p.add_argument("--layout", default=None, choices=["g64f16", "g32f32"],
                   help="packed layout (default: g64f16; g32f32 for --workload linear)")
    p.add_argument("--batch", type=int, default=1)
    p.add_argument("--no-graph", action="store_true", help="launch eagerly, no HIP graph")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    return p.parse_args()


def layout(name):
    return (64, "f16", 2) if name == "g64f16" else (32, "f32", 4)


def linear_bytes(s, m, n, G, sb):
    return n * (m + (m // G) * sb) + 4 * s * m + 4 * s * n


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


class Bench:
    def __init__(self, args, ctx, torch):
        from lama32_mojo_amd import q8hip
        self.q8hip = q8hip
        self.args, self.ctx, self.torch = args, ctx, torch
        self.G, self.scale, self.sb = layout(args.layout)
        self.stream = torch.cuda.ExternalStream(ctx.stream)

    # ---- weights --------------------------------------------------------------
    def pack_arena(self, shapes, seeds):
        """Pack random bf16 weights of the given (n, m) shapes into one arena
        (PAD head, contiguous); returns (buffer, u16 offsets)."""
        q8hip, torch = self.q8hip, self.torch
        offs, top = [], 32
        for n, m in shapes:
            offs.append(top)
            top += n * q8hip.rowstride_u16(m, self.G, self.scale)
        w = q8hip.Buffer.alloc(self.ctx, 2 * top)
        for (n, m), off, seed in zip(shapes, offs, seeds):
            gen = torch.Generator(device="cuda")
            gen.manual_seed(seed)
            wt = (torch.randn((n, m), device="cuda", dtype=torch.float32, generator=gen)
                  * 0.02).to(torch.bfloat16)
            torch.cuda.synchronize()
            src = q8hip.Buffer.wrap(self.ctx, wt.data_ptr(), wt.numel() * 2)
            q8hip.quantize_pack(self.ctx, src, 0, q8hip.Q8_SRC_BF16, n, m, w, off,
                                self.G, self.scale)
            self.ctx.sync()
            src.free()
            del wt
        return w, offs

    def activations(self, count, seed, bf16=False):
        torch = self.torch
        gen = torch.Generator(device="cuda")
        gen.manual_seed(seed)
        t = torch.randn(count, device="cuda", dtype=torch.float32, generator=gen)
        if bf16:
            t = t.to(torch.bfloat16)
        torch.cuda.synchronize()
        return t

    # ---- timing -----------------------------------------------------------------
    def events(self):
        torch = self.torch
        return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def time_steps(self, step, steps, warmup):
        torch = self.torch
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        e0, e1 = self.events()
        e0.record(self.stream)
        w0 = time.perf_counter()
        for _ in range(steps):
            step()
        e1.record(self.stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps, time.perf_counter() - w0

    def capture(self, launches):
        """HIP graph of a list of launch closures (None when --no-graph)."""
        if self.args.no_graph:
            return None
        self.ctx.graph_begin()
        for f in launches:
            f()
        return self.ctx.graph_end()

    def run_graph_or_eager(self, graph, launches):
        if graph is not None:
            return lambda: graph.launch()
        return lambda: [f() for f in launches]


# ---------------------------------------------------------------------------
# decode (Llama-3.2-1B / Qwen3-8B)
# ---------------------------------------------------------------------------

def decode_shapes(cfg):
    H, QD = cfg["hidden"], cfg["heads"] * cfg["head_dim"]
    KVD, I, V = cfg["kv_heads"] * cfg["head_dim"], cfg["inter"], cfg["vocab"]
    per_layer = [(QD + 2 * KVD, H), (H, QD), (2 * I, H), (H, I)]
    shapes, seeds = [], []
    for L in range(cfg["layers"]):
        for p, sh in enumerate(per_layer):
            shapes.append(sh)
            seeds.append(100 * L + p)
    shapes.append((V, H))
    seeds.append(99999)
    return shapes, seeds


def run_decode(B: Bench, cfg):
    args, q8hip, ctx = B.args, B.q8hip, B.ctx
    G, scale, sb = B.G, B.scale, B.sb
    s = args.batch
    shapes, seeds = decode_shapes(cfg)
    head = len(shapes) - 1
    n_h, m_h = shapes[head]
    # lm_head twice (second copy only for the roofline timing loop)
    w, offs = B.pack_arena(shapes + [shapes[head]], seeds + [seeds[head] + 1])
    aoffs, top = [], 32
    for n, m in shapes:
        aoffs.append((top, top + s * m))
        top += s * m + s * n
    xa = B.activations(top, 1)
    a = q8hip.Buffer.wrap(ctx, xa.data_ptr(), 4 * top)
    step_bytes = sum(linear_bytes(s, m, n, G, sb) for n, m in shapes)

    def launcher(i, woff=None):
        n, m = shapes[i]
        ox, oy = aoffs[i]
        wo = offs[i] if woff is None else woff
        return lambda: q8hip.linear(ctx, w, wo, a, ox, oy, s, m, n, G, scale)

    launches = [launcher(i) for i in range(len(shapes))]
    graph = B.capture(launches)
    step = B.run_graph_or_eager(graph, launches)
    ms, wall = B.time_steps(step, args.steps, args.warmup)
    value = step_bytes / (ms * 1e-3) / 1e9

    # roofline kernel: lm_head GEMV, back-to-back over two copies
    heads = [launcher(head), launcher(head, offs[head + 1])]
    kk = max(args.steps, 20)
    head_ms, _ = B.time_steps(lambda: [h() for h in heads], kk // 2, 2)
    head_ms /= 2
    head_bytes = linear_bytes(s, m_h, n_h, G, sb)
    achieved = head_bytes / (head_ms * 1e-3) / 1e9

    cpu = None
    if not args.no_cpu:
        packs = []
        for i in list(range(4)) + [head]:
            n, m = shapes[i]
            rs = q8hip.rowstride_u16(m, G, scale)
            pk = w.download((n, rs), np.uint16, 2 * offs[i])
            packs.append((pk, s, m))
        cpu = cpu_baseline(packs, G, scale, args.cpu_seconds,
                           "(layer-0 q|k|v, o, gate|up, down + lm_head)")
    if graph is not None:
        graph.destroy()
    w.free()
    return {
        "metric": f"Q8 GEMV GB/s (% of HBM peak); decode tok/s batch {s}, {cfg['name']} Q8",
        "value": round(value, 1),
        "unit": "GB/s",
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "dtype": "int8xf32",
        "data": "synthetic (random-init N(0,0.02) bf16 weights packed on GPU; x ~ N(0,1))",
        "config": {"workload": f"{cfg['name']} decode step batch {s}: all Q8 linears "
                               f"({len(shapes)} GEMVs, fused qkv / gate|up, lm_head "
                               f"{n_h}x{m_h})",
                   "layout": f"G={G} {scale} scales", "batch": s,
                   "bytes_per_step": step_bytes, "graph": graph is not None,
                   "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 1),
                   "linears_only_steps_per_s": round(1000.0 / ms, 1),
                   "wall_s": round(wall, 3)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(G, sb),
                     "kernel": f"lm_head GEMV {n_h}x{m_h}: {head_bytes} B/launch, "
                               f"{head_ms * 1e3:.2f} us avg over {kk} launches"},
        "cpu_baseline": cpu,
    }


# ---------------------------------------------------------------------------
# full decode step (Llama-3.2-1B model on the layer kernels, captured graph)
# ---------------------------------------------------------------------------

def measured_traffic(G: int, sb: int):
    """The lm_head GEMV's HBM bytes per launch from the committed counter
    passes (profiles/lm_head_gemv_pmc.md), for the layout they measured."""
    if (G, sb) != (64, 2):
        return None
    try:
        with open(os.path.join(ROOT, "profiles", "lm_head_gemv_pmc.md")) as f:
            for line in f:
                if line.strip().startswith("- traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def run_decode_model(B: Bench, ctxlen: int = 1024, cfg=None, tok_metric: bool = False):
    from lama32_mojo_amd import model as gm

    args, q8hip, ctx, torch = B.args, B.q8hip, B.ctx, B.torch
    G, scale, sb = B.G, B.scale, B.sb
    cfg = cfg or gm.LLAMA_32_1B
    K, W = args.steps, args.warmup
    maxlen = ctxlen + W + K + 8
    m = gm.Q8Llama(ctx, cfg, maxlen, G, scale, seed=7)
    # a context of ctxlen cached tokens: random binary16 K/V rows (their
    # values do not change the work of a step)
    kvd = cfg.kv_dim()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(11)
    kvt = torch.empty(2 * cfg.layers * maxlen * kvd, dtype=torch.float16, device="cuda")
    kvt.normal_(generator=gen)
    torch.cuda.synchronize()
    src = q8hip.Buffer.wrap(ctx, kvt.data_ptr(), kvt.numel() * 2)
    # copy through the host once (the cache is a library buffer)
    m.kv.upload(src.download((kvt.numel(),), np.float16))
    src.free()
    del kvt
    m.n_cached = ctxlen
    m.prime_decode(128000 % cfg.vocab)
    ms, wall = B.time_steps(lambda: m.graph.launch(), K, W)
    pos_end = int(m.posbuf.download((1,), np.int32)[0])
    assert pos_end == ctxlen + W + K, pos_end
    weight_bytes = 2 * (m.w.top - 32)
    mean_ctx = ctxlen + W + (K + 1) / 2.0
    kv_bytes = int(cfg.layers * 2 * mean_ctx * kvd * 2)
    step_bytes = weight_bytes + kv_bytes
    value = step_bytes / (ms * 1e-3) / 1e9
    tok_s = 1000.0 / ms

    # roofline kernel: the lm_head GEMV (tied embed table), back-to-back over
    # two copies so the 256 MB MALL cannot serve it
    n_h, m_h = cfg.vocab, cfg.hidden
    w2, offs2 = B.pack_arena([(n_h, m_h), (n_h, m_h)], [5, 6])
    xa = B.activations(32 + m_h + n_h, 1)
    a = q8hip.Buffer.wrap(ctx, xa.data_ptr(), 4 * (32 + m_h + n_h))
    heads = [(lambda o=o: q8hip.linear(ctx, w2, o, a, 32, 32 + m_h, 1, m_h, n_h, G, scale))
             for o in offs2]
    kk = max(K, 20)
    head_ms, _ = B.time_steps(lambda: [h() for h in heads], kk // 2, 2)
    head_ms /= 2
    head_bytes = linear_bytes(1, m_h, n_h, G, sb)
    achieved = head_bytes / (head_ms * 1e-3) / 1e9
    w2.free()

    cpu = None
    if not args.no_cpu:
        lo = m.lo[0]
        H, QD, KVD, I = cfg.hidden, cfg.q_dim(), cfg.kv_dim(), cfg.inter
        packs = []
        for off, n, mm in [(lo.q, QD + 2 * KVD, H), (lo.o, H, QD), (lo.gate, 2 * I, H),
                           (lo.down, H, I), (m.w.o("model.embed_tokens.weight"), n_h, m_h)]:
            rs = q8hip.rowstride_u16(mm, G, scale)
            packs.append((m.w.buf.download((n, rs), np.uint16, 2 * off), 1, mm))
        cpu = cpu_baseline(packs, G, scale, args.cpu_seconds,
                           "(layer-0 q|k|v, o, gate|up, down + lm_head)")
    m.close()
    if tok_metric:
        # the reference's published Q8 figure: Qwen3-0.6B decode, batch 1,
        # 22-29 tok/s on an Apple M4 GPU (QUANTIZATION.md:28)
        head = {"metric": f"decode tok/s batch 1, {cfg.name} Q8", "value": round(tok_s, 1),
                "unit": "tok/s", "vs_baseline": round(tok_s / 29.0, 1)}
    else:
        head = {"metric": f"Q8 GEMV GB/s (% of HBM peak); decode tok/s batch 1, {cfg.name} Q8",
                "value": round(value, 1), "unit": "GB/s"}
    return {
        **head,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "dtype": "int8xf32",
        "data": "synthetic (random-init N(0,0.02) bf16 weights packed on GPU, norms ~1; "
                "random fp16 KV context)",
        "config": {"workload": f"{cfg.name} decode step batch 1 at KV context {ctxlen}: "
                               f"embedding gather, {cfg.layers} layers (rmsnorm + fused "
                               "q|k|v GEMV, "
                               + ("q/k head norms + " if cfg.qk_norm else "")
                               + "RoPE + fp16 KV append + attention, merge, o GEMV "
                               "+ residual, rmsnorm + fused gate|up GEMV + swiglu, down GEMV "
                               f"+ residual), final norm + lm_head GEMV {n_h}x{m_h}, argmax; "
                               "one HIP graph per token",
                   "layout": f"G={G} {scale} scales", "batch": 1, "tok_s": round(tok_s, 1),
                   "weight_bytes_per_token": weight_bytes, "kv_bytes_per_token": kv_bytes,
                   "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 1),
                   "graph": True, "wall_s": round(wall, 3)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(G, sb),
                     "kernel": f"lm_head GEMV {n_h}x{m_h}: {head_bytes} B/launch, "
                               f"{head_ms * 1e3:.2f} us avg over {kk} launches"},
        "cpu_baseline": cpu,
    }


def run_lmhead_pmc(B: Bench):
    """The launches the counter passes read (see the module docstring)."""
    q8hip, ctx, torch = B.q8hip, B.ctx, B.torch
    G, scale, sb = B.G, B.scale, B.sb
    nbytes = 1 << 30
    src = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda").normal_()
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    n_h, m_h = LLAMA_1B["vocab"], LLAMA_1B["hidden"]
    w2, offs2 = B.pack_arena([(n_h, m_h), (n_h, m_h)], [5, 6])
    xa = B.activations(32 + m_h + n_h, 1)
    a = q8hip.Buffer.wrap(ctx, xa.data_ptr(), 4 * (32 + m_h + n_h))
    for i in range(8):
        q8hip.linear(ctx, w2, offs2[i % 2], a, 32, 32 + m_h, 1, m_h, n_h, G, scale)
    ctx.sync()
    w2.free()
    return {"metric": "counter-pass launches (no timing)", "value": 0, "unit": "none",
            "ms_per_step": 0.0, "higher_is_better": True, "dtype": "int8xf32",
            "data": "synthetic", "config": {"workload": "3 x 1 GiB copy, 8 x lm_head GEMV "
                                                        f"{n_h}x{m_h}",
                                            "copy_bytes": nbytes,
                                            "lm_head_bytes": linear_bytes(1, m_h, n_h, G, sb)}}


def run_e2e_8b(B: Bench, prompt: int = 2048, gen: int = 256):
    """Llama-3.1-8B: prefill `prompt` random ids, then `gen` greedy steps."""
    from lama32_mojo_amd import model as gm

    args, q8hip, ctx, torch = B.args, B.q8hip, B.ctx, B.torch
    G, scale, sb = B.G, B.scale, B.sb
    cfg = gm.LLAMA_31_8B
    m = gm.Q8Llama(ctx, cfg, prompt + gen + 8, G, scale, seed=3, max_prefill=prompt)
    ids = np.random.default_rng(3).integers(0, cfg.vocab, size=prompt).tolist()
    m.forward_argmax(ids[:64])                 # warm-up: first launches, then forget
    m.reset()
    torch.cuda.synchronize()
    e0, e1 = B.events()
    e0.record(B.stream)
    first = m.forward_argmax(ids)
    e1.record(B.stream)
    torch.cuda.synchronize()
    prefill_ms = e0.elapsed_time(e1)
    # decode: capture, then replays that read the previous id on the device
    steps = gen - 1
    warm = min(args.warmup, 8)
    m.decode_steps(first, warm)
    ms, wall = B.time_steps(lambda: m.graph.launch(), steps - warm, 0)
    m.n_cached += steps - warm
    assert int(m.posbuf.download((1,), np.int32)[0]) == prompt + steps
    tok_s = 1000.0 / ms
    H, L, QD, KVD, I = cfg.hidden, cfg.layers, cfg.q_dim(), cfg.kv_dim(), cfg.inter
    lin_flops = 2.0 * prompt * L * H * (QD + 2 * KVD + I * 3) + 2.0 * prompt * L * QD * H
    weight_bytes = 2 * (m.w.top - 32)

    # roofline kernel: the untied lm_head GEMV 128256 x 4096 over two copies
    n_h, m_h = cfg.vocab, cfg.hidden
    w2, offs2 = B.pack_arena([(n_h, m_h), (n_h, m_h)], [5, 6])
    xa = B.activations(32 + m_h + n_h, 1)
    a = q8hip.Buffer.wrap(ctx, xa.data_ptr(), 4 * (32 + m_h + n_h))
    heads = [(lambda o=o: q8hip.linear(ctx, w2, o, a, 32, 32 + m_h, 1, m_h, n_h, G, scale))
             for o in offs2]
    head_ms, _ = B.time_steps(lambda: [h() for h in heads], 10, 2)
    head_ms /= 2
    head_bytes = linear_bytes(1, m_h, n_h, G, sb)
    achieved = head_bytes / (head_ms * 1e-3) / 1e9
    w2.free()
    m.close()
    return {
        "metric": f"decode tok/s batch 1 after a {prompt}-token prefill, {cfg.name} Q8",
        "value": round(tok_s, 1),
        "unit": "tok/s",
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "dtype": "int8xf32",
        "data": "synthetic (random-init N(0,0.02) bf16 weights packed on GPU, norms ~1; "
                "random prompt ids, seed 3)",
        "config": {"workload": f"{cfg.name} end to end: prefill {prompt} ids (7 Q8 GEMMs per "
                               "layer as f16-MFMA dequant-GEMMs, RoPE + "
                               "fp16 KV append, causal attention), then "
                               f"{gen} greedy steps of the captured decode graph",
                   "layout": f"G={G} {scale} scales", "batch": 1,
                   "prefill_ms": round(prefill_ms, 2),
                   "prefill_linear_tflops": round(lin_flops / (prefill_ms * 1e-3) / 1e12, 1),
                   "decode_ms_per_token": round(ms, 4),
                   "decode_weight_gbs": round(weight_bytes / (ms * 1e-3) / 1e9, 1),
                   "e2e_ms": round(prefill_ms + gen * ms, 1), "wall_s": round(wall, 3)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": None,
                     "kernel": f"lm_head GEMV {n_h}x{m_h}: {head_bytes} B/launch, "
                               f"{head_ms * 1e3:.2f} us avg over 10 launches"},
        "cpu_baseline": None,
    }


# ---------------------------------------------------------------------------
# single linear (8192 x 2048, rotated copies)
# ---------------------------------------------------------------------------

def run_linear(B: Bench):
    args, q8hip, ctx = B.args, B.q8hip, B.ctx
    G, scale, sb = B.G, B.scale, B.sb
    n, m, s = 8192, 2048, args.batch
    one = linear_bytes(s, m, n, G, sb)
    copies = 64
    w, offs = B.pack_arena([(n, m)] * copies, list(range(copies)))
    xa = B.activations(s * m + s * n + 32, 2)
    a = q8hip.Buffer.wrap(ctx, xa.data_ptr(), xa.numel() * 4)
    launches = [(lambda o=o: q8hip.linear(ctx, w, o, a, 0, s * m, s, m, n, G, scale))
                for o in offs]
    graph = B.capture(launches)
    step = B.run_graph_or_eager(graph, launches)
    ms, wall = B.time_steps(step, max(args.steps // 4, 5), args.warmup)
    per_launch_ms = ms / copies
    value = one / (per_launch_ms * 1e-3) / 1e9
    cpu = None
    if not args.no_cpu:
        rs = q8hip.rowstride_u16(m, G, scale)
        pk = w.download((n, rs), np.uint16, 2 * offs[0])
        cpu = cpu_baseline([(pk, s, m)], G, scale, args.cpu_seconds, f"{n}x{m} linear")
    if graph is not None:
        graph.destroy()
    w.free()
    return {
        "metric": "Q8 GEMV GB/s (% of HBM peak), single linear",
        "value": round(value, 1), "unit": "GB/s",
        "ms_per_step": round(per_launch_ms, 5), "higher_is_better": True,
        "dtype": "int8xf32", "data": "synthetic",
        "config": {"workload": f"single Q8 linear {n}x{m}, x f32 [{s},{m}], "
                               f"{copies} rotated weight copies ({copies * one / 1e9:.2f} GB)",
                   "layout": f"G={G} {scale} scales", "bytes_per_launch": one,
                   "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 1),
                   "graph": graph is not None, "wall_s": round(wall, 3)},
        "roofline": {"bound": "hbm", "achieved": round(value, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(value / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": f"GEMV {n}x{m}: {one} B/launch, {per_launch_ms * 1e3:.2f} us avg"},
        "cpu_baseline": cpu,
    }


# ---------------------------------------------------------------------------
# prefill GEMMs (Llama-3.2-1B, M = 512, bf16 activations)
# ---------------------------------------------------------------------------

def run_prefill(B: Bench, cfg=LLAMA_1B, M=512):
    args, q8hip, ctx, torch = B.args, B.q8hip, B.ctx, B.torch
    G, scale = B.G, B.scale
    H, QD = cfg["hidden"], cfg["heads"] * cfg["head_dim"]
    KVD, I = cfg["kv_heads"] * cfg["head_dim"], cfg["inter"]
    per_layer = [(QD, H), (KVD, H), (KVD, H), (H, QD), (I, H), (I, H), (H, I)]
    shapes, seeds = [], []
    for L in range(cfg["layers"]):
        for p, sh in enumerate(per_layer):
            shapes.append(sh)
            seeds.append(100 * L + p)
    w, offs = B.pack_arena(shapes, seeds)
    flops = sum(2 * M * n * m for n, m in shapes)
    # q|k|v and gate|up share their input and their packed rows are adjacent
    # in the arena, so each trio / pair is one GEMM over the stacked rows
    # (the same products; the decode step stacks them the same way)
    gemms = []
    for L in range(cfg["layers"]):
        b = 7 * L
        gemms += [(offs[b], QD + 2 * KVD, H), (offs[b + 3], H, QD), (offs[b + 4], 2 * I, H),
                  (offs[b + 6], H, I)]
    assert sum(2 * M * n * m for _, n, m in gemms) == flops
    kmax = max(m for _, _, m in gemms)
    nmax = max(n for _, n, _ in gemms)
    x = B.activations(M * kmax, 3, bf16=True)
    y = torch.empty(M * nmax, device="cuda", dtype=torch.float32)
    xb = q8hip.Buffer.wrap(ctx, x.data_ptr(), x.numel() * 2)
    yb = q8hip.Buffer.wrap(ctx, y.data_ptr(), y.numel() * 4)
    launches = [(lambda o=o, n=n, m=m: q8hip.linear_bf16act(ctx, w, o, xb, 0, yb, 0, M, m, n,
                                                            G, scale))
                for o, n, m in gemms]
    graph = B.capture(launches)
    step = B.run_graph_or_eager(graph, launches)
    ms, wall = B.time_steps(step, max(args.steps // 5, 5), args.warmup)
    tflops = flops / (ms * 1e-3) / 1e12
    # roofline kernel: the gate|up GEMM 512 x 16384 x 2048 (largest per-layer
    # shape), timed per call with its binary16 pre-pass included
    gi = 2
    kk = max(args.steps, 20)
    gms, _ = B.time_steps(lambda: launches[gi](), kk, 3)
    gflop = 2 * M * gemms[gi][1] * gemms[gi][2]
    g_tflops = gflop / (gms * 1e-3) / 1e12
    if graph is not None:
        graph.destroy()
    w.free()
    return {
        "metric": "Q8 prefill GEMM TFLOP/s (% of dense bf16 MFMA peak), Llama-3.2-1B M=512",
        "value": round(tflops, 2), "unit": "TFLOP/s", "ms_per_step": round(ms, 4),
        "higher_is_better": True, "dtype": "f16(q*s) x f16(x) -> f32", "data": "synthetic",
        "config": {"workload": f"{cfg['name']} prefill linears, M={M} bf16 activations, "
                               f"{cfg['layers']} layers x 7 projections as {len(gemms)} GEMMs "
                               "(q|k|v and gate|up stacked)",
                   "layout": f"G={G} {scale} scales", "flops_per_step": flops,
                   "pct_mfma_peak": round(100 * tflops / BF16_PEAK_TFLOPS, 2),
                   "graph": graph is not None, "wall_s": round(wall, 3)},
        "roofline": {"bound": "mfma", "achieved": round(g_tflops, 2), "peak": BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(g_tflops / BF16_PEAK_TFLOPS, 4),
                     "traffic": None,
                     "kernel": f"GEMM {M}x{gemms[gi][1]}x{gemms[gi][2]} (+ binary16 pre-pass): "
                               f"{gflop} flop/launch, {gms * 1e3:.2f} us avg"},
        "cpu_baseline": None,
    }


def cpu_baseline(packs, G, scale, budget_s, label):
    """The oracle's group-major fp32 restatement of k_mm_q8 over host copies
    of the packed weights, on the host cores (OpenMP)."""
    from oracle.q8_oracle import c_oracle
    cor = c_oracle()
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    rng = np.random.default_rng(5)
    xs = {}
    t0 = time.perf_counter()
    done_bytes = 0
    reps = 0
    sb = 2 if scale == "f16" else 4
    while True:
        for pk, s, m in packs:
            if (s, m) not in xs:
                xs[(s, m)] = rng.standard_normal((s, m), dtype=np.float32)
            cor.linear_f32(pk, xs[(s, m)], G, scale)
            done_bytes += linear_bytes(s, m, pk.shape[0], G, sb)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    return {"value": round(done_bytes / el / 1e9, 2), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": f"{reps} x {label} on {threads} threads in {el:.1f} s; "
                      f"oracle/q8_oracle.c q8o_linear_f32 (group-major fp32 restatement "
                      f"of k_mm_q8), {cpu_model()}"}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": f"--gpus {args.gpus}: this benchmark runs on exactly one "
                                   "GPU; multi-GPU runs are not part of this build"}))
        sys.exit(2)
    if args.layout is None:
        # the reference layout for the Llama-3.2-1B decode step; group 32
        # with f32 scales where the workload is defined with it
        args.layout = ("g64f16" if args.workload in ("decode", "decode-linears", "e2e-8b",
                                                     "lmhead-pmc", "qwen3-06b")
                       else "g32f32")
    import torch
    from lama32_mojo_amd import q8hip
    ctx = q8hip.Context(0)
    B = Bench(args, ctx, torch)
    if args.workload == "decode":
        res = run_decode_model(B)
    elif args.workload == "decode-linears":
        res = run_decode(B, LLAMA_1B)
    elif args.workload == "qwen3-06b":
        from lama32_mojo_amd import model as gm
        res = run_decode_model(B, ctxlen=128, cfg=gm.QWEN3_06B, tok_metric=True)
    elif args.workload == "lmhead-pmc":
        res = run_lmhead_pmc(B)
    elif args.workload == "e2e-8b":
        res = run_e2e_8b(B)
    elif args.workload == "qwen8b":
        res = run_decode(B, QWEN3_8B)
    elif args.workload == "linear":
        res = run_linear(B)
    else:
        res = run_prefill(B)
    out = {"metric": res.pop("metric"), "value": res.pop("value"), "unit": res.pop("unit"),
           "n_gpus": 1, "steps": args.steps, "warmup": args.warmup}
    out.update(res)
    out["scaling"] = "weak"
    out.setdefault("vs_baseline", None)
    order = ["metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
             "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config",
             "roofline", "cpu_baseline"]
    print(json.dumps({k: out[k] for k in order if k in out}), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
