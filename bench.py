#!/usr/bin/env python3
"""Benchmark of the Q8 (INT8 group-quantized, W8A32) linear path on one MI355X.

Default workload -- Llama-3.2-1B decode step, batch 1: every Q8 linear of
one decode step, as run_layer_q8 issues them (src/llama_q8.mojo:159-225,
qwen3_mojo/src/qwen_q8.mojo:139-145):
    16 layers x [ fused q|k|v 2048->3072, o 2048->2048,
                  fused gate|up 2048->16384, down 8192->2048 ]
    + tied lm_head 2048->128256
= 65 Q8 GEMVs streaming 1.274 GB of packed weights (G=64, f16 scales).
Weights are random bf16 ~N(0, 0.02) per tensor, packed on the GPU by
q8_quantize_pack into one weight arena (PAD head, tensors contiguous, so
q|k|v and gate|up run fused); activations are synthetic ~N(0, 1).

A step is one pass over all 65 GEMVs, replayed from one HIP graph.  `value`
is weight-stream throughput in GB/s: algorithmic bytes per step
(sum over GEMVs of n*(m + (m/G)*scale_bytes) + 4*s*m + 4*s*n) divided by the
time per step (HIP events on the library's stream around K replays).

`roofline` is for the lm_head GEMV (the largest launch, 128256 x 2048):
its algorithmic bytes per launch divided by its average launch duration,
timed with HIP events around back-to-back launches that alternate between
two copies of the table (542 MB, more than the 256 MB Infinity Cache).

`cpu_baseline` runs the oracle's group-major fp32 restatement of k_mm_q8
(oracle/q8_oracle.c, OpenMP) over the same packed weights on the host cores.

Other workloads (--workload):
  linear   one Q8 linear 8192x2048, x f32 [1, 2048], weights rotated over
           >= 64 copies (>= 1.1 GB) so no launch reads a cached matrix
  prefill  Llama-3.2-1B prefill linears, M = 512 bf16 activations, all 16
           layers x 7 unfused projections on the MFMA GEMM (TFLOP/s)
  qwen8b   Qwen3-8B decode step, --batch 1 / 4 / 16
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
                   choices=["decode", "linear", "prefill", "qwen8b"])
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
                     "traffic": None,
                     "kernel": f"lm_head GEMV {n_h}x{m_h}: {head_bytes} B/launch, "
                               f"{head_ms * 1e3:.2f} us avg over {kk} launches"},
        "cpu_baseline": cpu,
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
    kmax = max(m for _, m in shapes)
    nmax = max(n for n, _ in shapes)
    x = B.activations(M * kmax, 3, bf16=True)
    y = torch.empty(M * nmax, device="cuda", dtype=torch.float32)
    xb = q8hip.Buffer.wrap(ctx, x.data_ptr(), x.numel() * 2)
    yb = q8hip.Buffer.wrap(ctx, y.data_ptr(), y.numel() * 4)
    flops = sum(2 * M * n * m for n, m in shapes)
    launches = [(lambda i=i: q8hip.linear_bf16act(ctx, w, offs[i], xb, 0, yb, 0, M,
                                                  shapes[i][1], shapes[i][0], G, scale))
                for i in range(len(shapes))]
    graph = B.capture(launches)
    step = B.run_graph_or_eager(graph, launches)
    ms, wall = B.time_steps(step, max(args.steps // 5, 5), args.warmup)
    tflops = flops / (ms * 1e-3) / 1e12
    # roofline kernel: the gate/up GEMM 512 x 8192 x 2048 (largest per-layer shape)
    gi = 4
    kk = max(args.steps, 20)
    gms, _ = B.time_steps(lambda: launches[gi](), kk, 3)
    gflop = 2 * M * shapes[gi][0] * shapes[gi][1]
    g_tflops = gflop / (gms * 1e-3) / 1e12
    if graph is not None:
        graph.destroy()
    w.free()
    return {
        "metric": "Q8 prefill GEMM TFLOP/s (% of dense bf16 MFMA peak), Llama-3.2-1B M=512",
        "value": round(tflops, 2), "unit": "TFLOP/s", "ms_per_step": round(ms, 4),
        "higher_is_better": True, "dtype": "bf16xint8->f32", "data": "synthetic",
        "config": {"workload": f"{cfg['name']} prefill linears, M={M} bf16 activations, "
                               f"{cfg['layers']} layers x 7 projections ({len(shapes)} GEMMs)",
                   "layout": f"G={G} {scale} scales", "flops_per_step": flops,
                   "pct_mfma_peak": round(100 * tflops / BF16_PEAK_TFLOPS, 2),
                   "graph": graph is not None, "wall_s": round(wall, 3)},
        "roofline": {"bound": "mfma", "achieved": round(g_tflops, 2), "peak": BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(g_tflops / BF16_PEAK_TFLOPS, 4),
                     "traffic": None,
                     "kernel": f"GEMM {M}x{shapes[gi][0]}x{shapes[gi][1]}: {gflop} flop/launch, "
                               f"{gms * 1e3:.2f} us avg"},
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
        args.layout = "g32f32" if args.workload == "linear" else "g64f16"
    import torch
    from lama32_mojo_amd import q8hip
    ctx = q8hip.Context(0)
    B = Bench(args, ctx, torch)
    if args.workload == "decode":
        res = run_decode(B, LLAMA_1B)
    elif args.workload == "qwen8b":
        res = run_decode(B, QWEN3_8B)
    elif args.workload == "linear":
        res = run_linear(B)
    else:
        res = run_prefill(B)
    out = {"metric": res.pop("metric"), "value": res.pop("value"), "unit": res.pop("unit"),
           "n_gpus": 1, "steps": args.steps, "warmup": args.warmup}
    out.update(res)
    out.update({"scaling": "weak", "vs_baseline": None})
    order = ["metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
             "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config",
             "roofline", "cpu_baseline"]
    print(json.dumps({k: out[k] for k in order if k in out}), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
