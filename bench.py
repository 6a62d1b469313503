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

A step is one pass over all 65 GEMVs, replayed from a HIP graph.  `value`
is weight-stream throughput in GB/s: algorithmic bytes per step
(sum over GEMVs of n*(m + (m/G)*scale_bytes) + 4*s*m + 4*s*n) divided by the
measured time per step (HIP events on the library's stream).

`roofline` is for the lm_head GEMV launch (the largest single launch,
128256 x 2048): its algorithmic bytes divided by its average duration,
timed with HIP events around each of its launches inside the timed region.

`cpu_baseline` runs the oracle's group-major fp32 restatement of k_mm_q8
(oracle/q8_oracle.c, OpenMP) over the same packed weights on the host cores.

Other workloads (--workload): linear (one 8192x2048 Q8 linear, weights
rotated over >= 1 GiB of copies), prefill (Llama-3.2-1B M=512 bf16 GEMMs),
qwen8b (Qwen3-8B decode step, --batch 1/4/16).
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
    p.add_argument("--layout", default="g64f16", choices=["g64f16", "g32f32"])
    p.add_argument("--batch", type=int, default=1)
    p.add_argument("--no-graph", action="store_true", help="launch eagerly, no HIP graph")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    return p.parse_args()


def layout(args):
    return (64, "f16", 2) if args.layout == "g64f16" else (32, "f32", 4)


def linear_bytes(s, m, n, G, sb):
    return n * (m + (m // G) * sb) + 4 * s * m + 4 * s * n


class Setup:
    """Weight + activation arenas for a list of Q8 linears."""

    def __init__(self, ctx, torch, G, scale, sb):
        self.ctx, self.torch, self.G, self.scale, self.sb = ctx, torch, G, scale, sb

    def pack_tensors(self, shapes, seeds, w_arena_bytes_extra=0):
        """shapes: list of (n, m); packs each into the weight arena; returns u16 offsets."""
        from lama32_mojo_amd import q8, q8hip
        torch = self.torch
        PAD = q8.PAD
        offs, top = [], PAD
        for n, m in shapes:
            offs.append(top)
            top += n * q8hip.rowstride_u16(m, self.G, self.scale)
        self.w = q8hip.Buffer.alloc(self.ctx, 2 * top + w_arena_bytes_extra)
        for (n, m), off, seed in zip(shapes, offs, seeds):
            gen = torch.Generator(device="cuda")
            gen.manual_seed(seed)
            wt = (torch.randn((n, m), device="cuda", dtype=torch.float32, generator=gen)
                  * 0.02).to(torch.bfloat16)
            torch.cuda.synchronize()
            src = q8hip.Buffer.wrap(self.ctx, wt.data_ptr(), wt.numel() * 2)
            q8hip.quantize_pack(self.ctx, src, 0, q8hip.Q8_SRC_BF16, n, m, self.w, off,
                                self.G, self.scale)
            self.ctx.sync()
            src.free()
            del wt
        return offs, top


def timed_events(torch, stream):
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    return s, e


def cpu_baseline(packs, G, scale, budget_s, label):
    """Time the oracle's group-major fp32 GEMV over host copies of the packed
    weights; returns (GB/s, threads, sample description)."""
    from oracle.q8_oracle import c_oracle
    cor = c_oracle()
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    rng = np.random.default_rng(5)
    xs = {}
    t0 = time.perf_counter()
    done_bytes = 0
    reps = 0
    while True:
        for pk, s, m in packs:
            if (s, m) not in xs:
                xs[(s, m)] = rng.standard_normal((s, m), dtype=np.float32)
            cor.linear_f32(pk, xs[(s, m)], G, scale)
            done_bytes += linear_bytes(s, m, pk.shape[0], G, 2 if scale == "f16" else 4)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    return done_bytes / el / 1e9, threads, f"{reps} x {label} on {threads} threads, {el:.1f} s"


def decode_linears(cfg, batch):
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


def run_decode(args, ctx, torch, cfg):
    from lama32_mojo_amd import q8hip
    G, scale, sb = layout(args)
    S = Setup(ctx, torch, G, scale, sb)
    shapes, seeds = decode_linears(cfg, args.batch)
    offs, _ = S.pack_tensors(shapes, seeds)
    s = args.batch
    # activation arena: x and y per linear (x fixed synthetic, y written)
    aoffs, top = [], 32
    for n, m in shapes:
        aoffs.append((top, top + s * m))
        top += s * m + s * n
    a = q8hip.Buffer.alloc(ctx, 4 * top)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(1)
    xa = torch.randn(top, device="cuda", dtype=torch.float32, generator=gen)
    torch.cuda.synchronize()
    xa_np = xa.cpu().numpy()
    a.upload(xa_np)
    step_bytes = sum(linear_bytes(s, m, n, G, sb) for n, m in shapes)
    head = len(shapes) - 1

    def launch(i):
        n, m = shapes[i]
        ox, oy = aoffs[i]
        q8hip.linear(ctx, S.w, offs[i], a, ox, oy, s, m, n, G, scale)

    stream = torch.cuda.ExternalStream(ctx.stream)
    hs, he = timed_events(torch, stream)

    def step_eager(time_head=None):
        for i in range(len(shapes)):
            if i == head and time_head is not None:
                time_head[0].record(stream)
                launch(i)
                time_head[1].record(stream)
            else:
                launch(i)

    graph = None
    if not args.no_graph:
        ctx.graph_begin()
        for i in range(head):
            launch(i)
        g_layers = ctx.graph_end()
        ctx.graph_begin()
        launch(head)
        g_head = ctx.graph_end()
        graph = (g_layers, g_head)

    def step(time_head=None):
        if graph is None:
            step_eager(time_head)
            return
        graph[0].launch()
        if time_head is not None:
            time_head[0].record(stream)
        graph[1].launch()
        if time_head is not None:
            time_head[1].record(stream)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    head_ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in range(args.steps)]
    t_start, t_end = timed_events(torch, stream)
    torch.cuda.synchronize()
    t_start.record(stream)
    w0 = time.perf_counter()
    for k in range(args.steps):
        step(head_ev[k])
    t_end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    ms = t_start.elapsed_time(t_end) / args.steps
    head_ms = float(np.mean([e0.elapsed_time(e1) for e0, e1 in head_ev]))
    n_h, m_h = shapes[head]
    head_bytes = linear_bytes(s, m_h, n_h, G, sb)
    achieved = head_bytes / (head_ms * 1e-3) / 1e9
    value = step_bytes / (ms * 1e-3) / 1e9

    cpu = None
    if not args.no_cpu:
        # host copies of one layer's packed weights plus the lm_head
        packs = []
        for i in list(range(4)) + [head]:
            n, m = shapes[i]
            rs = q8hip.rowstride_u16(m, G, scale)
            pk = S.w.download((n, rs), np.uint16, 2 * offs[i])
            packs.append((pk, s, m))
        gbs, threads, sample = cpu_baseline(packs, G, scale, args.cpu_seconds,
                                            f"(layer-0 q|k|v, o, gate|up, down + lm_head)")
        cpu = {"value": round(gbs, 2), "unit": "GB/s", "cores": threads, "kind": "port",
               "sample": sample + "; oracle/q8_oracle.c q8o_linear_f32 (group-major fp32 "
               "restatement of k_mm_q8), " + cpu_model()}

    res = {
        "metric": "Q8 GEMV GB/s (% of HBM peak); decode tok/s batch 1, " + cfg["name"] + " Q8",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8xf32",
        "data": "synthetic (random-init N(0,0.02) bf16 weights packed on GPU; x ~ N(0,1))",
        "config": {"workload": f"{cfg['name']} decode step batch {s}: all Q8 linears "
                               f"({len(shapes)} GEMVs, fused qkv/gate|up, tied lm_head)",
                   "layout": f"G={G} {scale} scales", "batch": s,
                   "bytes_per_step": step_bytes, "graph": graph is not None,
                   "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 1),
                   "linears_only_tok_per_s": round(1000.0 / ms, 1),
                   "wall_s": round(wall, 3)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": None,
                     "kernel": f"lm_head GEMV {n_h}x{m_h} ({head_bytes} B/launch, "
                               f"{head_ms * 1e3:.2f} us avg)"},
        "cpu_baseline": cpu,
    }
    if graph is not None:
        graph[0].destroy()
        graph[1].destroy()
    return res


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": f"--gpus {args.gpus}: this benchmark runs on exactly one GPU; "
                                   "multi-GPU runs are not part of this build"}))
        sys.exit(2)
    import torch
    from lama32_mojo_amd import q8hip
    ctx = q8hip.Context(0)
    if args.workload == "decode":
        res = run_decode(args, ctx, torch, LLAMA_1B)
    elif args.workload == "qwen8b":
        res = run_decode(args, ctx, torch, QWEN3_8B)
    else:
        raise SystemExit(f"workload {args.workload} not implemented yet")
    print(json.dumps(res), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
