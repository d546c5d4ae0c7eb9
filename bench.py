#!/usr/bin/env python3
"""Benchmark: Qwen3-30B-A3B-shaped MoE-only decode stack at batch 1.

Workload: 48 MoE layers (D=2048, 128 experts, top-8,
expert intermediate 768, SMOE-Q4 g64), all ~15.4 GB of Q4 experts resident in
HBM, synthetic weights N(0, 0.02) from the counter-based generator, router
bf16 N(0, 0.02), norm weights 1.  One step = one token through all 48 MoE
blocks (RMSNorm -> router -> top-k -> fused Q4 expert FFN -> weighted combine
-> residual); step t+1 consumes step t's hidden state.  A step is captured
once as a HIP graph and replayed.

    python bench.py [--gpus 1] [--steps 256] [--warmup 16] [--config 30b|235b]

Prints one JSON line (metric, value = tok/s, roofline of the dominant kernel
from HIP events on its own stream, cpu_baseline = the oracle timed on a
bounded sample on this host).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "s-moe_amd"))

CONFIGS = {
    # 48-layer 30B-A3B stack, 256 decode steps
    "30b": dict(D=2048, E=128, K=8, I=768, layers=48, workload="qwen3-30b-a3b-moe-decode-stack"),
    # 94-layer 235B-A22B stack (~121 GB resident)
    "235b": dict(D=4096, E=128, K=8, I=1536, layers=94, workload="qwen3-235b-a22b-moe-decode-stack"),
}
HBM_PEAK_GBS = 8000.0
SEED = 20261201


def kernel_bytes(c):
    """Algorithmic HBM bytes per launch of each decode kernel (one token-layer)."""
    D, E, K, I = c["D"], c["E"], c["K"], c["I"]
    mat = D * I // 2 + D * I // 64 * 2            # packed nibbles + fp16 scales of one matrix
    return {
        # router bf16 + norm weights + hidden in + 8 experts' gate+up + h out
        "moe_up": E * D * 2 + D * 2 + D * 4 + K * 2 * mat + K * I * 4,
        # 8 experts' down + h in + weights + hidden read and written
        "moe_down": K * mat + K * I * 4 + K * 4 + 2 * D * 4,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--config", default="30b", choices=sorted(CONFIGS))
    ap.add_argument("--layers", type=int, default=0, help="override the layer count (0: config's)")
    ap.add_argument("--no-graph", action="store_true", help="launch eagerly instead of replaying a graph")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-layers", type=int, default=0, help="layers in the CPU sample (0: all)")
    ap.add_argument("--profile-steps", type=int, default=4)
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the expert-parallel design for more GPUs is described in DESIGN.md)", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import smoe_amd

    c = dict(CONFIGS[args.config])
    if args.layers:
        c["layers"] = args.layers
    D, E, K, I, NL = c["D"], c["E"], c["K"], c["I"], c["layers"]
    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    ctx = smoe_amd.Context()
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    ctx.set_stream(stream.cuda_stream)

    shape = smoe_amd.make_shape(D, E, K, I)
    off, raw, stride = smoe_amd.blob_layout(D, I)
    pool = torch.empty(NL * E * stride, dtype=torch.uint8, device=dev)
    ctx.synth_expert_pool(pool.data_ptr(), 0, NL, E, stride, shape, SEED, 0.02)
    router = torch.empty((NL, E * D), dtype=torch.int16, device=dev)
    for l in range(NL):
        ctx.synth_bf16(router[l].data_ptr(), E * D, SEED, smoe_amd.router_stream(l), 0.02)
    norm_w = torch.full((D,), 0x3F80, dtype=torch.int16, device=dev)
    hidden0 = torch.empty(D, dtype=torch.float32, device=dev)
    ctx.synth_normal(hidden0.data_ptr(), D, SEED, smoe_amd.hidden_stream(0), 1.0)
    hidden = hidden0.clone()
    layers = [smoe_amd.make_layer(norm_w.data_ptr(), router[l].data_ptr(), pool.data_ptr() + l * E * stride,
                                  stride, off) for l in range(NL)]
    ctx.reserve(shape, 1)
    torch.cuda.synchronize()

    def step():
        for l in range(NL):
            ctx.moe_decode(shape, layers[l], hidden.data_ptr(), 1)

    graph = None
    if not args.no_graph:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            step()
        torch.cuda.synchronize()
        run = graph.replay
    else:
        run = step

    hidden.copy_(hidden0)
    for _ in range(args.warmup):
        run()
    torch.cuda.synchronize()

    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        run()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = ev0.elapsed_time(ev1)
    elapsed = max(wall, gpu_ms / 1e3)
    ms_per_step = elapsed * 1e3 / args.steps
    tok_s = args.steps / elapsed

    if args.profile_steps <= 0:
        print(json.dumps({"value": round(tok_s, 2), "ms_per_step": round(ms_per_step, 4)}), flush=True)
        ctx.close()
        return
    # per-kernel durations: HIP events around each launch on the launch stream
    ctx.profile_enable(True)
    for _ in range(args.profile_steps):
        step()
    torch.cuda.synchronize()
    kb = kernel_bytes(c)
    kern = {}
    for kid, name in ((smoe_amd.KERNEL_MOE_UP, "moe_up"), (smoe_amd.KERNEL_MOE_DOWN, "moe_down")):
        n, ms = ctx.profile_read(kid)
        if n:
            avg_us = ms * 1e3 / n
            kern[name] = dict(launches=n, avg_us=round(avg_us, 3), bytes=kb[name],
                              gbs=round(kb[name] / (avg_us * 1e-6) / 1e9, 1))
    ctx.profile_enable(False)
    dom = max(kern, key=lambda k: kern[k]["avg_us"] * kern[k]["launches"])
    layer_bytes = kb["moe_up"] + kb["moe_down"]
    layer_us = kern["moe_up"]["avg_us"] + kern["moe_down"]["avg_us"]
    roofline = {
        "bound": "hbm", "kernel": dom,
        "achieved": kern[dom]["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": round(kern[dom]["gbs"] / HBM_PEAK_GBS, 4), "traffic": None,
        "bytes_per_launch": kb[dom], "avg_us": kern[dom]["avg_us"],
    }

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(ctx, c, shape, pool, router, norm_w, hidden0, stride, off, args.cpu_layers or NL)

    line = {
        "metric": "MoE decode tok/s & achieved HBM GB/s, Qwen3-30B/235B-shaped Q4 layers",
        "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (counter-based N(0,0.02) weights quantized to SMOE-Q4; N(0,1) hidden)",
        "config": {"workload": c["workload"], "d_model": D, "n_experts": E, "top_k": K, "d_ff": I,
                   "layers": NL, "batch": 1, "decode_steps": args.steps,
                   "quant": "SMOE-Q4 g64 fp16 absmax", "launch": "hip-graph" if graph else "eager",
                   "resident_expert_bytes": NL * E * raw},
        "roofline": roofline,
        "kernels": kern,
        "layer_kernels_gbs": round(layer_bytes / (layer_us * 1e-6) / 1e9, 1),
        "layer_gbs_in_stack": round((sum(kb.values())) * NL * tok_s / 1e9, 1),
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    ctx.close()


def cpu_baseline(ctx, c, shape, pool, router, norm_w, hidden0, stride, off, n_layers):
    """The oracle (CPU restatement, one thread) on one decode step through
    n_layers layers of the same stack; each layer's weights are copied to the
    host before its timed region.  Also reports how far the GPU's one-step
    result is from it (layers run teacher-forced on the oracle's own state)."""
    import numpy as np
    import torch

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    D, E, K, I = c["D"], c["E"], c["K"], c["I"]
    oshape = dict(d_model=D, n_experts=E, top_k=K, d_ff=I, group_size=64, norm_topk=1)
    h_norm = norm_w.cpu().numpy().view(np.uint16)
    h = hidden0.cpu().numpy().astype(np.float32)
    gpu_h = hidden0.clone()
    total = 0.0
    id_mismatch = 0
    worst = 0.0
    layer_bytes = E * stride
    for l in range(n_layers):
        h_pool = pool[l * layer_bytes:(l + 1) * layer_bytes].cpu().numpy()
        h_router = router[l].cpu().numpy().view(np.uint16)
        # GPU on the oracle's input (teacher forcing keeps the comparison per layer)
        gpu_h.copy_(torch.from_numpy(h))
        ids = torch.zeros(K, dtype=torch.int32, device="cuda")
        lay = __import__("smoe_amd").make_layer(norm_w.data_ptr(), router[l].data_ptr(),
                                                pool.data_ptr() + l * layer_bytes, stride, off)
        ctx.moe_decode(shape, lay, gpu_h.data_ptr(), 1, ids.data_ptr())
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        out, oid, ow, _lg, _nr, yo = O.moe_decode_layer(oshape, h_norm, h_router, h_pool, stride, off, h)
        total += time.perf_counter() - t0
        g = gpu_h.cpu().numpy()
        id_mismatch += int((ids.cpu().numpy().view(np.uint32) != oid).sum())
        dref = (ow.astype(np.float64)[:, None] * yo.astype(np.float64)).sum(0)
        tau = 1e-2 * np.sqrt(np.mean(dref ** 2))
        diff = np.maximum(np.abs((g.astype(np.float64) - h) - dref) - np.spacing(np.abs(g)), 0.0)
        worst = max(worst, float(np.max(diff / np.maximum(np.abs(dref), tau))))
        h = out
    return {
        "value": round(1.0 / total * (n_layers / c["layers"]), 4) if total > 0 else None,
        "unit": "tok/s", "cores": 1, "kind": "port",
        "sample": f"1 decode step through {n_layers} of {c['layers']} layers (batch 1), oracle single thread; "
                  f"value scaled to a full {c['layers']}-layer step; {total:.2f} s of CPU work",
        "cpu_seconds": round(total, 3),
        "parity_vs_gpu": {"ids_mismatch": id_mismatch, "max_rel_err_moe_delta": float(f"{worst:.3e}")},
    }


if __name__ == "__main__":
    main()
