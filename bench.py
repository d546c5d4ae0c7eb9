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
    python bench.py --rocprof-summary DIR [--pmc-out FILE]   (summarise a rocprofv3 run)

Prints one JSON line: metric, value = tok/s over the timed replays, the
roofline of the dominant kernel (its average duration from HIP start/stop
events that its own dispatches record on the launch stream), parity = the
timed engine against the CPU oracle on step 0 (teacher-forced and end to
end), cpu_baseline = the CPU oracle timed on a bounded sample on this host,
and configs = BASELINE.json's other configs measured in the same run:
configs[2] (the 94-layer 235B stack), configs[3] (512-token prefill, one 30B
layer) and configs[4] (64 Zipf tokens, one 235B layer).
"""
from __future__ import annotations

import argparse
import csv
import glob
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
MFMA_F16_PEAK_TFLOPS = 2500.0    # dense f16 / bf16 MFMA, MI355X
SEED = 20261201
KERNEL_SYMBOLS = {"moe_up": "k_moe_up", "moe_down": "k_down_combine", "moe_layer": "k_moe_layer",
                  "moe_chain": "k_moe_chain"}


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def kernel_bytes(c):
    """Algorithmic HBM bytes per launch of each decode kernel: one token-layer
    for the one- and two-launch paths; one token through every layer for the
    whole-step kernels (per layer the same bytes as one k_moe_layer launch:
    k * B_expert + 2 E D router + 2 D norm weights + 4 D hidden in + 4 D out)."""
    D, E, K, I = c["D"], c["E"], c["K"], c["I"]
    # packed nibbles + fp16 scales of one matrix (scale+min format: + bf16 mins)
    mat = D * I // 2 + D * I // 64 * 2 * (2 if c.get("quant") else 1)
    # the whole block: router bf16 + norm weights + 8 experts' gate/up/down + hidden in and out
    layer = K * 3 * mat + 2 * E * D + 2 * D + 8 * D
    return {
        "moe_chain": c["layers"] * layer,
        "moe_layer": layer,
        # router bf16 + norm weights + hidden in + 8 experts' gate+up + h out
        "moe_up": E * D * 2 + D * 2 + D * 4 + K * 2 * mat + K * I * 4,
        # 8 experts' down + h in + weights + hidden read and written
        "moe_down": K * mat + K * I * 4 + K * 4 + 2 * D * 4,
    }


def pmc_traffic(kernel, workload):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 --pmc
    summary (FETCH_SIZE + WRITE_SIZE, each scaled by the copy-kernel
    calibration), or None when no summary for this kernel and workload exists."""
    path = os.path.join(ROOT, "profiles", "pmc_traffic.json")
    try:
        with open(path) as f:
            data = json.load(f)
    except (OSError, ValueError):
        return None
    ent = data.get(workload, {}).get(KERNEL_SYMBOLS[kernel], {})
    return int(ent["traffic_bytes"]) if "traffic_bytes" in ent else None


def calibrate_copy(args, dev):
    """For PMC runs: a plain streaming kernel of known size, b = -a over N MiB
    of fp32 (reads N MiB and writes N MiB), against which FETCH_SIZE and
    WRITE_SIZE are scaled."""
    if not args.calibrate_copy_mib:
        return
    import torch
    n = (args.calibrate_copy_mib << 20) // 4
    a = torch.ones(n, dtype=torch.float32, device=dev)
    b = torch.empty_like(a)
    for _ in range(4):
        torch.neg(a, out=b)
    torch.cuda.synchronize()
    del a, b
    log(f"counter calibration: 4 x neg over {args.calibrate_copy_mib} MiB")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--config", default="30b", choices=sorted(CONFIGS))
    ap.add_argument("--workload", default="decode", choices=("decode", "prefill", "batched", "vault", "prefill_stack", "trunk"),
                    help="decode: the 48/94-layer batch-1 stack (default); prefill: 512 tokens through one "
                         "30B layer (configs[3]); batched: 64 tokens through one 235B layer with a Zipf "
                         "router (configs[4]); vault: .smoe vault -> HBM pool load rate (--layers layers "
                         "of the --config shape, default 4); prefill_stack: a 512-token prompt through the "
                         "whole --config MoE stack, whole prompt per layer vs the reference's 64-token chunks; trunk: the "
                         "dense-trunk GEMV and decode attention layer (30B head layout)")
    ap.add_argument("--replicas", type=int, default=4, help="prefill/batched: layer replicas rotated")
    ap.add_argument("--layers", type=int, default=0, help="override the layer count (0: config's)")
    ap.add_argument("--no-graph", action="store_true", help="launch eagerly instead of replaying a graph")
    ap.add_argument("--engine", default="chain", choices=("stack", "split", "chain", "layers"),
                    help="chain: smoe_hip_moe_decode_stack, one launch per step (default); stack: the same "
                         "entry point with one launch per layer; split: two launches per layer; layers: one "
                         "smoe_hip_moe_decode call per layer")
    ap.add_argument("--no-configs", action="store_true",
                    help="decode: skip the configs block (configs 3, 4 and 5 after the headline)")
    ap.add_argument("--quant", default="smoeq4", choices=("smoeq4", "scale_min"),
                    help="decode: the 4-bit group format of the experts (smoeq4: the reference's fp16 absmax; "
                         "scale_min: a bf16 scale and min per group, the configs' wording)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU work the baseline sample aims at")
    ap.add_argument("--profile-steps", type=int, default=8, help="replays of the event-timed step (0: skip)")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="first run a plain streaming kernel over this many MiB (PMC calibration)")
    ap.add_argument("--rocprof-summary", metavar="DIR", help="summarise a rocprofv3 output directory and exit")
    ap.add_argument("--pmc-out", metavar="FILE", help="with --rocprof-summary: merge PMC traffic into FILE")
    args = ap.parse_args()

    if args.rocprof_summary:
        rocprof_summary(args.rocprof_summary, args.config, args.pmc_out, args.calibrate_copy_mib, args.workload)
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(over more GPUs the path would shard by expert: a dispatch of the normed tokens and a "
              "combine of the weighted expert outputs per layer; not built here)", file=sys.stderr)
        sys.exit(2)

    import torch

    import smoe_amd

    if args.workload == "vault":
        vault_bench(args)
        return
    if args.workload == "prefill_stack":
        prefill_stack_bench(args)
        return
    if args.workload == "trunk":
        trunk_bench(args)
        return
    if args.workload != "decode":
        line = grouped_line(args.workload, args.replicas, max(4, args.steps // 8), max(1, args.warmup // 4),
                            args.calibrate_copy_mib)
        print(json.dumps(line), flush=True)
        return

    line = decode_line(args, args.config, args.steps, args.warmup, cpu=not args.no_cpu_baseline)
    if not args.no_configs and args.config == "30b" and not args.layers:
        # the other configs of BASELINE.json, measured in the same run on
        # fixed, short schedules (the headline above is configs[1])
        torch.cuda.empty_cache()
        line["configs"] = configs_block(args)
    print(json.dumps(line), flush=True)


def configs_block(args):
    """configs[2] (the 94-layer 235B stack), configs[3] (512-token prefill
    through one 30B layer) and configs[4] (64 Zipf tokens through one 235B
    layer): throughput, time per call, roofline fraction of the dominant
    kernel and its counter traffic where a committed summary holds it."""
    import torch
    out = {}
    sub = argparse.Namespace(**vars(args))
    sub.layers = 0
    sub.calibrate_copy_mib = 0
    sub.profile_steps = 4
    d = decode_line(sub, "235b", 32, 4, cpu=False)
    out["3"] = {k: d[k] for k in ("value", "unit", "ms_per_step", "steps", "warmup", "config", "roofline")}
    out["3"]["us_per_layer"] = round(d["ms_per_step"] * 1e3 / d["config"]["layers"], 2)
    out["3"]["parity"] = d.get("parity")
    torch.cuda.empty_cache()
    # config 2 again in the configs' literal format (bf16 scale and min per group)
    sub.quant = "scale_min"
    d = decode_line(sub, "30b", 64, 8, cpu=False)
    sub.quant = "smoeq4"
    out["2_scale_min"] = {k: d[k] for k in ("value", "unit", "ms_per_step", "steps", "warmup", "config", "roofline",
                                             "parity")}
    out["2_scale_min"]["us_per_layer"] = round(d["ms_per_step"] * 1e3 / d["config"]["layers"], 2)
    torch.cuda.empty_cache()
    for cid, wl in (("4", "prefill"), ("5", "batched")):
        g = grouped_line(wl, 4, 16, 2, 0)
        out[cid] = {k: g[k] for k in ("value", "unit", "us_per_layer_call", "layer_bytes", "layer_gbs",
                                      "layer_tflops", "config", "roofline", "mfma", "kernels", "steps")}
        out[cid]["layer_frac"] = round(g["layer_gbs"] / HBM_PEAK_GBS, 4)
        torch.cuda.empty_cache()
    return out


def decode_line(args, cname, steps, warmup, cpu=True):
    """The decode bench of one stack config: tok/s over `steps` timed graph
    replays of a whole step, the event-timed dominant kernel's roofline, the
    parity leg (through the timed engine) and, when `cpu`, the CPU baseline."""
    import torch

    import smoe_amd

    c = dict(CONFIGS[cname])
    if args.layers:
        c["layers"] = args.layers
    c["quant"] = smoe_amd.QUANT_Q4_SCALE_MIN if getattr(args, "quant", "smoeq4") == "scale_min" else 0
    if c["quant"]:
        c["workload"] += "-scale-min"
    D, E, K, I, NL = c["D"], c["E"], c["K"], c["I"], c["layers"]
    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    ctx = smoe_amd.Context()
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    ctx.set_stream(stream.cuda_stream)

    calibrate_copy(args, dev)

    shape = smoe_amd.make_shape(D, E, K, I, quant=c["quant"])
    off, raw, stride = smoe_amd.blob_layout(D, I, quant=c["quant"])
    log(f"generating {NL} layers x {E} experts ({NL * E * stride / 1e9:.1f} GB) on the GPU")
    pool = torch.empty(NL * E * stride, dtype=torch.uint8, device=dev)
    t_gen = time.perf_counter()
    for l0 in range(0, NL, 8):            # in chunks, with progress lines
        n = min(8, NL - l0)
        ctx.synth_expert_pool(pool.data_ptr() + l0 * E * stride, l0, n, E, stride, shape, SEED, 0.02)
        torch.cuda.synchronize()
        log(f"  layers {l0}..{l0 + n - 1} generated ({time.perf_counter() - t_gen:.1f} s)")
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
    layer_arr = (smoe_amd.SmoeMoeLayer * NL)(*layers)

    ctx.set_decode_engine({"chain": smoe_amd.DECODE_CHAIN,
                           "split": smoe_amd.DECODE_SPLIT}.get(args.engine, smoe_amd.DECODE_LAUNCHES))
    if args.engine in ("stack", "split", "chain"):

        def step():
            ctx.moe_decode_stack(shape, layer_arr, hidden.data_ptr())
    else:
        def step():
            for l in range(NL):
                ctx.moe_decode(shape, layers[l], hidden.data_ptr(), 1)
    step()                      # scratch and layer table, outside capture
    torch.cuda.synchronize()

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
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()

    # timed region: K steps, synchronised on both sides
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(steps):
        run()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = ev0.elapsed_time(ev1)
    elapsed = max(wall, gpu_ms / 1e3)
    ms_per_step = elapsed * 1e3 / steps
    tok_s = steps / elapsed
    log(f"{cname}: timed {steps} steps: {ms_per_step:.4f} ms/step, {tok_s:.1f} tok/s")
    ctx.synchronize()   # raises if a kernel reported an error (e.g. exchange time-out)

    line = {
        "metric": "MoE decode tok/s & achieved HBM GB/s, Qwen3-30B/235B-shaped Q4 layers",
        "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": steps,
        "warmup": warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None,
        "dtype": "f32 (Q4 weights; activations as 22-bit fixed point per 32-column chunk, exact int32 dot "
                 "products; fp32 router, softmax, SiLU and combine)",
        "data": "synthetic (counter-based N(0,0.02) weights quantized to SMOE-Q4; N(0,1) hidden)",
        "config": {"workload": c["workload"], "d_model": D, "n_experts": E, "top_k": K, "d_ff": I,
                   "layers": NL, "batch": 1, "decode_steps": steps,
                   "quant": "Q4 g64 bf16 scale + bf16 min" if c["quant"] else "SMOE-Q4 g64 fp16 absmax",
                   "launch": "hip-graph" if graph else "eager",
                   "engine": {"stack": "stack API, per-layer launches",
                              "split": "stack API, two launches per layer",
                              "chain": "stack API, one launch per step running the one-launch layer schedule "
                                       "layer after layer",
                              "layers": "one decode call per layer"}[args.engine],
                   "resident_expert_bytes": NL * E * raw},
    }

    if args.profile_steps > 0:
        kb = kernel_bytes(c)
        kern, how = kernel_times(ctx, torch, stream, step, args.profile_steps)
        for name, (n, avg_us) in kern.items():
            kern[name] = dict(launches=n, avg_us=round(avg_us, 3), bytes=kb[name],
                              gbs=round(kb[name] / (avg_us * 1e-6) / 1e9, 1))
        dom = max(kern, key=lambda k: kern[k]["avg_us"] * kern[k]["launches"])
        traffic = pmc_traffic(dom, c["workload"])
        line["roofline"] = {
            "bound": "hbm", "achieved": kern[dom]["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(kern[dom]["gbs"] / HBM_PEAK_GBS, 4), "traffic": traffic,
            "kernel": KERNEL_SYMBOLS[dom], "bytes_per_launch": kb[dom], "avg_us": kern[dom]["avg_us"],
            "timing": how,
        }
        ceil = stream_ceiling(ctx, torch, pool)
        if ceil:
            line["roofline"]["ceiling"] = ceil
            line["roofline"]["frac_of_ceiling"] = round(kern[dom]["gbs"] / ceil["achieved"], 4)
        line["kernels"] = kern
        layer_bytes = kb["moe_chain"] // NL
        line["layer_bytes"] = layer_bytes
        # whole-step algorithmic bytes over the timed step time (launch gaps included)
        line["stack_gbs"] = round(layer_bytes * NL * tok_s / 1e9, 1)

    ctx.synchronize()
    line["parity"] = parity_leg(ctx, c, shape, pool, router, norm_w, hidden0, stride, off, args.engine,
                                layer_arr, all_layers=cpu)
    if cpu:
        line["cpu_baseline"] = cpu_baseline(c, pool, router, norm_w, hidden0, stride, off, args.cpu_seconds)
    ctx.close()
    return line


def kernel_times(ctx, torch, stream, step, replays):
    """Average duration of each decode kernel: the step is replayed eagerly
    `replays` times with profiling on, so every launch carries HIP start/stop
    events that its own dispatch records on the launch stream
    (hipExtLaunchKernel) -- kernel execution time without launch gaps."""
    import smoe_amd
    ctx.profile_enable(True)
    for _ in range(replays):
        step()
    torch.cuda.synchronize()
    out = _read_profile(ctx, smoe_amd)
    ctx.profile_enable(False)
    return out, "hipExtLaunchKernel start/stop events on the launch stream, eager replays of the step"


def stream_ceiling(ctx, torch, pool, launches=6):
    """The device's streaming-read ceiling, measured in this run: k_stream_read
    over the first 2 GiB of the expert pool (8x the Infinity Cache), timed by
    its dispatch events like the decode kernels; the first launch is a
    warm-up."""
    import smoe_amd
    nbytes = min(pool.numel(), 2 << 30) // 4096 * 4096
    if nbytes < (256 << 20):
        return None
    sink = torch.zeros(1, dtype=torch.int32, device=pool.device)
    ctx.stream_read(pool.data_ptr(), nbytes, sink.data_ptr())
    torch.cuda.synchronize()
    ctx.profile_enable(True)
    for _ in range(launches):
        ctx.stream_read(pool.data_ptr(), nbytes, sink.data_ptr())
    torch.cuda.synchronize()
    n, ms = ctx.profile_read(smoe_amd.KERNEL_STREAM)
    ctx.profile_enable(False)
    if not n:
        return None
    us = ms * 1e3 / n
    gbs = nbytes / (us * 1e-6) / 1e9
    log(f"streaming-read ceiling: {nbytes / 2**30:.1f} GiB in {us:.1f} us = {gbs:.0f} GB/s")
    return {"achieved": round(gbs, 1), "unit": "GB/s", "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4),
            "kernel": "k_stream_read", "bytes": nbytes, "avg_us": round(us, 2),
            "how": "non-temporal 128-bit loads, 1 KiB per wave instruction, 8 in flight per wave, "
                   "2048 blocks x 4 waves, over the expert pool; dispatch events"}


def _read_profile(ctx, smoe_amd):
    out = {}
    for kid, name in ((smoe_amd.KERNEL_MOE_UP, "moe_up"), (smoe_amd.KERNEL_MOE_DOWN, "moe_down"),
                      (smoe_amd.KERNEL_MOE_LAYER, "moe_layer"), (smoe_amd.KERNEL_CHAIN, "moe_chain")):
        n, ms = ctx.profile_read(kid)
        if n:
            out[name] = (n, ms * 1e3 / n)
    return out


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo, as lscpu reports it)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.lower().startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _oracle():
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    return O


def parity_leg(ctx, c, shape, pool, router, norm_w, hidden0, stride, off, engine, layer_arr, all_layers=True):
    """How far the timed engine is from the CPU oracle on step 0 (the oracle
    is the checker here, never the thing measured):
    - teacher-forced: each layer run by the timed engine (a one-layer stack
      call: the chained kernel for the default engine) on the oracle's own
      input of that layer; ids must match exactly, the MoE delta is compared
      with the per-element metric of the parity tests;
    - end to end: the whole timed step from the same input, its per-layer ids
      against the oracle's free-running ones (layers agreeing before the first
      difference) and, if all agree, the final hidden state's error.
    all_layers=False checks layers 0, n/2 and n-1 teacher-forced only."""
    import numpy as np
    import torch

    import smoe_amd

    O = _oracle()
    D, E, K, I, NL = c["D"], c["E"], c["K"], c["I"], c["layers"]
    oshape = dict(d_model=D, n_experts=E, top_k=K, d_ff=I, group_size=64, norm_topk=1, quant=c.get("quant", 0))
    h_norm = norm_w.cpu().numpy().view(np.uint16)
    lb = E * stride
    cores = O.usable_cores()
    sel = range(NL) if all_layers else sorted({0, NL // 2, NL - 1})
    # the whole timed step, with its routing
    full = hidden0.clone()
    fids = torch.zeros((NL, K), dtype=torch.int32, device="cuda")
    if engine == "layers":
        for l in range(NL):
            lay = layer_arr[l]
            ctx.moe_decode(shape, lay, full.data_ptr(), 1, fids[l].data_ptr())
    else:
        ctx.moe_decode_stack(shape, layer_arr, full.data_ptr(), fids.data_ptr())
    torch.cuda.synchronize()
    fids = fids.cpu().numpy().view(np.uint32)
    h = hidden0.cpu().numpy().astype(np.float32)
    gpu_h = hidden0.clone()
    ids = torch.zeros(K, dtype=torch.int32, device="cuda")
    id_mismatch, worst, agree, first_diff = 0, 0.0, 0, None
    with O.threads(cores):
        for l in range(NL):
            hp = pool[l * lb:(l + 1) * lb].cpu().numpy()
            hr = router[l].cpu().numpy().view(np.uint16)
            out, oid, ow, _lg, _nr, yo = O.moe_decode_layer(oshape, h_norm, hr, hp, stride, off, h)
            if first_diff is None and (fids[l] == oid).all():
                agree += 1
            elif first_diff is None:
                first_diff = l
            if l in sel:
                gpu_h.copy_(torch.from_numpy(h))
                lay = (smoe_amd.SmoeMoeLayer * 1)(layer_arr[l])
                if engine == "layers":
                    ctx.moe_decode(shape, layer_arr[l], gpu_h.data_ptr(), 1, ids.data_ptr())
                else:
                    ctx.moe_decode_stack(shape, lay, gpu_h.data_ptr(), ids.data_ptr())
                torch.cuda.synchronize()
                g = gpu_h.cpu().numpy()
                id_mismatch += int((ids.cpu().numpy().view(np.uint32) != oid).sum())
                dref = (ow.astype(np.float64)[:, None] * yo.astype(np.float64)).sum(0)
                tau = 1e-2 * np.sqrt(np.mean(dref ** 2))
                diff = np.maximum(np.abs((g.astype(np.float64) - h) - dref) - np.spacing(np.abs(g)), 0.0)
                worst = max(worst, float(np.max(diff / np.maximum(np.abs(dref), tau))))
            h = out
    res = {"engine": {"chain": "k_moe_chain (one-layer stack calls)", "stack": "smoe_hip_moe_decode_stack, per-layer",
                      "split": "two launches per layer", "layers": "smoe_hip_moe_decode"}[engine],
           "teacher_forced": {"layers": len(sel), "ids_mismatch": id_mismatch,
                              "max_rel_err_moe_delta": float(f"{worst:.3e}"), "bound": 1e-3},
           "end_to_end": {"layers_ids_equal_before_first_difference": agree, "of": NL}}
    if first_diff is None:
        f = full.cpu().numpy().astype(np.float64)
        tau = 1e-2 * np.sqrt(np.mean(h.astype(np.float64) ** 2))
        res["end_to_end"]["final_hidden_max_rel_err"] = float(
            f"{np.max(np.abs(f - h) / np.maximum(np.abs(h), tau)):.3e}")
    log(f"{c['workload']}: parity {res}")
    return res


def cpu_baseline(c, pool, router, norm_w, hidden0, stride, off, target_s):
    """The CPU oracle (fp32 restatement of the reference's arithmetic) on whole
    decode steps of the same stack, timed two ways on this host: one thread
    (the reference's CPU routing code is single-threaded) and every usable
    core (OpenMP over output rows; each row keeps its sequential fp32 sum, so
    the results are bit-identical, which is asserted).  Each leg: one warm-up
    iteration, then the median of >= 5 timed iterations of whole steps, the
    iteration size chosen so a leg takes about `target_s` / 2 seconds.  Host
    copies of the weights are made before any timing.  For stacks too large
    for a quick host copy (the 94-layer 235B stack) a stated prefix of layers
    is timed and the per-layer time scaled to the whole stack."""
    import numpy as np

    O = _oracle()
    D, E, K, I, NL = c["D"], c["E"], c["K"], c["I"], c["layers"]
    oshape = dict(d_model=D, n_experts=E, top_k=K, d_ff=I, group_size=64, norm_topk=1, quant=c.get("quant", 0))
    h_norm = norm_w.cpu().numpy().view(np.uint16)
    layer_bytes = E * stride
    n_cpu = NL if NL * layer_bytes <= 20e9 else 8          # layers copied to the host
    log(f"cpu baseline: copying {n_cpu} of {NL} layers to host")
    h_pools = [pool[l * layer_bytes:(l + 1) * layer_bytes].cpu().numpy() for l in range(n_cpu)]
    h_routers = [router[l].cpu().numpy().view(np.uint16) for l in range(n_cpu)]
    cores = O.usable_cores()

    def run_layers(h):
        for l in range(n_cpu):
            h = O.moe_decode_layer(oshape, h_norm, h_routers[l], h_pools[l], stride, off, h)[0]
        return h

    def leg(n_threads, budget_s):
        """median seconds per pass over the n_cpu layers, and the passes
        per timed iteration"""
        with O.threads(n_threads):
            t0 = time.perf_counter()
            h_out = run_layers(hidden0.cpu().numpy().astype(np.float32))      # warm-up
            one = time.perf_counter() - t0
            per_iter = max(1, int(budget_s / 5 / max(one, 1e-6)))
            times = []
            while len(times) < 5 or (sum(times) < budget_s and len(times) < 15):
                t0 = time.perf_counter()
                for _ in range(per_iter):
                    run_layers(hidden0.cpu().numpy().astype(np.float32))
                times.append((time.perf_counter() - t0) / per_iter)
            log(f"cpu baseline: {n_threads} thread(s): {len(times)} iterations of {per_iter} pass(es), "
                f"median {np.median(times):.3f} s per pass over {n_cpu} layers")
        return float(np.median(times)), per_iter, len(times), h_out

    t1, it1, n1, h1 = leg(1, target_s / 2)
    tn, itn, nn, hn = leg(cores, target_s / 2)
    if not np.array_equal(h1, hn):
        raise SystemExit("bench.py: the threaded CPU oracle differs from the single-threaded one")
    scale = NL / n_cpu
    tok1, tokn = 1.0 / (t1 * scale), 1.0 / (tn * scale)
    expert_gb = (K * 3 * (D * I // 2 + D * I // 64 * 2) + 2 * E * D + 12 * D) * NL / 1e9
    subset = "" if n_cpu == NL else f" (first {n_cpu} of {NL} layers timed, scaled to {NL})"
    return {
        "value": round(tokn, 4), "unit": "tok/s", "cores": cores, "kind": "port",
        "sample": f"whole decode steps through the {NL}-layer stack (batch 1){subset}: oracle with OpenMP over "
                  f"output rows on {cores} threads, median of {nn} iterations of {itn} step(s) after a warm-up; "
                  f"weights copied to host before timing",
        "gbs": round(expert_gb * tokn, 3),
        "single_thread": {"value": round(tok1, 4), "unit": "tok/s", "cores": 1, "gbs": round(expert_gb * tok1, 3),
                          "sample": f"median of {n1} iterations of {it1} step(s){subset}"},
        "cpu_model": cpu_model(), "nproc": os.cpu_count(), "threads_bit_identical": True,
    }


# ---------------------------------------------------------------------------
# prefill and batched decode: the grouped path
# ---------------------------------------------------------------------------
GROUPED = {
    "prefill": dict(D=2048, E=128, K=8, I=768, T=512, zipf=None,
                    workload="qwen3-30b-a3b-moe-prefill-512"),
    "batched": dict(D=4096, E=128, K=8, I=1536, T=64, zipf=1.1,
                    workload="qwen3-235b-a22b-moe-batched-decode-64-zipf1.1"),
}


def trunk_bench(args):
    """Dense trunk around the MoE block: GB/s of the bf16 GEMV (an o_proj-sized
    and an lm_head-sized matrix) and time of one decode attention layer
    (Qwen3-30B-A3B layout: 32 query / 4 KV heads of 128, d_model 2048) at
    several context lengths.  Algorithmic bytes: the bf16 weights once, plus
    for attention the K and V rows of the valid positions (fp32) and x/outputs.
    Times from HIP events around --steps back-to-back calls on the stream."""
    import torch

    import smoe_amd

    ctx = smoe_amd.Context()
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    ctx.set_stream(stream.cuda_stream)
    steps = max(4, args.steps if args.steps != 256 else 50)

    def timed_us(fn):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / steps

    out = {"gemv": {}, "attention": {}}
    for name, (rows, cols) in (("o_proj_2048x4096", (2048, 4096)), ("lm_head_151936x2048", (151936, 2048))):
        w = torch.empty(rows * cols, dtype=torch.int16, device="cuda")
        ctx.synth_bf16(w.data_ptr(), rows * cols, SEED, 0xABC0 + rows, 0.02)
        x = torch.randn(cols, device="cuda")
        y = torch.empty(rows, device="cuda")
        us = timed_us(lambda: ctx.matvec_bf16(w.data_ptr(), x.data_ptr(), y.data_ptr(), rows, cols))
        b = rows * cols * 2 + cols * 4 + rows * 4
        out["gemv"][name] = {"us": round(us, 2), "bytes": b, "gbs": round(b / us / 1e3, 1),
                             "frac": round(b / us / 1e3 / HBM_PEAK_GBS, 3)}
        log(f"gemv {name}: {us:.2f} us, {b / us / 1e3:.0f} GB/s")
        del w
    d_model, nh, nkv, hd = 2048, 32, 4, 128
    q_dim, kv_dim = nh * hd, nkv * hd
    W = {}
    for i, (n, (r, c)) in enumerate(dict(q=(q_dim, d_model), k=(kv_dim, d_model), v=(kv_dim, d_model),
                                         o=(d_model, q_dim)).items()):
        W[n] = torch.empty(r * c, dtype=torch.int16, device="cuda")
        ctx.synth_bf16(W[n].data_ptr(), r * c, SEED, 0xABD0 + i, 0.02)
    nw = torch.full((hd,), 0x3F80, dtype=torch.int16, device="cuda")
    wbytes = sum(t.numel() * 2 for t in W.values())
    for ctx_len in (1024, 4096, 32768):
        kc = torch.randn(ctx_len, kv_dim, device="cuda")
        vc = torch.randn(ctx_len, kv_dim, device="cuda")
        buf = {n: torch.zeros(sz, device="cuda") for n, sz in (("x", d_model), ("q", q_dim), ("k", kv_dim),
                                                                ("v", kv_dim), ("att", q_dim), ("o", d_model),
                                                                ("cos", hd // 2), ("sin", hd // 2))}
        buf["x"].normal_()
        buf["cos"].fill_(1.0)
        a = smoe_amd.SmoeAttnLayerArgs()
        a.w_q, a.w_k, a.w_v, a.w_o = (W[n].data_ptr() for n in "qkvo")
        a.q_norm_w = a.k_norm_w = nw.data_ptr()
        a.rope_cos, a.rope_sin, a.normed_in = buf["cos"].data_ptr(), buf["sin"].data_ptr(), buf["x"].data_ptr()
        a.qbuf, a.kbuf, a.vbuf = buf["q"].data_ptr(), buf["k"].data_ptr(), buf["v"].data_ptr()
        a.k_cache, a.v_cache, a.attn_out, a.o_out = (kc.data_ptr(), vc.data_ptr(), buf["att"].data_ptr(),
                                                     buf["o"].data_ptr())
        a.d_model, a.q_dim, a.kv_dim, a.head_dim, a.num_heads, a.num_kv_heads = d_model, q_dim, kv_dim, hd, nh, nkv
        a.slot, a.valid, a.attn_ctx, a.attn_scale = ctx_len - 1, ctx_len, ctx_len, 1.0 / hd ** 0.5
        us = timed_us(lambda: ctx.attention_layer(a))
        b = wbytes + 2 * ctx_len * kv_dim * 4 + (d_model + q_dim) * 4
        out["attention"][f"ctx{ctx_len}"] = {"us": round(us, 2), "bytes": b, "gbs": round(b / us / 1e3, 1),
                                              "frac": round(b / us / 1e3 / HBM_PEAK_GBS, 3)}
        log(f"attention ctx {ctx_len}: {us:.2f} us, {b / us / 1e3:.0f} GB/s")
        del kc, vc
    ctx.synchronize()
    lm = out["gemv"]["lm_head_151936x2048"]
    line = {"metric": "dense-trunk bf16 GEMV GB/s (lm_head-sized)", "value": lm["gbs"], "unit": "GB/s",
            "n_gpus": 1, "steps": steps, "higher_is_better": True, "dtype": "bf16 weights, f32 accumulate",
            "data": "synthetic", "config": {"workload": "qwen3-30b-a3b-dense-trunk", "head_layout": "32q/4kv x 128"},
            **out}
    print(json.dumps(line), flush=True)
    ctx.close()


def prefill_stack_bench(args):
    """Tokens/s of a T=512 prompt through every MoE layer of the --config stack
    (smoe_hip_moe_prefill_stack; attention is not part of this path), with the
    whole prompt per layer and, as the reference walks it, in 64-token chunks
    (prefill.hpp:33): the chunked order streams every touched expert once per
    chunk instead of once per pass.  Same results either way (tokens are
    independent inside the MoE block)."""
    import torch

    import smoe_amd

    c = dict(CONFIGS[args.config])
    if args.layers:
        c["layers"] = args.layers
    D, E, K, I, NL = c["D"], c["E"], c["K"], c["I"], c["layers"]
    T, CH = 512, 64
    dev = torch.device("cuda", 0)
    ctx = smoe_amd.Context()
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    ctx.set_stream(stream.cuda_stream)
    shape = smoe_amd.make_shape(D, E, K, I)
    off, raw, stride = smoe_amd.blob_layout(D, I)
    log(f"prefill_stack: generating {NL} layers x {E} experts ({NL * E * stride / 1e9:.1f} GB)")
    pool = torch.empty(NL * E * stride, dtype=torch.uint8, device=dev)
    for l0 in range(0, NL, 8):
        n = min(8, NL - l0)
        ctx.synth_expert_pool(pool.data_ptr() + l0 * E * stride, l0, n, E, stride, shape, SEED, 0.02)
        torch.cuda.synchronize()
    router = torch.empty((NL, E * D), dtype=torch.int16, device=dev)
    for l in range(NL):
        ctx.synth_bf16(router[l].data_ptr(), E * D, SEED, smoe_amd.router_stream(l), 0.02)
    norm_w = torch.full((D,), 0x3F80, dtype=torch.int16, device=dev)
    h0 = torch.empty((T, D), dtype=torch.float32, device=dev)
    for t in range(T):
        ctx.synth_normal(h0[t].data_ptr(), D, SEED, smoe_amd.hidden_stream(t), 1.0)
    layers = (smoe_amd.SmoeMoeLayer * NL)(*[smoe_amd.make_layer(norm_w.data_ptr(), router[l].data_ptr(),
                                                                pool.data_ptr() + l * E * stride, stride, off)
                                           for l in range(NL)])
    hidden = h0.clone()

    def whole():
        ctx.moe_prefill_stack(shape, layers, hidden.data_ptr(), T)

    def chunked():
        for t0 in range(0, T, CH):
            ctx.moe_prefill_stack(shape, layers, hidden[t0:].data_ptr(), CH)

    res = {}
    outs = {}
    for name, fn in (("whole", whole), ("chunk64", chunked)):
        hidden.copy_(h0)
        fn()                      # warm-up (and scratch)
        torch.cuda.synchronize()
        ts = []
        for _ in range(max(1, min(args.steps, 5))):
            hidden.copy_(h0)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            ts.append(time.perf_counter() - t0)
        res[name] = min(ts)
        outs[name] = hidden.clone()
        log(f"prefill_stack {name}: {res[name] * 1e3:.2f} ms for {T} tokens x {NL} layers")
    ctx.synchronize()
    same = bool(torch.equal(outs["whole"], outs["chunk64"]))
    line = {
        "metric": "MoE prefill tok/s, whole prompt per layer", "value": round(T / res["whole"], 1),
        "unit": "tok/s", "n_gpus": 1, "steps": max(1, min(args.steps, 5)), "higher_is_better": True,
        "ms_per_prompt": round(res["whole"] * 1e3, 2), "us_per_layer": round(res["whole"] * 1e6 / NL, 1),
        "chunk64": {"tok_s": round(T / res["chunk64"], 1), "ms_per_prompt": round(res["chunk64"] * 1e3, 2)},
        "speedup_vs_chunk64": round(res["chunk64"] / res["whole"], 2), "chunked_equal_bitwise": same,
        "dtype": "f32 (f16 hi/lo MFMA operands)", "data": "synthetic",
        "config": {"workload": c["workload"] + "-prefill-512", "layers": NL, "tokens": T, "chunk": CH,
                   "d_model": D, "n_experts": E, "top_k": K, "d_ff": I},
    }
    print(json.dumps(line), flush=True)
    ctx.close()
    if not same:
        sys.exit(1)


def vault_bench(args):
    """Load rate of smoe_hip_vault_load: a vault of --layers synthetic layers
    (the --config expert shape, all E experts) is written to a temporary file
    from a pool generated on the GPU, then opened (every descriptor checked)
    and copied into a fresh device pool, timed; the loaded pool must equal the
    source bit for bit.  The file is read back from the page cache (dropping
    it needs root), so the rate is host memory -> pinned staging -> PCIe ->
    HBM, not disk."""
    import tempfile

    import torch

    import smoe_amd
    from smoe_amd import vault as V

    c = CONFIGS[args.config]
    D, E, K, I = c["D"], c["E"], c["K"], c["I"]
    NL = args.layers or 4
    dev = torch.device("cuda", 0)
    ctx = smoe_amd.Context()
    shape = smoe_amd.make_shape(D, E, K, I)
    off, raw, stride = smoe_amd.blob_layout(D, I)
    src = torch.empty(NL * E * stride, dtype=torch.uint8, device=dev)
    ctx.synth_expert_pool(src.data_ptr(), 0, NL, E, stride, shape, SEED, 0.02)
    host = src.cpu().numpy()
    tmpdir = os.environ.get("TMPDIR", "/tmp")
    with tempfile.NamedTemporaryFile(suffix=".smoe", dir=tmpdir) as tf:
        t0 = time.perf_counter()
        V.write_vault(tf.name, list(range(NL)), E, D, I,
                      lambda l, e: host[(l * E + e) * stride:(l * E + e) * stride + raw].tobytes())
        log(f"vault: wrote {NL} layers x {E} experts ({os.path.getsize(tf.name) / 1e9:.2f} GB) "
            f"in {time.perf_counter() - t0:.1f} s")
        del host
        dst = torch.empty_like(src)
        v = smoe_amd.Vault(tf.name)
        v.load(dst.data_ptr(), dst.numel())                # warm: page cache and pinned allocation
        times = []
        for _ in range(max(1, min(args.steps, 5))):
            dst.zero_()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            v2 = smoe_amd.Vault(tf.name)
            v2.load(dst.data_ptr(), dst.numel())
            times.append(time.perf_counter() - t0)
            v2.close()
        v.close()
        same = bool(torch.equal(dst, src))
    best = min(times)
    line = {
        "metric": "vault -> HBM expert pool load rate", "value": round(dst.numel() / best / 1e9, 2),
        "unit": "GB/s", "n_gpus": 1, "steps": len(times), "higher_is_better": True,
        "ms_per_load": round(best * 1e3, 2), "bytes": dst.numel(), "bit_exact": same,
        "source": "page cache (file written just before)", "data": "synthetic SMOE-Q4 layers",
        "config": {"workload": c["workload"] + "-vault-load", "layers": NL, "n_experts": E, "d_model": D,
                   "d_ff": I},
    }
    print(json.dumps(line), flush=True)
    ctx.close()
    if not same:
        sys.exit(1)


def grouped_line(workload, replicas, steps, warmup, calibrate_mib=0):
    """Tokens/s of the grouped path (smoe_hip_moe_prefill) on one layer shape,
    rotating over layer replicas (the expert bytes of one replica exceed the
    256 MB Infinity Cache only partly), each call on the same T seeded hidden
    rows; `steps` graph replays of one call per replica are timed.  Per-kernel
    times from dispatch events; the roofline is the grouped gate/up GEMM's
    (the dominant kernel), with its MFMA rate against the f16 dense peak."""
    import torch

    import smoe_amd

    g = GROUPED[workload]
    D, E, K, I, T, R = g["D"], g["E"], g["K"], g["I"], g["T"], replicas
    dev = torch.device("cuda", 0)
    calibrate_copy(argparse.Namespace(calibrate_copy_mib=calibrate_mib), dev)
    ctx = smoe_amd.Context()
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    ctx.set_stream(stream.cuda_stream)
    shape = smoe_amd.make_shape(D, E, K, I)
    off, raw, stride = smoe_amd.blob_layout(D, I)
    log(f"{workload}: {R} replicas of one layer ({R * E * stride / 1e9:.1f} GB), T={T}")
    pool = torch.empty(R * E * stride, dtype=torch.uint8, device=dev)
    ctx.synth_expert_pool(pool.data_ptr(), 0, R, E, stride, shape, SEED, 0.02)
    router = torch.empty((R, E * D), dtype=torch.int16, device=dev)
    norm_w = torch.full((D,), 0x3F80, dtype=torch.int16, device=dev)
    h0 = torch.empty((T, D), dtype=torch.float32, device=dev)
    for t in range(T):
        ctx.synth_normal(h0[t].data_ptr(), D, SEED, smoe_amd.hidden_stream(t), 1.0)
    u = None
    if g["zipf"]:
        from smoe_amd import synthetic
        u = synthetic.zipf_direction(D, SEED)
        synthetic.zipf_hidden(h0, u)     # a fixed component along u (|x . u| = 8 of ~64 norm)
    for l in range(R):
        ctx.synth_bf16(router[l].data_ptr(), E * D, SEED, smoe_amd.router_stream(l), 0.02)
        if u is not None:
            synthetic.zipf_bias_router(router[l], u, D, E, l, g["zipf"], SEED)
    layers = [smoe_amd.make_layer(norm_w.data_ptr(), router[l].data_ptr(), pool.data_ptr() + l * E * stride,
                                  stride, off) for l in range(R)]
    hidden = h0.clone()
    ids = torch.zeros((T, K), dtype=torch.int32, device=dev)
    ctx.moe_prefill(shape, layers[0], hidden.data_ptr(), T, ids.data_ptr())   # allocates scratch
    torch.cuda.synchronize()

    def step():
        for l in range(R):
            hidden.copy_(h0)
            ctx.moe_prefill(shape, layers[l], hidden.data_ptr(), T, ids.data_ptr())

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        step()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(steps):
        graph.replay()
    ev1.record(stream)
    torch.cuda.synchronize()
    elapsed = max(time.perf_counter() - t0, ev0.elapsed_time(ev1) / 1e3)
    calls = steps * R
    us_per_layer = elapsed * 1e6 / calls
    ctx.synchronize()
    counts = torch.bincount(ids.view(-1).long(), minlength=E).cpu()
    touched = int((counts > 0).sum())
    # per-kernel times (eager, dispatch events)
    ctx.profile_enable(True)
    for _ in range(2):
        step()
    torch.cuda.synchronize()
    kern = {}
    for kid, name in smoe_amd.KERNEL_NAMES.items():
        n, ms = ctx.profile_read(kid)
        if n:
            kern[name] = dict(launches=n, avg_us=round(ms * 1e3 / n, 3))
    ctx.profile_enable(False)
    mat = D * I // 2 + D * I // 64 * 2
    expert_bytes = 3 * mat * touched
    layer_bytes = expert_bytes + 2 * E * D + T * D * 8
    pairs = T * K
    flops = 6 * D * I * pairs + 2 * E * D * T
    gu, dn = kern.get("grouped_gate_up"), kern.get("grouped_down")
    gu_bytes, dn_bytes = 2 * mat * touched, mat * touched
    gu_us = gu["avg_us"] if gu else None
    mfma_flops = 2 * 4 * D * I * pairs                   # gate + up, hi and lo operand planes
    line = {
        "metric": f"MoE {workload} tok/s & achieved HBM GB/s",
        "value": round(T * calls / elapsed, 1), "unit": "tok/s", "n_gpus": 1, "steps": steps,
        "warmup": warmup, "us_per_layer_call": round(us_per_layer, 2),
        "higher_is_better": True, "dtype": "f32 (f16 hi/lo MFMA)",
        "data": "synthetic (counter-based N(0,0.02) weights quantized to SMOE-Q4; N(0,1) hidden"
                + (", router rows biased along a unit vector for Zipf s=1.1 popularity)" if u is not None else ")"),
        "config": {"workload": g["workload"], "d_model": D, "n_experts": E, "top_k": K, "d_ff": I, "tokens": T,
                   "replicas": R, "touched_experts": touched, "max_tokens_per_expert": int(counts.max())},
        "layer_bytes": layer_bytes, "layer_gbs": round(layer_bytes / (us_per_layer * 1e-6) / 1e9, 1),
        "layer_tflops": round(flops / (us_per_layer * 1e-6) / 1e12, 2),
        "roofline": {
            "bound": "hbm", "kernel": "k_grouped_mm<true>",
            "achieved": round(gu_bytes / (gu_us * 1e-6) / 1e9, 1) if gu else None,
            "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gu_bytes / (gu_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4) if gu else None,
            "traffic": grouped_traffic(g["workload"], "k_grouped_mm<true>"), "bytes_per_launch": gu_bytes,
            "avg_us": gu_us,
        },
        "mfma": {
            "kernel": "k_grouped_mm<true>", "tflops_algorithmic": round(4 * D * I * pairs / (gu_us * 1e-6) / 1e12, 1)
            if gu else None,
            "tflops_executed": round(mfma_flops / (gu_us * 1e-6) / 1e12, 1) if gu else None,
            "peak_tflops": MFMA_F16_PEAK_TFLOPS,
            "frac_executed": round(mfma_flops / (gu_us * 1e-6) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4) if gu else None,
            "layer_frac": round(flops / (us_per_layer * 1e-6) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
        },
        "down": {"kernel": "k_grouped_down", "bytes_per_launch": dn_bytes,
                 "gbs": round(dn_bytes / (dn["avg_us"] * 1e-6) / 1e9, 1) if dn else None,
                 "traffic": grouped_traffic(g["workload"], "k_grouped_down")},
        "kernels": kern,
    }
    ctx.close()
    return line


def grouped_traffic(workload, symbol):
    path = os.path.join(ROOT, "profiles", "pmc_traffic.json")
    try:
        with open(path) as f:
            return int(json.load(f)[workload][symbol]["traffic_bytes"])
    except (OSError, ValueError, KeyError):
        return None


# ---------------------------------------------------------------------------
# rocprofv3 summaries (the text committed under profiles/)
# ---------------------------------------------------------------------------
def rocprof_summary(d, config, pmc_out, copy_mib, workload="decode"):
    """Print a per-kernel summary of a rocprofv3 output directory: kernel
    stats (--kernel-trace --stats) and, for --pmc runs, the average counter
    value per dispatch of each kernel.  A kernel's full-size dispatches (at
    least half its largest) are also summarised apart: the parity leg runs the
    decode kernel on one layer at a time beside the whole-step launches.  With
    --pmc-out (and the size given by --calibrate-copy-mib), FETCH_SIZE/WRITE_SIZE
    of the decode kernels' full-size dispatches are scaled by expected/measured
    of the same counter for the calibration kernel (b = -a over that many MiB:
    reads and writes exactly that much) and merged into that JSON file."""
    for p in sorted(glob.glob(os.path.join(d, "**", "*kernel_stats.csv"), recursive=True)):
        print(f"== {os.path.basename(p)}")
        print(f"{'calls':>7} {'avg_us':>9} {'min_us':>9} {'max_us':>9} {'pct':>6}  kernel")
        for r in csv.DictReader(open(p)):
            print(f"{int(r['Calls']):7d} {float(r['AverageNs']) / 1e3:9.3f} {float(r['MinNs']) / 1e3:9.3f} "
                  f"{float(r['MaxNs']) / 1e3:9.3f} {float(r['Percentage']):6.2f}  {r['Name'][:90]}")
    for p in sorted(glob.glob(os.path.join(d, "**", "*kernel_trace.csv"), recursive=True)):
        durs = {}
        for r in csv.DictReader(open(p)):
            durs.setdefault(r["Kernel_Name"], []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
        print(f"== {os.path.basename(p)}: full-size dispatches (at least half the kernel's longest)")
        print(f"{'calls':>7} {'avg_us':>9} {'min_us':>9} {'max_us':>9} {'of':>6}  kernel")
        for k, v in sorted(durs.items(), key=lambda kv: -sum(kv[1])):
            big = [x for x in v if x >= 0.5 * max(v)]
            print(f"{len(big):7d} {sum(big) / len(big):9.3f} {min(big):9.3f} {max(big):9.3f} {len(v):6d}  {k[:90]}")
    per = {}
    for p in sorted(glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)):
        for r in csv.DictReader(open(p)):
            key = (r["Kernel_Name"], r["Counter_Name"])
            disp = r.get("Dispatch_Id") or r.get("Correlation_Id") or str(len(per.get(key, {})))
            per.setdefault(key, {})
            per[key][disp] = per[key].get(disp, 0.0) + float(r["Counter_Value"])
    if not per:
        return
    acc, full = {}, {}
    for key, dv in per.items():
        v = list(dv.values())
        acc[key] = (sum(v), len(v))
        big = [x for x in v if x >= 0.5 * max(v)]
        full[key] = (sum(big), len(big))
    print("== counters (average per dispatch; full-size dispatches: at least half the largest)")
    for (k, cn), (tot, n) in sorted(acc.items()):
        ft, fn = full[(k, cn)]
        print(f"{cn:>12} {tot / n:14.1f}  n={n:5d}  full-size {ft / fn:14.1f}  n={fn:5d}  {k[:80]}")
    if not (pmc_out and copy_mib):
        return
    data = json.load(open(pmc_out)) if os.path.exists(pmc_out) else {}
    if workload in GROUPED:
        ent = data.setdefault(GROUPED[workload]["workload"], {})
        symbols = ("k_grouped_mm<true>", "k_grouped_down", "k_grouped_mm<false>")
    else:
        ent = data.setdefault(CONFIGS[config]["workload"], {})
        symbols = tuple(KERNEL_SYMBOLS.values())
    for cn in ("FETCH_SIZE", "WRITE_SIZE"):
        copies = [tot / n for (k, c2), (tot, n) in acc.items() if c2 == cn and "neg_kernel" in k]
        if not copies:
            continue
        copy_kib = max(copies)
        scale = copy_mib * 1024.0 / copy_kib        # expected KiB / measured KiB for the copy
        data.setdefault("_calibration", {})[cn] = {"copy_mib": copy_mib, "copy_kib_measured": round(copy_kib, 1),
                                                    "scale": round(scale, 4)}
        for sym in symbols:
            vals = [tot / n for (k, c2), (tot, n) in full.items() if c2 == cn and sym in k]
            if vals:
                e = ent.setdefault(sym, {})
                e[cn + "_kib"] = round(vals[0], 1)
                e[cn + "_bytes_scaled"] = int(vals[0] * 1024 * scale)
                if "FETCH_SIZE_bytes_scaled" in e and "WRITE_SIZE_bytes_scaled" in e:
                    e["traffic_bytes"] = e["FETCH_SIZE_bytes_scaled"] + e["WRITE_SIZE_bytes_scaled"]
    with open(pmc_out, "w") as f:
        json.dump(data, f, indent=1, sort_keys=True)
    print(f"== merged into {pmc_out}")


if __name__ == "__main__":
    main()
