#!/usr/bin/env python3
"""Decode-attention benchmark on one MI355X.

Workload of the headline number (value): GPT-2 124M 12-layer decode-attention stack with
a BF16 KV cache, B=1, NH=12, hd=64, T=1024 attended positions (cur_len=1023).  A step is
one decode token: 12 attention calls, one per layer, each over that layer's own cache
(12 x 3 MiB).  The 12 calls are captured once in a HIP graph and replayed, as the
reference engine replays its whole-step graph; value = microseconds per attention call.

Also reported in the same JSON line:
  roofline      the dominant kernel (split with in-kernel merge, BF16) at T=1024
  cpu_baseline  single-threaded restatement of the reference CPU attention on the same
                shape (the oracle; a reported baseline, not the target)
  extra         eager per-call time, and the scaled-up ragged configuration: 64
                sequences x NH=12, BF16, lengths ~ U[1, 8192] (~0.8 GB of KV read per call)

Inputs are synthetic (seeded N(0,1)), resident in HBM before timing starts.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
HD = 64
METRIC = "µs per decode-attention call + achieved HBM GB/s (% of peak), T=1024"


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200, help="timed decode steps (12 calls each)")
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--strategy", default="auto")
    p.add_argument("--S", type=int, default=0, help="0 auto, >0 reference partition, <0 rows/segment")
    p.add_argument("--c5-reps", type=int, default=50)
    p.add_argument("--c5-strategy", default="auto")
    p.add_argument("--c5-S", type=int, default=0)
    p.add_argument("--no-c5", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--no-cpu", action="store_true")
    return p.parse_args()


def bytes_per_call(lengths, NH, kv_bytes, act_bytes, B):
    """Algorithmic HBM bytes: K+V rows actually attended, plus q in and out."""
    return int(sum(2 * NH * L * HD * kv_bytes for L in lengths) + B * NH * HD * 2 * act_bytes)


def bench_c2(args, torch, kvattn, dev):
    L, B, NH, maxT, T = 12, 1, 12, 1024, 1024
    g = torch.Generator(device=dev)
    g.manual_seed(2)
    caches = [torch.randn(2 * B * NH * maxT * HD, generator=g, device=dev, dtype=torch.float32)
              .to(torch.bfloat16) for _ in range(L)]
    qkvs = [torch.randn(B * 3 * NH * HD, generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
            for _ in range(L)]
    outs = [torch.empty(B * NH * HD, device=dev, dtype=torch.bfloat16) for _ in range(L)]
    cur = torch.tensor([T - 1], dtype=torch.int32, device=dev)
    ws = kvattn.Workspace(B, NH, maxT, args.S)

    def step():
        for l in range(L):
            kvattn.decode(outs[l], qkvs[l], caches[l], B, NH, HD, maxT, kv_dtype="bf16", cur_len=cur,
                          len_hint=T - 1, S=args.S, strategy=args.strategy, **ws.kwargs())

    # eager
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    eager_ms_step = e0.elapsed_time(e1) / args.steps

    # graph: the 12 calls captured once, replayed per step
    s = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            step()
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    e0.record()
    for _ in range(args.steps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    graph_ms_step = e0.elapsed_time(e1) / args.steps

    # parity spot check of the last layer against a float64 torch reference on the CPU
    cs = caches[-1].float().view(2, B, NH, maxT, HD)[:, 0, :, :T].cpu().double()
    q = qkvs[-1].float().view(B, 3, NH, HD)[0, 0].cpu().double()
    sc = torch.einsum("hd,htd->ht", q, cs[0]) / (HD ** 0.5)
    ref = torch.einsum("ht,htd->hd", torch.softmax(sc, dim=1), cs[1])
    got = outs[-1].float().view(NH, HD).cpu().double()
    rel = float(((got - ref).norm(dim=1) / ref.norm(dim=1)).max())
    return {
        "layers": L, "B": B, "NH": NH, "T": T, "maxT": maxT,
        "graph_ms_step": graph_ms_step, "eager_ms_step": eager_ms_step,
        "bytes_per_call": bytes_per_call([T], NH, 2, 2, B),
        "rel_err_vs_f64": rel,
        "caches": caches, "qkvs": qkvs,
    }


def bench_c5(args, torch, kvattn, dev):
    B, NH, maxT = 64, 12, 8192
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    lens = torch.randint(1, maxT + 1, (B,), generator=g, device=dev, dtype=torch.int32)
    cur = (lens - 1).contiguous()
    cache = torch.empty(2 * B * NH * maxT * HD, device=dev, dtype=torch.bfloat16)
    chunk = 1 << 26
    for i in range(0, cache.numel(), chunk):
        n = min(chunk, cache.numel() - i)
        cache[i:i + n] = torch.randn(n, generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
    qkv = torch.randn(B * 3 * NH * HD, generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
    out = torch.empty(B * NH * HD, device=dev, dtype=torch.bfloat16)
    ws = kvattn.Workspace(B, NH, maxT, args.c5_S)

    def call():
        kvattn.decode(out, qkv, cache, B, NH, HD, maxT, kv_dtype="bf16", cur_len=cur, lens_per_seq=True,
                      S=args.c5_S, strategy=args.c5_strategy, **ws.kwargs())

    for _ in range(5):
        call()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.c5_reps):
        call()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1000.0 / args.c5_reps
    lh = [int(x) for x in lens.cpu().tolist()]
    nbytes = bytes_per_call(lh, NH, 2, 2, B)
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"workload": "64 seqs x NH=12 x hd=64, BF16 KV, lengths U[1,8192] (seed 5)",
            "sum_len": sum(lh), "bytes_per_call": nbytes, "us_per_call": us, "GBps": gbs,
            "frac_of_hbm_peak": gbs / HBM_PEAK_GBS, "strategy": args.c5_strategy, "S": args.c5_S}


def cpu_baseline(seconds, torch, c2):
    from oracle import oracle
    import numpy as np
    B, NH, maxT, T = 1, 12, 1024, 1024
    cache = c2["caches"][0].float().cpu().numpy()
    qkv = c2["qkvs"][0].float().cpu().numpy()
    t1 = oracle.time_attention_f32(qkv, cache, T, B, NH, HD, maxT, 1)
    reps = max(3, int(seconds * 1e6 / max(t1, 1.0)))
    med = oracle.time_attention_f32(qkv, cache, T, B, NH, HD, maxT, reps)
    cpu = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"value": med, "unit": "us/call", "cores": 1, "kind": "port",
            "sample": f"attention_kv_cpu restated (oracle, FP32, single thread), B=1 NH=12 hd=64 T=1024 "
                      f"(bf16 cache decoded to FP32), median of {reps} calls",
            "host_cpu": cpu, "host_nproc": os.cpu_count(), "reps": reps}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU: the decode-attention path has no "
                                   "cross-GPU exchange here; run with --gpus 1"}))
        sys.exit(2)
    import torch
    from cuda_gpt2_inference_amd import kvattn
    if not os.path.exists(kvattn.LIB_PATH):
        import __graft_entry__
        __graft_entry__.build()
    kvattn.lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    c2 = bench_c2(args, torch, kvattn, dev)
    us_call = c2["graph_ms_step"] * 1000.0 / c2["layers"]
    eager_us_call = c2["eager_ms_step"] * 1000.0 / c2["layers"]
    achieved = c2["bytes_per_call"] / (us_call * 1e-6) / 1e9
    c5 = None if args.no_c5 else bench_c5(args, torch, kvattn, dev)
    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds, torch, c2)

    line = {
        "metric": METRIC,
        "value": round(us_call, 4),
        "unit": "us/call",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(c2["graph_ms_step"], 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "GPT-2 124M 12-layer decode-attention stack, BF16 KV cache, B=1, NH=12, hd=64, "
                               "T=1024 (cur_len=1023); one step = 12 calls replayed as a HIP graph",
                   "batch": 1, "heads": 12, "head_dim": 64, "context": 1024, "layers": 12,
                   "kv_dtype": "bf16", "accumulate": "f32", "strategy": args.strategy, "S": args.S},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 5), "traffic": None,
                     "kernel": "split_kernel<BF16, last-block merge>",
                     "bytes_per_launch": c2["bytes_per_call"], "us_per_launch": round(us_call, 4)},
        "cpu_baseline": cpu,
        "extra": {"eager_us_per_call": round(eager_us_call, 4),
                  "rel_err_vs_f64": c2["rel_err_vs_f64"],
                  "gpu_vs_cpu_speedup": (round(cpu["value"] / us_call, 1) if cpu else None),
                  "c5": c5, "gpu": torch.cuda.get_device_name(dev), "host": platform.node()},
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
