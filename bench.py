#!/usr/bin/env python3
"""Benchmark: attention forward TFLOP/s and % of the fp16 MFMA peak on one
MI355X at B=4, H=16, N=1024, d=64.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config C2|C3]

A "step" is one attention forward over the whole batch, inputs resident in
HBM. W untimed warmup steps, then exactly K steps between two hipEvents
recorded on the stream the kernel runs on, after a device synchronize on both
sides. Prints ONE JSON line on stdout (diagnostics go to stderr), with the
roofline of the kernel and the CPU baseline (the staged naive attention in
fp32 torch on this host's cores, on the same seeded inputs) beside it.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(REPO, "cs348k-fast-attention-grammar_amd")
sys.path.insert(0, PKG)
sys.path.insert(0, REPO)

METRIC = "attn fwd TFLOP/s, % fp16 MFMA peak (B4 H16 N1024 d64); descent evals/min"
PEAK_TFLOPS = {"fp16": 2500.0, "bf16": 2500.0}     # MI355X dense MFMA, published
HBM_PEAK_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_baseline(cfg, seed: int, budget_s: float = 12.0) -> dict:
    """Staged naive attention (oracle/naive_torch.py) in fp32 on this host's
    CPU cores, on the same seeded inputs rounded to the config dtype. One
    warmup, then reps until ~budget_s of CPU work (>= 5 reps); median."""
    import torch
    from grammar.workloads import attention_inputs
    from oracle.naive_torch import staged_attention
    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    q, k, v = attention_inputs(cfg, seed=seed)
    q, k, v = q.float(), k.float(), v.float()
    kt = k.transpose(-1, -2).contiguous()
    staged_attention(q, kt, v, causal=cfg.causal)           # warmup
    times = []
    t_start = time.perf_counter()
    while len(times) < 5 or (time.perf_counter() - t_start < budget_s and len(times) < 50):
        t0 = time.perf_counter()
        staged_attention(q, kt, v, causal=cfg.causal)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {
        "value": cfg.flops / med / 1e12,
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"full {cfg.name} batch (B{cfg.B} H{cfg.H} N{cfg.N} d{cfg.D}), staged 8-pass naive "
                   f"attention, torch fp32 on CPU, median of {len(times)} reps after 1 warmup "
                   f"({med * 1e3:.1f} ms/rep; os.cpu_count()={cores})"),
        "ms": med * 1e3,
    }


def measured_traffic(cfg, bm: int, bn: int):
    """HBM bytes per launch for this kernel configuration from the committed
    rocprofv3 FETCH_SIZE/WRITE_SIZE measurement (profiles/traffic.json),
    scaled by the copy-calibration factors; None if not measured."""
    path = os.path.join(REPO, "profiles", "traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
        k = t["kernels"][f"{cfg.name}:{cfg.dtype}:bm{bm}:bn{bn}"]
        c = t["calibration"]
        return int((k["fetch_kib"] * c["fetch_factor"] + k["write_kib"] * c["write_factor"]) * 1024)
    except (OSError, KeyError, ValueError):
        return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="C2", choices=["C2", "C3"])
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--block-m", type=int, default=128, help="queries per workgroup")
    ap.add_argument("--block-n", type=int, default=128, help="keys per tile")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="instead of the benchmark, run --steps plain device copies of MIB MiB "
                         "(the known-size reference that scales rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the attention kernel on one GPU's share); "
              "--gpus must be 1", file=sys.stderr)
        return 2

    import torch
    from grammar.attention import flash_attention_fwd
    from grammar.workloads import CONFIGS, attention_inputs

    dev = torch.device("cuda:0")
    if args.copy_calibration:
        n = args.copy_calibration * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(max(1, args.steps)):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] copy calibration: {args.steps} copies of {args.copy_calibration} MiB")
        return 0

    cfg = CONFIGS[args.config]
    if cfg.D == 128 and args.block_n > 64:
        args.block_n = 64
    q, k, v = (t.to(dev) for t in attention_inputs(cfg, seed=args.seed))
    out = torch.empty_like(q)
    kernel = {"name": "gr_flash_fwd (hand-written)", "block_m": args.block_m, "block_n": args.block_n}

    def step():
        flash_attention_fwd(q, k, v, causal=cfg.causal, out=out,
                            block_m=kernel["block_m"], block_n=kernel["block_n"])

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    tflops = cfg.flops / (ms * 1e-3) / 1e12
    peak = PEAK_TFLOPS[cfg.dtype]
    log(f"[bench] {cfg.name}: {ms * 1e3:.2f} us/step  {tflops:.1f} TFLOP/s  {100 * tflops / peak:.1f}% of peak")

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(cfg, args.seed)
        log(f"[bench] cpu baseline: {cpu['ms']:.1f} ms/rep  {cpu['value'] * 1e3:.2f} GFLOP/s on {cpu['cores']} threads")
        cpu.pop("ms")

    rec = {
        "metric": METRIC,
        "value": round(tflops, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg.dtype,
        "data": "synthetic (seeded N(0,1) inputs)",
        "config": {"workload": f"attention forward {cfg.name}: B{cfg.B} H{cfg.H} N{cfg.N} d{cfg.D} "
                               f"{cfg.dtype}{' causal' if cfg.causal else ''}",
                   "B": cfg.B, "H": cfg.H, "N": cfg.N, "D": cfg.D, "causal": cfg.causal,
                   "kernel": kernel, "parallelism": "single GPU"},
        "pct_peak": round(100 * tflops / peak, 2),
        "evals_per_min": None,
        "roofline": {"bound": "mfma", "achieved": round(tflops, 3), "peak": peak, "unit": "TFLOP/s",
                     "frac": round(tflops / peak, 5),
                     "traffic": measured_traffic(cfg, args.block_m, args.block_n)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
