"""The Design-for-Descent ablations on the MI355X: one descent per grammar
principle left out (full, no_reversibility, no_repairability,
no_jump_continuity, no_local_control; run_attention_search.py
`principle_config`), each into its own run directory, then every durable best
kernel of each run re-timed on its own (the reference keeps
runs/attn_*/{config.json, log.jsonl, kernels/best_it*.py} and re-benches each
best_it* into runs/attn_*/results/it*.json; run_attention_search.py:117-166,
bench.py:89-140).

The default workload is the reference's own: one head, N = 512, d = 64, fp32,
64 iterations, Stage 2 every 4 iterations with K = 5, seed 0 -- the runs
behind results/attn-*.json. --b/--h/--n/--d/--dtype select another one.

    python run_ablations.py --out runs/ablations/ref_n512_fp32 [--budget 120] [--rules reference]

Each run directory gets config.json, log.jsonl, kernels/best_it*.{hip,json}
(RunLogger), results/it*.json (the re-timed best kernels) and summary.json.

    python run_ablations.py --export SRC DEST   # the compact copy kept under runs/ablations/
    python run_ablations.py --retime DIR        # re-time the best kernels of an ablation directory

Every re-timing runs the kernel for 50 ms first (the clocks ramp up under
load), then takes the median of three batches of back-to-back runs.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import re
import sys
import time

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

PRINCIPLES = ("full", "no_reversibility", "no_repairability", "no_jump_continuity", "no_local_control")


def retime_bests(run_dir: str, steps: int, warmup: int) -> list:
    """Re-time every kernels/best_it*.hip of a run on its own and write
    results/it<N>.json; returns [(iteration, ms, TFLOP/s)]."""
    import torch
    from grammar.hip_module import HipModule
    from grammar.workloads import torch_dtype
    kdir = os.path.join(run_dir, "kernels")
    rdir = os.path.join(run_dir, "results")
    os.makedirs(rdir, exist_ok=True)
    out = []
    names = sorted((f for f in os.listdir(kdir) if re.fullmatch(r"best_it\d+\.hip", f)),
                   key=lambda f: int(re.findall(r"\d+", f)[0]))
    for name in names:
        it = int(re.findall(r"\d+", name)[0])
        with open(os.path.join(kdir, name)) as f:
            mod = HipModule(f.read())
        g = torch.Generator("cpu").manual_seed(0)
        dt = torch_dtype(mod.plan["dtype"])
        tensors = {n: torch.randn(tuple(s), generator=g).to(dt).cuda() for n, s in mod.KERNEL_META["inputs"]}
        tensors.update(mod.allocate("cuda"))
        plan = mod.bind(tensors)
        for _ in range(warmup):
            plan.run()
        torch.cuda.synchronize()
        from grammar import runtime as rt
        # the clocks ramp up over tens of milliseconds of load: 50 ms of the
        # kernel first, then the median of three batches
        t0 = time.time()
        while time.time() - t0 < 0.05:
            plan.time(0, 50, rt.GR_TIME_BATCH)
        ms = sorted(plan.time(0, steps, rt.GR_TIME_BATCH) for _ in range(3))[1]
        flops = mod.KERNEL_META["flops"]
        rec = {"label": f"best_it{it}", "device": torch.cuda.get_device_name(0), "source": f"kernels/{name}",
               "config": {"dtype": mod.plan["dtype"], "inputs": mod.KERNEL_META["inputs"],
                          "output": mod.KERNEL_META["output"]},
               "stats": {"ms": ms, "tflops": flops / (ms * 1e-3) / 1e12, "flops": flops, "steps": steps,
                         "warmup": warmup, "stages": len(mod.plan["steps"]),
                         "lowering": [s["lowering"] for s in mod.plan["steps"]]}}
        with open(os.path.join(rdir, f"it{it}.json"), "w") as f:
            json.dump(rec, f, indent=1)
        out.append((it, ms, rec["stats"]["tflops"]))
        del plan, tensors, mod
    return out


def export_compact(src: str, dest: str) -> None:
    """Copy the parts of an ablation directory worth keeping in the
    repository: summary.json, and per run config.json, summary.json,
    kernels/, results/ and a log.jsonl whose records keep `best_key` only
    where it changes (the resume snapshot stays behind)."""
    import shutil
    os.makedirs(dest, exist_ok=True)
    shutil.copy(os.path.join(src, "summary.json"), os.path.join(dest, "summary.json"))
    for principle in sorted(os.listdir(src)):
        run = os.path.join(src, principle)
        if not os.path.isdir(run):
            continue
        out = os.path.join(dest, principle)
        os.makedirs(out, exist_ok=True)
        for name in ("config.json", "summary.json"):
            if os.path.exists(os.path.join(run, name)):
                shutil.copy(os.path.join(run, name), os.path.join(out, name))
        for sub in ("kernels", "results"):
            if os.path.isdir(os.path.join(run, sub)):
                shutil.copytree(os.path.join(run, sub), os.path.join(out, sub), dirs_exist_ok=True)
        last_key = None
        with open(os.path.join(run, "log.jsonl")) as f, open(os.path.join(out, "log.jsonl"), "w") as g:
            for line in f:
                rec = json.loads(line)
                if rec.get("best_key") == last_key:
                    rec.pop("best_key", None)
                else:
                    last_key = rec.get("best_key")
                g.write(json.dumps(rec) + "\n")


def retime_dir(out: str, steps: int) -> None:
    """Re-time the durable best kernels of every run under an ablation
    directory (results/it*.json and each run's summary.json rewritten)."""
    top = os.path.join(out, "summary.json")
    with open(top) as f:
        whole = json.load(f)
    for principle, rec in whole["principles"].items():
        run_dir = os.path.join(out, principle)
        rec["retimed_best"] = [{"iter": i, "ms": ms, "tflops": tf} for i, ms, tf in retime_bests(run_dir, steps, 20)]
        with open(os.path.join(run_dir, "summary.json"), "w") as f:
            json.dump(rec, f, indent=1)
        print(f"{principle}: " + ", ".join(f"it{r['iter']} {r['ms'] * 1e3:.1f} us" for r in rec["retimed_best"]),
              flush=True)
    with open(top, "w") as f:
        json.dump(whole, f, indent=1)


def main(argv=None) -> int:
    if argv is None and len(sys.argv) == 4 and sys.argv[1] == "--export":
        export_compact(sys.argv[2], sys.argv[3])
        return 0
    if argv is None and len(sys.argv) == 3 and sys.argv[1] == "--retime":
        retime_dir(sys.argv[2], 200)
        return 0
    ap = argparse.ArgumentParser()
    ap.add_argument("--out", default="runs/ablations/ref_n512_fp32")
    ap.add_argument("--principles", default=",".join(PRINCIPLES))
    ap.add_argument("--n", type=int, default=512)
    ap.add_argument("--d", type=int, default=64)
    ap.add_argument("--b", type=int, default=None)
    ap.add_argument("--h", type=int, default=None)
    ap.add_argument("--dtype", default="fp32", choices=["fp32", "fp16", "bf16"])
    ap.add_argument("--iters", type=int, default=64)
    ap.add_argument("--budget", type=float, default=0.0, help="wall seconds per descent (0 = all iterations)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--retime-steps", type=int, default=200, dest="retime_steps")
    ap.add_argument("--rules", default="full", choices=["full", "reference"],
                    help="this grammar's rule set or the reference's seven rules")
    args = ap.parse_args(argv)

    import run_attention_search as RS
    summary = {}
    for principle in args.principles.split(","):
        run_dir = os.path.join(args.out, principle)
        cli = ["--n", str(args.n), "--d", str(args.d), "--dtype", args.dtype, "--iters", str(args.iters),
               "--every", "4", "--k", "5", "--seed", str(args.seed), "--principle", principle,
               "--run-dir", run_dir, "--time-budget", str(args.budget), "--rules", args.rules]
        if args.b is not None:
            cli += ["--b", str(args.b)]
        if args.h is not None:
            cli += ["--h", str(args.h)]
        print(f"===== ablation {principle}: run_attention_search.py {' '.join(cli)}", flush=True)
        best, ev = RS.main(cli)
        st = ev.stats()
        ev.close()
        retimed = retime_bests(run_dir, args.retime_steps, 20)
        best_loss = ev(best)
        summary[principle] = {"best_loss_ms": None if best_loss >= 1e9 else best_loss,
                              "best_kind": "feasible" if best_loss < 1e9 else ("penalty" if best_loss < math.inf
                                                                               else "infeasible"),
                              "stages": [[l.out, list(l.tile_shape)] for l in best.body],
                              "iterations": getattr(ev, "iterations", None), "wall_s": st["wall_s"],
                              "timed_variants": st["timed_variants"], "hiprtc_compiles": st["hiprtc_compiles"],
                              "evals_per_min": st["evals_per_min"],
                              "retimed_best": [{"iter": i, "ms": ms, "tflops": tf} for i, ms, tf in retimed]}
        with open(os.path.join(run_dir, "summary.json"), "w") as f:
            json.dump(summary[principle], f, indent=1)
        print(f"===== {principle}: {summary[principle]['best_kind']} best {summary[principle]['best_loss_ms']} ms, "
              f"{len(retimed)} best kernels re-timed", flush=True)
    with open(os.path.join(args.out, "summary.json"), "w") as f:
        json.dump({"workload": {k: getattr(args, k) for k in ("b", "h", "n", "d", "dtype", "iters", "seed", "rules")},
                   "principles": summary}, f, indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
