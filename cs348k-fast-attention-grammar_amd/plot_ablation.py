"""Summarise and plot the Design-for-Descent ablations from run directories
(the log.jsonl that RunLogger writes), as the reference's plot_ablation.py
does (plot_ablation.py:55-68 best-feasible curve, :115-174 the figures):

  ablation.png          best feasible runtime against iteration, one line per
                        run (a run that never reached a feasible program is
                        listed as such)
  flops_vs_runtime.png  for one run: the program's FLOPs (flat: the same
                        computation) against its runtime (dropping)
  summary.md            the same curves as a table: best feasible ms at each
                        iteration where some run improved, the iteration of
                        first feasibility, evals/min and the re-timed best
                        kernels (results/it*.json) when present

    python plot_ablation.py full=runs/ablations/x/full no_reversibility=... \
        [--headline runs/ablations/x/full] [--out-dir runs/ablations/x]

Every positional argument is LABEL=RUN_DIR. matplotlib is optional: without
it only summary.md is written.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import re

PENALTY = 1e9          # losses at or above this are penalties (grammar.optimization.MEM_PENALTY_BASE)


def read_log(run_dir: str) -> list:
    with open(os.path.join(run_dir, "log.jsonl")) as f:
        return [json.loads(line) for line in f if line.strip()]


def _num(x) -> float:
    return math.inf if x == "inf" else float(x)


def feasible_best(records: list) -> list:
    """[(iteration, best feasible ms so far or None)], in log order."""
    best, out = math.inf, []
    for r in records:
        b = _num(r["best_loss"])
        if b < PENALTY:
            best = min(best, b)
        out.append((r["iter"], best if best < PENALTY else None))
    return out


def retimed(run_dir: str) -> list:
    """[(iteration, ms, TFLOP/s)] from results/it*.json, by iteration."""
    rdir = os.path.join(run_dir, "results")
    if not os.path.isdir(rdir):
        return []
    rows = []
    for name in os.listdir(rdir):
        m = re.fullmatch(r"it(\d+)\.json", name)
        if m:
            with open(os.path.join(rdir, name)) as f:
                st = json.load(f)["stats"]
            rows.append((int(m.group(1)), st["ms"], st["tflops"]))
    return sorted(rows)


def summary_markdown(runs: dict) -> str:
    curves = {label: feasible_best(read_log(d)) for label, d in runs.items()}
    lines = ["| run | first feasible iteration | best feasible ms | at iteration | stages at the end | "
             "evals/min | best kernel re-timed (ms, TFLOP/s) |", "|---|---|---|---|---|---|---|"]
    for label, d in runs.items():
        recs = read_log(d)
        curve = curves[label]
        first = next((it for it, v in curve if v is not None), None)
        final = curve[-1][1] if curve else None
        at = next((it for it, v in curve if v is not None and v == final), None)
        ev = recs[-1].get("eval", {}) if recs else {}
        rt = retimed(d)
        best_rt = min(rt, key=lambda r: r[1]) if rt else None
        lines.append(f"| {label} | {first if first is not None else 'never'} | "
                     f"{'%.4f' % final if final is not None else '—'} | {at if at is not None else '—'} | "
                     f"{recs[-1]['n_stages'] if recs else '—'} | "
                     f"{'%.0f' % ev['evals_per_min'] if 'evals_per_min' in ev else '—'} | "
                     f"{'it%d: %.4f ms, %.3f' % best_rt if best_rt else '—'} |")
    # the curves where anything moved
    iters = sorted({it for c in curves.values() for it, _ in c})
    labels = list(runs)
    table = ["", "Best feasible ms after each iteration where some run improved:", "",
             "| iteration | " + " | ".join(labels) + " |", "|---|" + "---|" * len(labels)]
    last = {l: None for l in labels}
    for it in iters:
        now = {l: dict(curves[l]).get(it, last[l]) for l in labels}
        if any(now[l] != last[l] for l in labels):
            table.append(f"| {it} | " + " | ".join("%.4f" % now[l] if now[l] is not None else "—" for l in labels) + " |")
        last = now
    return "\n".join(lines + table) + "\n"


def plot(runs: dict, headline: str | None, out_dir: str) -> list:
    try:
        import matplotlib
        matplotlib.use("Agg")
        import matplotlib.pyplot as plt
    except ImportError:
        return []
    written = []
    fig, ax = plt.subplots(figsize=(7, 4.5))
    for label, d in runs.items():
        curve = feasible_best(read_log(d))
        pts = [(it, v) for it, v in curve if v is not None]
        if pts:
            ax.step([p[0] for p in pts], [p[1] for p in pts], where="post", marker="o", ms=3, label=label)
        else:
            ax.plot([], [], label=f"{label} (never feasible)")
    ax.set_xlabel("iteration")
    ax.set_ylabel("best feasible runtime (ms)")
    ax.set_yscale("log")
    ax.set_title("Descent on the MI355X: best runtime by grammar property")
    ax.grid(True, which="both", alpha=0.3)
    ax.legend(fontsize=8)
    fig.tight_layout()
    path = os.path.join(out_dir, "ablation.png")
    fig.savefig(path, dpi=120)
    plt.close(fig)
    written.append(path)
    if headline:
        recs = read_log(headline)
        its = [r["iter"] for r in recs]
        ms = [_num(r["loss"]) if _num(r["loss"]) < PENALTY else float("nan") for r in recs]
        fl = [r["flops"] / 1e6 if r.get("flops") else float("nan") for r in recs]
        fig, ax1 = plt.subplots(figsize=(7, 4.5))
        ax1.step(its, ms, where="post", color="tab:blue", label="runtime (ms)")
        ax1.set_yscale("log")
        ax1.set_xlabel("iteration")
        ax1.set_ylabel("runtime (ms)", color="tab:blue")
        ax2 = ax1.twinx()
        ax2.plot(its, fl, color="tab:red", ls="--", label="FLOPs (M)")
        ax2.set_ylabel("FLOPs (millions)", color="tab:red")
        ax1.set_title("Same computation, less time: FLOPs flat, runtime falling")
        ax1.grid(True, alpha=0.3)
        fig.tight_layout()
        path = os.path.join(out_dir, "flops_vs_runtime.png")
        fig.savefig(path, dpi=120)
        plt.close(fig)
        written.append(path)
    return written


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("runs", nargs="+", help="LABEL=RUN_DIR")
    ap.add_argument("--headline", default=None)
    ap.add_argument("--out-dir", default=".", dest="out_dir")
    args = ap.parse_args(argv)
    runs = dict(r.split("=", 1) for r in args.runs)
    os.makedirs(args.out_dir, exist_ok=True)
    md = summary_markdown(runs)
    with open(os.path.join(args.out_dir, "summary.md"), "w") as f:
        f.write(md)
    print(md)
    for p in plot(runs, args.headline, args.out_dir):
        print(f"wrote {p}")
    return 0


if __name__ == "__main__":
    import sys
    sys.exit(main())
