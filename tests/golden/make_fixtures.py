"""Write tests/golden/reference_runs.json from the reference's own search logs.

Reads only data files of the reference (runs/*/log.jsonl, JSON lines written by
its RunLogger, grammar/optimization.py:842-867) -- no reference code is
imported or run. A record's `best_key` is the structural key of the best
program; in the records where the iteration's program became the new best
(loss == best_loss, best changed) and at iteration 0, that program is exactly
the one whose `flops`, `flops_exact` and `peak_tile_bytes` the record holds.

    python tests/golden/make_fixtures.py [/root/reference]
"""
import glob
import json
import os
import sys

ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
out = []
for path in sorted(glob.glob(os.path.join(ref, "runs", "**", "log.jsonl"), recursive=True)):
    run = os.path.relpath(os.path.dirname(path), os.path.join(ref, "runs"))
    prev = None
    for line in open(path):
        r = json.loads(line)
        became_best = r["loss"] == r["best_loss"] and (prev is None or r["best_loss"] != prev)
        if r["iter"] == 0 or became_best:
            out.append({"run": run, "iter": r["iter"], "loss_kind": r["loss_kind"], "key": r["best_key"],
                        "flops": r["flops"], "flops_exact": r["flops_exact"],
                        "peak_tile_bytes": r["peak_tile_bytes"], "stages": r["stages"]})
        prev = r["best_loss"]
dest = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_runs.json")
with open(dest, "w") as f:
    json.dump({"source": "runs/*/log.jsonl of the reference (RunLogger records)", "records": out}, f)
print(f"{len(out)} records -> {dest}")
