"""bench.py contract checks that need no GPU: one GPU only, and the traffic
table lookup."""
import json
import os
import subprocess
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_exits_with_message():
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_measured_traffic_uses_calibrated_counters():
    sys.path.insert(0, REPO)
    import bench
    t = json.load(open(os.path.join(REPO, "profiles", "traffic.json")))
    key = "C2:fp16:flash:bm256:bn128"
    k, c = t["kernels"][key], t["calibration"]
    want = int((k["fetch_kib"] * c["fetch_factor"] + k["write_kib"] * c["write_factor"]) * 1024)
    assert bench.measured_traffic(key) == want
    # close to the algorithmic 32 MiB of Q, K^T, V read and O written
    assert abs(want - 4 * 4 * 16 * 1024 * 64 * 2) / want < 0.05
    assert bench.measured_traffic("no:such:kernel") is None


def test_committed_best_programs_rebuild():
    sys.path.insert(0, os.path.join(REPO, "cs348k-fast-attention-grammar_amd"))
    from grammar.kernel_ast import emit_module, program_from_key, structural_key
    from grammar.hip_backend import parse_plan
    runs = os.path.join(REPO, "cs348k-fast-attention-grammar_amd", "runs")
    lowerings = {}
    for name in ("attn_c2_best.json", "attn_c3_best.json", "mlp_c4_best.json"):
        saved = json.load(open(os.path.join(runs, name)))
        p = program_from_key(saved["key"])
        assert structural_key(program_from_key(structural_key(p))) == structural_key(p)
        lowerings[name] = [s["lowering"] for s in parse_plan(emit_module(p))["steps"]]
    assert lowerings["attn_c2_best.json"] == ["flash"]
    assert lowerings["attn_c3_best.json"] == ["flash"]
    # X W1's 1,376 tiles leave a part-filled last round: its stage renders a
    # second (tail) launch
    assert lowerings["mlp_c4_best.json"] == ["gemm", "gemm", "gemm"]


def test_save_best_round_trip(tmp_path):
    # the --save-best writer of the search drivers reproduces a committed file's
    # key, stage tiles and (renderer-chosen) lowering
    sys.path.insert(0, os.path.join(REPO, "cs348k-fast-attention-grammar_amd"))
    from grammar.hip_module import save_best
    from grammar.kernel_ast import program_from_key
    saved = json.load(open(os.path.join(REPO, "cs348k-fast-attention-grammar_amd", "runs", "mlp_c4_best.json")))
    out = tmp_path / "best.json"
    rec = save_best(str(out), program_from_key(saved["key"]), "doc", 1.0, 7,
                    {"evals_per_min": 2.0, "timed_variants": 3})
    again = json.load(open(out))
    assert again == rec
    assert again["key"] == saved["key"] and again["stages"] == saved["stages"]
    assert [lw[:2] for lw in again["lowering"]] == [lw[:2] for lw in saved["lowering"]]
    assert (again["best_loss_ms"], again["iterations"], again["timed_variants"]) == (1.0, 7, 3)


def test_best_so_far_curve_keeps_improvements_only():
    sys.path.insert(0, REPO)
    import bench
    timeline = [{"t": 0.5, "loss": 0.3}, {"t": 1.0, "loss": 0.5}, {"t": 1.2, "loss": float("inf")},
                {"t": 1.5, "loss": 0.1}, {"t": 2.0, "loss": 0.1}]
    curve = bench.best_so_far(timeline, 1e12)
    assert [p[1] for p in curve] == [1, 4]          # variant index of each improvement
    assert [p[2] for p in curve] == [0.3, 0.1]      # best ms, strictly decreasing
    assert curve[-1][3] == round(1e12 / 0.1e-3 / 1e12, 1)


def test_committed_best_program_per_config():
    sys.path.insert(0, REPO)
    import bench
    for cfg in ("C2", "C3"):
        path = bench.best_program_path(cfg)
        assert os.path.basename(path) == f"attn_{cfg.lower()}_best.json" and os.path.exists(path)
