"""CPU tests of the descent (proxy loss, no GPU): parameter vector naming and
coupling, rewrite menus, Stage 1/2, the outer loop, run logs and JSON
snapshot/resume. The reference has no tests for its optimizer; these pin the
behaviour its code states (grammar/optimization.py:342-1035)."""
import json
import math
import os
import random

import pytest

import grammar_cases as C
from grammar import optimization as O
from grammar.kernel_ast import structural_key, Compute, ReductionLoop


def _ev():
    return O.Evaluator(O.EvalConfig(proxy=True, mem_budget=64 * 1024, max_compile_risk=256))


def test_parameter_vector_names_and_coupling():
    p = C.p_attention_atomic()
    names = [q.name for q in O.parameter_vector(p)]
    assert names[:2] == ["TILE_S[0]", "TILE_S[1]"]
    assert "TILE_mx[1]" not in names        # mx is [N,1]: its collapsed dim is not a knob
    q = O.parameter_vector(p, couple=True)
    assert len(q) == 1 and q[0].name == "TILE_GLOBAL"
    q[0].set(16)
    assert all(t == 16 for l in p.body for d, t in enumerate(l.tile_shape) if p.tensors[l.out][d] > 1)


def test_ladder_includes_extent_and_clamps():
    tp = O.TileParam("x", 48, 16)
    assert tp.ladder() == [16, 32, 48]


def test_loss_kinds_and_ordering():
    assert O.loss_kind(math.inf) == "infeasible"
    assert O.loss_kind(O.MEM_PENALTY_BASE + 3) == "penalty"
    assert O.loss_kind(0.1) == "feasible"
    assert O._better(0.1, O.MEM_PENALTY_BASE) and O._better(O.MEM_PENALTY_BASE, math.inf)


def test_gates_penalise_without_compiling():
    from grammar.kernel_ast import Program, ParallelLoop, Load, Store
    ev = O.Evaluator(O.EvalConfig(proxy=False, mem_budget=32 * 1024))
    p = C.p_attention_atomic()                 # (64,128) tiles: S row 64*128*4 = 32 KiB
    assert ev._gated(p) is None
    for l in p.body:
        l.tile_shape = tuple(max(t, 128) for t in l.tile_shape)
    loss = ev._gated(p)                        # 128x128 fp32 tiles: 64 KiB > 32 KiB
    assert loss is not None and loss >= O.MEM_PENALTY_BASE


def test_enumerate_rewrites_atomic_menu():
    p = C.p_attention_atomic()
    labels = [r.label for r in O.enumerate_rewrites(p, O.DEFAULT_RULES)]
    assert "subtile(matmul,dd)" in labels and "subtile(matmul,j)" in labels
    assert "merge(S,mx)" not in labels               # S is read by mx and sb
    assert "merge(mx,sb)" in labels
    ref_only = [r.label for r in O.enumerate_rewrites(p, O.REFERENCE_RULES)]
    assert not any(l.startswith(("fuse_softmax", "sink_compute")) for l in ref_only)


def test_rewrite_descriptor_reresolves_on_clone():
    from grammar import rewrites as R
    p = C.p_matmul_full_k()
    rw = next(r for r in O.enumerate_rewrites(p, ("subtile_reduction",)))
    q = R.clone_program(p)
    out = rw.resolve(q)
    assert out is not None and any(isinstance(s, ReductionLoop) for s in out.body[0].body)


def test_stage1_improves_proxy_and_does_not_mutate():
    p = C.p_matmul_reduction()
    key = structural_key(p)
    q, loss = O.stage1_sweep(p, _ev(), neighbor=False)
    assert structural_key(p) == key
    assert loss <= _ev()(p)


def test_autotune_runs_logs_and_resumes(tmp_path):
    run = str(tmp_path / "run")
    p = C.p_attention_atomic()
    cfg = O.SearchConfig(iters=6, N=2, K=3, seed=0, verbose=False, run_dir=run)
    best = O.autotune(p, _ev(), cfg)
    recs = [json.loads(l) for l in open(os.path.join(run, "log.jsonl"))]
    assert [r["iter"] for r in recs] == list(range(0, 7))
    assert all("time" in r and "eval" in r for r in recs)
    assert recs[-1]["best_loss"] <= recs[0]["best_loss"]
    snap = O.load_snapshot(run)
    assert snap["iteration"] == 6 and structural_key(snap["best_prog"]) == structural_key(best)
    # resume continues from the snapshot with the exact RNG stream
    cfg2 = O.SearchConfig(iters=8, N=2, K=3, seed=0, verbose=False, run_dir=run, resume=True)
    O.autotune(p, _ev(), cfg2)
    recs2 = [json.loads(l) for l in open(os.path.join(run, "log.jsonl"))]
    assert [r["iter"] for r in recs2][-2:] == [7, 8]


def test_resume_is_deterministic(tmp_path):
    p = C.p_attention_atomic()
    a, b = str(tmp_path / "a"), str(tmp_path / "b")
    O.autotune(p, _ev(), O.SearchConfig(iters=8, N=2, K=3, seed=1, verbose=False, run_dir=a))
    O.autotune(p, _ev(), O.SearchConfig(iters=4, N=2, K=3, seed=1, verbose=False, run_dir=b))
    O.autotune(p, _ev(), O.SearchConfig(iters=8, N=2, K=3, seed=1, verbose=False, run_dir=b, resume=True))
    la = [json.loads(l)["best_key"] for l in open(os.path.join(a, "log.jsonl"))]
    lb = [json.loads(l)["best_key"] for l in open(os.path.join(b, "log.jsonl"))]
    assert la[-1] == lb[-1]


def test_descent_can_reach_flash_structure_under_proxy():
    """From the 3-stage attention the full grammar can reach one stage whose
    key loop holds the online softmax (the flash structure)."""
    from grammar import rewrites as R
    p = C.p_attention()
    q = R.merge(p, p.body[0], p.body[1])
    q = R.fuse_softmax(q, q.body[0], q.body[1])
    labels = [r.label for r in O.enumerate_rewrites(q, O.DEFAULT_RULES)]
    assert "subtile(softmax_matmul,j)" in labels
    assert "split_softmax" in labels


def test_stage1_reaches_template_tilings_in_one_move():
    """A stage that lowers to the GEMM only when both its tile dims are in the
    GEMM's set (here the LN block's r = a @ W2 + X at 16 x 16, generic) is
    moved there by Stage 1's template snaps, which a one-coordinate sweep
    cannot do when every single-dim move keeps the generic lowering."""
    import run_mlp_search as RM
    from grammar import rewrites as R
    from grammar.hip_backend import template_tilings, parse_plan
    from grammar.kernel_ast import emit_module
    from grammar.optimization import stage1_sweep
    p = RM.build_mlp_ln(256, 512, 1024)
    p = R.merge(p, p.body[2], p.body[3])
    p = R.merge(p, p.body[0], p.body[1])
    for l in p.body[:2]:
        l.tile_shape = (16, 16)
    r = p.body[1]
    shapes = template_tilings(r, p)
    assert (64, 64) in shapes and (32, 128) in shapes and (16, 16) not in shapes

    class Lowering:
        """Score: 1 per generic stage, 0.1 per template stage: every
        single-dim move from 16 x 16 keeps stage r generic and scores the same."""
        def __init__(self):
            self.seen = 0

        def prefetch(self, programs):
            pass

        def __call__(self, prog):
            self.seen += 1
            try:
                steps = parse_plan(emit_module(prog))["steps"]
            except Exception:
                return 1e9                        # over LDS or not renderable: a penalty

            return sum(0.1 if s["lowering"] in ("gemm", "flash") else 1.0 for s in steps)

    import grammar.optimization as O
    out, _ = stage1_sweep(p, Lowering(), ladder=(16, 32, 64, 128, 256))
    lowerings = [s["lowering"] for s in parse_plan(emit_module(out))["steps"]]
    assert lowerings[:2] == ["gemm", "gemm"], lowerings
    # without the snaps the sweep stays on the generic lowering
    keep = O._template_snaps
    O._template_snaps = lambda work, params, ev, loss: loss
    try:
        out, _ = stage1_sweep(p, Lowering(), ladder=(16, 32, 64, 128, 256))
    finally:
        O._template_snaps = keep
    assert [s["lowering"] for s in parse_plan(emit_module(out))["steps"]][:2] == ["generic", "generic"]


def test_refine_needs_timed_scores():
    """Re-timing the finalists is a GPU step: proxy scores have nothing to re-time."""
    ev = _ev()
    ev(C.p_attention_atomic())
    with pytest.raises(RuntimeError, match="proxy"):
        ev.refine(k=3)
