"""GPU parity of what the benchmark times: the committed descent-found
programs for C2, C3 and C4 rendered by the HIP backend and run at their full
configs against the CPU oracle, and the live descent loop (render -> hiprtc
compile -> tolerance check -> hipEvent timing) on a small attention problem,
including a variant the checker must reject.

Reference behaviour pinned: the descent loss and its scores
(grammar/optimization.py:251-300), the final `verify` of the best program
(run_attention_search.py:169-181), the MLP block (run_mlp_search.py:42-127).
Tolerance: max-abs <= 2e-2, mean-abs <= 2e-3 against the fp32 CPU oracle on
the same rounded inputs."""
import json
import math
import os

import numpy as np
import pytest
import torch

from conftest import PKG
from oracle import attention as O

pytestmark = pytest.mark.gpu


def _cuda():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    return torch.device("cuda:0")


def _case(msg):
    print(f"[case] {msg}", flush=True)


def _load(name):
    from grammar.kernel_ast import program_from_key
    with open(os.path.join(PKG, "runs", name)) as f:
        saved = json.load(f)
    return program_from_key(saved["key"]), saved


def _check(got, ref, what):
    got = got.float().cpu().numpy() if isinstance(got, torch.Tensor) else got
    mx, mn = O.errors(got, ref)
    print(f"[check] {what}: max-abs {mx:.3e} mean-abs {mn:.3e}", flush=True)
    assert np.isfinite(mx) and mx <= O.MAX_ABS_TOL and mn <= O.MEAN_ABS_TOL, (what, mx, mn)


def test_committed_c2_program_full_config_vs_oracle():
    dev = _cuda()
    from grammar.hip_module import HipModule
    from grammar.kernel_ast import emit_module
    from grammar.workloads import C2, attention_inputs
    prog, saved = _load("attn_c2_best.json")
    _case(f"committed C2 program {saved['stages']}")
    mod = HipModule(emit_module(prog))
    assert [s["lowering"] for s in mod.plan["steps"]] == ["flash"]
    q, k, v = attention_inputs(C2, seed=0)
    kt = k.transpose(-1, -2).contiguous()
    out = mod.fn(kt.to(dev), q.to(dev), v.to(dev))
    torch.cuda.synchronize()
    ref = O.attention(q.float().numpy(), kt.float().numpy(), v.float().numpy(), k_transposed=True)
    _check(out, ref, "C2 descent program (all 64 heads)")
    again = mod.fn(kt.to(dev), q.to(dev), v.to(dev))
    assert torch.equal(out, again), "descent-found C2 kernel is not deterministic"


def test_committed_c3_program_sampled_heads_vs_oracle():
    dev = _cuda()
    from grammar.hip_module import HipModule
    from grammar.kernel_ast import emit_module
    from grammar.workloads import C3, attention_inputs
    prog, saved = _load("attn_c3_best.json")
    _case(f"committed C3 program {saved['stages']}")
    mod = HipModule(emit_module(prog))
    q, k, v = attention_inputs(C3, seed=0)
    kt = k.transpose(-1, -2).contiguous()
    out = mod.fn(kt.to(dev), q.to(dev), v.to(dev)).float().cpu()
    assert torch.isfinite(out).all()
    for b, h in ((0, 0), (1, 31), (0, 17)):
        ref = O.attention(q[b, h].float().numpy(), k[b, h].float().numpy(), v[b, h].float().numpy(), causal=True)
        _check(out[b, h], ref, f"C3 descent program head ({b},{h})")


def test_committed_c4_program_sampled_rows_vs_oracle():
    dev = _cuda()
    from grammar.hip_module import HipModule
    from grammar.kernel_ast import emit_module
    from grammar.workloads import C4, mlp_inputs
    prog, saved = _load("mlp_c4_best.json")
    _case(f"committed C4 program {saved['stages']}")
    mod = HipModule(emit_module(prog))
    x, w1, w2 = mlp_inputs(C4, seed=0)
    named = {"X": x.to(dev), "W1": w1.to(dev), "W2": w2.to(dev)}
    y = mod.fn(*[named[n] for n in mod.inputs])
    torch.cuda.synchronize()
    rows = np.random.default_rng(3).choice(C4.M, 192, replace=False)
    ref = O.mlp_silu(x[rows].float().numpy(), w1.float().numpy(), w2.float().numpy(), dtype=np.float32)
    _check(y[torch.as_tensor(rows, device=dev)], ref, "C4 descent program rows")


def _small_attention():
    import run_attention_search as RS
    return RS.build_attention(256, 64, B=1, H=2, dtype="fp16"), RS.attention_reference(1.0 / math.sqrt(64))


def test_live_descent_finds_a_kernel_that_passes_the_oracle(tmp_path, monkeypatch):
    dev = _cuda()
    monkeypatch.setenv("GR_CACHE_DIR", str(tmp_path / "co"))
    from grammar.hip_module import HipModule
    from grammar.kernel_ast import emit_module, kernel_meta
    from grammar.optimization import EvalConfig, Evaluator, SearchConfig, autotune
    prog, ref = _small_attention()
    _case("live descent B1 H2 N256 d64 fp16, 8 iterations")
    ev = Evaluator(EvalConfig(seed=0), reference=ref)
    try:
        best = autotune(prog, ev, SearchConfig(iters=8, N=2, K=4, seed=0, verbose=False, time_budget_s=60))
        st = ev.stats()
        print(f"[descent] {st}", flush=True)
        assert st["timed_variants"] > 0 and st["hiprtc_compiles"] > 0
        assert ev(best) < 1e9
        assert len(ev.timeline) == st["timed_variants"]
        # the best program against the CPU oracle on fresh seeded inputs
        g = torch.Generator("cpu").manual_seed(11)
        ins = {n: torch.randn(tuple(s), generator=g).half() for n, s in kernel_meta(best)["inputs"]}
        mod = HipModule(emit_module(best))
        out = mod.fn(*[ins[n].to(dev) for n in mod.inputs])
        torch.cuda.synchronize()
        oref = O.attention(ins["Q"].float().numpy(), ins["KT"].float().numpy(), ins["V"].float().numpy(),
                           k_transposed=True)
        _check(out, oref, "live descent best")
        # the finalists re-timed side by side: distinct scored programs, fastest first, and
        # the one returned is a scored, checked program that also passes the oracle
        from grammar.kernel_ast import structural_key
        fast, recs = ev.refine(k=3, rounds=2, iters=20, ramp_ms=5.0)
        print(f"[refine] {[(r['stages'], r['search_ms'], r['refined_ms']) for r in recs]}", flush=True)
        assert 1 <= len(recs) <= 3
        assert [r["refined_ms"] for r in recs] == sorted(r["refined_ms"] for r in recs)
        assert all(r["refined_ms"] > 0 for r in recs)
        assert structural_key(fast) in ev._cache and ev(fast) < 1e9
        assert len({emit_module(r["program"]) for r in recs}) == len(recs)
        mod = HipModule(emit_module(fast))
        out = mod.fn(*[ins[n].to(dev) for n in mod.inputs])
        torch.cuda.synchronize()
        _check(out, oref, "refined best")
    finally:
        ev.close()


def test_c5_descent_at_its_own_workload(tmp_path, monkeypatch):
    """C5 as configured: the descent from the naive 8-stage program at
    B4 H16 N1024 d64 fp16, 500 iterations (Stage 2 every 4, K = 5) with a
    60 s budget and an empty code-object cache, then the reference's final
    step: its best program checked against the closed form
    (run_attention_search.py:235-271, verify at :169-181). Here the refined
    best also runs on all 64 heads against the CPU oracle."""
    import time
    dev = _cuda()
    monkeypatch.setenv("GR_CACHE_DIR", str(tmp_path / "co"))
    import run_attention_search as RS
    from grammar.hip_module import HipModule
    from grammar.kernel_ast import emit_module
    from grammar.optimization import EvalConfig, Evaluator, SearchConfig, autotune
    from grammar.workloads import C2, attention_inputs
    prog = RS.build_attention(1024, 64, B=4, H=16, dtype="fp16")
    _case("C5 descent B4 H16 N1024 d64 fp16, 500 iterations, 60 s budget, empty code-object cache")
    budget = 60.0
    ev = Evaluator(EvalConfig(seed=0), reference=RS.attention_reference(1.0 / math.sqrt(64)))
    try:
        t0 = time.time()
        best = autotune(prog, ev, SearchConfig(iters=500, N=4, K=5, seed=0, verbose=False, time_budget_s=budget))
        wall = time.time() - t0
        st = ev.stats()
        rate = 60.0 * st["timed_variants"] / wall
        print(f"[descent] C5: {ev.iterations} iterations in {wall:.1f} s, {st['timed_variants']} timed, "
              f"{st['hiprtc_compiles']} compiles, {st['code_cache_hits']} code-cache hits, {rate:.0f} evals/min",
              flush=True)
        assert ev.iterations == 500 or wall >= budget
        assert st["timed_variants"] > 0 and st["hiprtc_compiles"] > 0
        assert rate >= 30.0, rate
        assert ev(best) < 1e9
        best, finalists = ev.refine(k=6)
        print(f"[refine] {[(r['stages'], round(r['refined_ms'] * 1e3, 2)) for r in finalists]}", flush=True)
    finally:
        ev.close()
    # the reference's final verify (seeded inputs, torch closed form on the GPU)
    assert RS.verify(best, 1024, 64)
    q, k, v = attention_inputs(C2, seed=0)
    kt = k.transpose(-1, -2).contiguous()
    mod = HipModule(emit_module(best))
    out = mod.fn(kt.to(dev), q.to(dev), v.to(dev))
    torch.cuda.synchronize()
    ref = O.attention(q.float().numpy(), kt.float().numpy(), v.float().numpy(), k_transposed=True)
    _check(out, ref, "C5 descent best (all 64 heads)")


def test_evaluator_rejects_a_variant_that_fails_the_checker(tmp_path, monkeypatch):
    _cuda()
    monkeypatch.setenv("GR_CACHE_DIR", str(tmp_path / "co"))
    from grammar.optimization import EvalConfig, Evaluator
    prog, ref = _small_attention()
    _case("evaluator: correct vs deliberately wrong reference")
    good = Evaluator(EvalConfig(seed=0), reference=ref)
    bad = Evaluator(EvalConfig(seed=0), reference=lambda named: ref(named) * 1.5 + 0.25)
    try:
        loss = good(prog)
        assert 0 < loss < 1e9 and good.stats()["timed_variants"] == 1
        assert bad(prog) == math.inf
        assert bad.stats()["timed_variants"] == 0     # never timed
        assert len(bad.timeline) == 0
    finally:
        good.close()
        bad.close()


def test_evaluator_checking_build_gate(tmp_path, monkeypatch):
    """checked_build: a variant with a generic stage also runs its checking
    build (LDS/global bounds, LDS races between barriers) before it is timed;
    the atomic attention program's stages report nothing and it is scored."""
    _cuda()
    monkeypatch.setenv("GR_CACHE_DIR", str(tmp_path / "co"))
    import grammar_cases as C
    from grammar.optimization import EvalConfig, Evaluator
    from test_check_build import _generic, fit_for_check
    prog = _generic(C.p_attention_atomic())
    fit_for_check(prog)          # tiles whose shadow words fit in LDS
    _case("evaluator: checking build of the atomic attention program")
    ev = Evaluator(EvalConfig(seed=0, checked_build=True))
    try:
        loss = ev(prog)
        st = ev.stats()
        assert 0 < loss < 1e9, loss
        assert st["checked_builds"] == 1 and st["check_findings"] == 0 and st["timed_variants"] == 1
    finally:
        ev.close()


def _ln_block_f64(x, w1, w2, eps=1e-5):
    """relu(X W1) W2 + X, then LayerNorm over the row without an affine part,
    in float64 (run_mlp_search.py:138-149)."""
    x, w1, w2 = (np.asarray(t, dtype=np.float64) for t in (x, w1, w2))
    r = np.maximum(x @ w1, 0.0) @ w2 + x
    mu = r.mean(axis=1, keepdims=True)
    var = ((r - mu) ** 2).mean(axis=1, keepdims=True)
    return (r - mu) / np.sqrt(var + eps)


def test_committed_ln_block_program_vs_closed_form():
    """The descent-found reference MLP + LayerNorm block (runs/mlp_ln_best.json:
    split-K fp32 GEMMs whose partial products the row stages sum on load),
    run twice in a row (the second run must not see the first one's partials
    twice) against the float64 closed form at the reference's 1e-3 bar."""
    dev = _cuda()
    import run_mlp_search as RM
    from grammar.hip_module import HipModule
    from grammar.kernel_ast import emit_module
    prog, saved = _load("mlp_ln_best.json")
    _case(f"committed LN block program {saved['stages']}")
    mod = HipModule(emit_module(prog))
    steps = mod.plan["steps"]
    print(f"[plan] {[(s['lowering'], s.get('tiles', {}).get('ksplit')) for s in steps]}", flush=True)
    named = RM.mlp_inputs(256, 512, 1024, "fp32", seed=5, device="cpu")
    want = _ln_block_f64(named["X"].numpy(), named["W1"].numpy(), named["W2"].numpy())
    args = [named[n].to(dev) for n in mod.inputs]
    first = mod.fn(*args)
    torch.cuda.synchronize()
    first = first.cpu().numpy()
    second = mod.fn(*args).cpu().numpy()
    for got, what in ((first, "first run"), (second, "second run")):
        err = float(np.max(np.abs(got - want)))
        print(f"[check] LN block {what}: max-abs {err:.3e}", flush=True)
        assert np.isfinite(err) and err <= 1e-3, (what, err)
    # LayerNorm rows: mean 0 and variance var/(var+eps) ~ 1
    assert np.max(np.abs(first.mean(axis=1))) < 1e-4


@pytest.mark.parametrize("rules", ["ref_n512_fp32", "ref_n512_fp32_reference_rules"])
def test_committed_reference_workload_best_vs_oracle(rules):
    """The durable best kernel of the full-rule descent at the reference's own
    workload (one head, N = 512, d = 64, fp32; runs/ablations/<rules>/full),
    loaded from its committed .hip as bench.py --kernel loads it, against the
    float64 oracle at the reference's 1e-3 bar (run_attention_search.py:160-181)."""
    dev = _cuda()
    import glob
    import re
    from grammar.hip_module import HipModule
    kdir = os.path.join(PKG, "runs", "ablations", rules, "full", "kernels")
    last = max(glob.glob(os.path.join(kdir, "best_it*.hip")), key=lambda p: int(re.findall(r"\d+", os.path.basename(p))[0]))
    _case(f"reference-workload best {rules}: {os.path.basename(last)}")
    with open(last) as f:
        mod = HipModule(f.read())
    g = torch.Generator("cpu").manual_seed(21)
    ins = {n: torch.randn(tuple(s), generator=g) for n, s in mod.KERNEL_META["inputs"]}
    out = mod.fn(*[ins[n].to(dev) for n in mod.inputs])
    torch.cuda.synchronize()
    q, kt, v = (ins[n].double().numpy() for n in ("Q", "KT", "V"))
    ref = O.attention(q, kt, v, k_transposed=True, dtype=np.float64)
    err = float(np.max(np.abs(out.double().cpu().numpy() - ref)))
    print(f"[check] {rules} {[s['lowering'] for s in mod.plan['steps']]}: max-abs {err:.3e}", flush=True)
    assert np.isfinite(err) and err <= 1e-3
