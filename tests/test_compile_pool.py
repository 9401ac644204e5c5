"""CPU tests of the descent's failure paths (no GPU): hiprtc compiles in
killable worker processes, a compile past its limit scored as a penalty, a
renderer exception scored inf, and a run killed with SIGKILL resumed from its
snapshot. These pin the scoring contract of the reference's evaluator
(grammar/optimization.py:164-249 scores, :262-283 compile timeout, :966-976
resume)."""
import json
import math
import os
import signal
import subprocess
import sys
import time

import pytest

import grammar_cases as C
from conftest import PKG, REPO
from grammar import optimization as O
from grammar.compile_pool import CompilePool, CompileTimeout, WorkerDied
from grammar.kernel_ast import structural_key

FAKE = [sys.executable, "-u", os.path.join(REPO, "tests", "fake_compile_worker.py")]


def test_real_worker_compiles_on_the_host():
    pool = CompilePool(workers=1, timeout=120)
    try:
        code = pool.compile('#include "gr_common.h"\n'
                            'extern "C" __global__ void k(float* x) { x[threadIdx.x] = gr_exp2(1.0f); }\n')
        assert code[:4] == b"\x7fELF" and len(code) > 1000
        from grammar import runtime as rt
        with pytest.raises(rt.CompileError) as ei:
            pool.compile('extern "C" __global__ void k(float* x) { not c++; }\n')
        assert "error" in str(ei.value).lower()
    finally:
        pool.close()


def test_hung_compile_is_killed_and_the_pool_recovers():
    pool = CompilePool(workers=1, timeout=1.0, worker_cmd=FAKE)
    try:
        assert pool.compile("a") == b"CODE:a"
        t0 = time.monotonic()
        with pytest.raises(CompileTimeout):
            pool.compile("HANG")
        assert time.monotonic() - t0 < 15
        # the next job gets a fresh worker: the hung one cost one limit, not the pool
        assert pool.compile("b") == b"CODE:b"
        assert pool.timeouts == 1 and pool.spawned == 2
        with pytest.raises(WorkerDied):
            pool.compile("CRASH")
        assert pool.compile("c") == b"CODE:c"
    finally:
        pool.close()


def test_concurrent_jobs_with_one_hung():
    pool = CompilePool(workers=3, timeout=1.5, worker_cmd=FAKE)
    try:
        futs = [pool.submit(s) for s in ("x", "HANG", "y", "z", "FAIL")]
        assert futs[0].result() == b"CODE:x"
        with pytest.raises(CompileTimeout):
            futs[1].result()
        assert futs[2].result() == b"CODE:y" and futs[3].result() == b"CODE:z"
        with pytest.raises(Exception) as ei:
            futs[4].result()
        assert "fake compile failure" in str(ei.value)
    finally:
        pool.close()


def test_evaluator_scores_a_hung_compile_as_penalty(tmp_path, monkeypatch):
    monkeypatch.setenv("GR_CACHE_DIR", str(tmp_path / "co"))
    monkeypatch.setattr(O, "emit_module", lambda p: "HANG " + str(id(p)))
    pool = CompilePool(workers=1, timeout=1.0, worker_cmd=FAKE)
    ev = O.Evaluator(O.EvalConfig(proxy=False, compile_timeout=1.0, mem_budget=0), compiler=pool)
    try:
        assert ev(C.p_matmul_reduction()) == O.MEM_PENALTY_BASE
        assert ev.stats()["compile_timeouts"] == 1 and ev.stats()["timed_variants"] == 0
    finally:
        ev.close()


def test_evaluator_scores_a_failed_compile_and_a_render_error_as_inf(tmp_path, monkeypatch):
    monkeypatch.setenv("GR_CACHE_DIR", str(tmp_path / "co"))
    pool = CompilePool(workers=1, timeout=5.0, worker_cmd=FAKE)
    ev = O.Evaluator(O.EvalConfig(proxy=False, mem_budget=0), compiler=pool)
    try:
        monkeypatch.setattr(O, "emit_module", lambda p: "FAIL " + str(id(p)))
        assert ev(C.p_matmul_reduction()) == math.inf

        def boom(p):
            raise RuntimeError("renderer bug")
        monkeypatch.setattr(O, "emit_module", boom)
        assert ev(C.p_attention_atomic()) == math.inf
        assert ev.stats()["timed_variants"] == 0
    finally:
        ev.close()


_RUNNER = """
import sys
sys.path[:0] = [{pkg!r}, {tests!r}]
import grammar_cases as C
from grammar import optimization as O
ev = O.Evaluator(O.EvalConfig(proxy=True, mem_budget=64 * 1024, max_compile_risk=256))
O.autotune(C.p_attention_atomic(), ev, O.SearchConfig(iters={iters}, N=2, K=3, seed=3, verbose=False,
                                                      run_dir={run!r}, resume={resume}))
"""


def _runner(run, iters, resume=False):
    code = _RUNNER.format(pkg=PKG, tests=os.path.join(REPO, "tests"), iters=iters, run=run, resume=resume)
    return [sys.executable, "-c", code]


def test_sigkill_mid_run_then_resume(tmp_path):
    """A descent killed with SIGKILL resumes from its last snapshot: the log
    keeps only whole records up to the snapshot's iteration, and the resumed
    run ends where an uninterrupted run with the same seed ends."""
    whole, cut = str(tmp_path / "whole"), str(tmp_path / "cut")
    total = 40
    subprocess.run(_runner(whole, total), check=True, timeout=600)
    proc = subprocess.Popen(_runner(cut, 100000))
    snap = os.path.join(cut, "snapshot.json")
    try:
        t0 = time.monotonic()
        while time.monotonic() - t0 < 300:
            try:
                with open(snap) as f:
                    if json.load(f)["iteration"] >= 6:
                        break
            except (OSError, ValueError):
                pass
            time.sleep(0.005)
        proc.send_signal(signal.SIGKILL)
    finally:
        proc.wait(timeout=60)
    st = O.load_snapshot(cut)
    k = st["iteration"]
    assert 6 <= k < total
    subprocess.run(_runner(cut, total, resume=True), check=True, timeout=600)
    recs = [json.loads(line) for line in open(os.path.join(cut, "log.jsonl"))]
    assert [r["iter"] for r in recs] == list(range(0, total + 1))
    ref = [json.loads(line) for line in open(os.path.join(whole, "log.jsonl"))]
    assert recs[-1]["best_key"] == ref[-1]["best_key"]
    assert recs[-1]["best_loss"] == ref[-1]["best_loss"]
    assert structural_key(O.load_snapshot(cut)["best_prog"]) == structural_key(O.load_snapshot(whole)["best_prog"])
