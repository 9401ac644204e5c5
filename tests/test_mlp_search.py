"""The MLP programs of run_mlp_search.py (the reference's relu + residual +
LayerNorm block, run_mlp_search.py:42-127, and the C4 SiLU block): stage
structure, FLOP counts against the closed forms, the tile interpreter against
float64 math, and which stages the HIP renderer lowers to the MFMA GEMM."""
import numpy as np
import pytest

from grammar import optimization as O
from grammar import rewrites as R
from grammar.kernel_ast import emit_module, program_flops, validate
from grammar.hip_backend import parse_plan
from oracle.grammar_interp import run_program
from oracle import attention as OA

import run_mlp_search as RM


def _ins(M, Dm, H, seed=0):
    rng = np.random.default_rng(seed)
    return {"X": rng.standard_normal((M, Dm)).astype(np.float32),
            "W1": (rng.standard_normal((Dm, H)) / np.sqrt(Dm)).astype(np.float32),
            "W2": (rng.standard_normal((H, Dm)) / np.sqrt(H)).astype(np.float32)}


def test_silu_block_structure_and_flops():
    p = RM.build_mlp_silu(8192, 4096, 11008, tile=128)
    validate(p)
    assert [l.out for l in p.body] == ["h", "a", "y"]
    flops, exact = program_flops(p)
    # two GEMMs (2MNK each) + one pointwise op per element of h
    assert exact and flops == 2 * 2 * 8192 * 4096 * 11008 + 8192 * 11008


@pytest.mark.parametrize("sk", [None, 32])
def test_silu_block_interpreter_matches_closed_form(sk):
    p = RM.build_mlp_silu(64, 64, 128, tile=32, subtile_k=sk, dtype="fp32")
    ins = _ins(64, 64, 128)
    got = run_program(p, ins)["y"]
    ref = OA.mlp_silu(ins["X"], ins["W1"], ins["W2"], dtype=np.float64)
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-5)


def test_ln_block_interpreter_matches_closed_form():
    p = RM.build_mlp_ln(64, 64, 128, tile=32, subtile_k=32)
    validate(p)
    ins = _ins(64, 64, 128, 1)
    got = run_program(p, ins)["out"]
    r = np.maximum(ins["X"].astype(np.float64) @ ins["W1"], 0) @ ins["W2"] + ins["X"]
    ref = (r - r.mean(1, keepdims=True)) / np.sqrt(r.var(1, keepdims=True) + 1e-5)
    assert np.allclose(got, ref, rtol=1e-4, atol=1e-4)
    # LayerNorm's two row sums over one stored tensor: merge_reductions applies
    # once both are sub-tiled
    labels = [r.label for r in O.enumerate_rewrites(p, O.DEFAULT_RULES)]
    assert any(l.startswith("subtile(rowsum") for l in labels)


def test_silu_fusion_lowers_both_stages_to_gemm():
    p = RM.build_mlp_silu(512, 256, 512, tile=128, subtile_k=64)
    steps = parse_plan(emit_module(p))["steps"]
    assert [s["lowering"] for s in steps] == ["gemm", "rows", "gemm"]
    q = R.merge(p, p.body[0], p.body[1])
    steps = parse_plan(emit_module(q))["steps"]
    assert [s["lowering"] for s in steps] == ["gemm", "gemm"]
    assert "gr_gemm_body<_Float16, 128, 128, 64, 2, 2, false, 2>" in emit_module(q)   # SiLU epilogue


def test_proxy_descent_on_ln_block_runs():
    p = RM.build_mlp_ln(128, 128, 256, tile=32, subtile_k=32)
    ev = O.Evaluator(O.EvalConfig(proxy=True))
    best = O.autotune(p, ev, O.SearchConfig(iters=4, N=2, K=4, seed=0, verbose=False))
    assert ev(best) <= ev(p)
    validate(best)
