"""fuse_softmax_chain / fuse_attention: the composite rewrite that gathers a
row softmax spread over several stages (merge by merge) and fuses it into the
P @ V stage, optionally with the score stages too. Every intermediate program
and the result must compute the same attention as the closed form (numpy tile
interpreter); the fully fused form must be the one stage the flash lowering
accepts."""
import numpy as np
import pytest

from grammar import optimization as O
from grammar import rewrites as R
from grammar.kernel_ast import Compute, ReductionLoop, validate
from grammar.hip_backend import _match_flash
from oracle.grammar_interp import run_program

import run_attention_search as RS


def _ins(N, d, seed=0):
    rng = np.random.default_rng(seed)
    return {"Q": rng.standard_normal((N, d)).astype(np.float32),
            "KT": rng.standard_normal((d, N)).astype(np.float32),
            "V": rng.standard_normal((N, d)).astype(np.float32)}


def _closed_form(ins, scale):
    s = (ins["Q"].astype(np.float64) @ ins["KT"]) * scale
    e = np.exp(s - s.max(-1, keepdims=True))
    return (e / e.sum(-1, keepdims=True)) @ ins["V"]


@pytest.mark.parametrize("with_scores", [False, True])
def test_chain_fusion_preserves_attention(with_scores):
    p = RS.build_attention(64, 16, tile=16)
    ins = _ins(64, 16)
    q = R.fuse_softmax_chain(p, p.body[-1], with_scores=with_scores)
    validate(q)
    assert [l.out for l in q.body] == (["O"] if with_scores else ["S", "Ss", "O"])
    assert np.allclose(run_program(q, ins)["O"], _closed_form(ins, 0.25), rtol=1e-4, atol=1e-4)
    assert len(p.body) == 8                      # the input program is untouched


def test_chain_fusion_accepts_subtiled_row_reductions():
    """rowmax and rowsum computed over key sub-tiles (ReductionLoops) still
    form the canonical chain."""
    p = RS.build_attention(64, 16, tile=16)
    for name in ("mx", "sm"):
        stage = next(l for l in p.body if l.out == name)
        red = next(s for s in stage.body if isinstance(s, Compute) and s.op in ("rowmax", "rowsum"))
        p = R.subtile_reduction(p, red, "j", tile=32)
    assert any(isinstance(s, ReductionLoop) for l in p.body for s in l.body if l.out == "mx")
    q = R.fuse_softmax_chain(p, p.body[-1], with_scores=True)
    ins = _ins(64, 16, 1)
    assert np.allclose(run_program(q, ins)["O"], _closed_form(ins, 0.25), rtol=1e-4, atol=1e-4)


def test_fused_attention_stage_lowers_to_flash():
    p = RS.build_attention(1024, 64, tile=128, B=4, H=16, dtype="fp16")
    q = R.fuse_softmax_chain(p, p.body[-1], with_scores=True)
    f = _match_flash(q.body[0], q)
    assert f is not None and f["BM"] == 128 and f["BN"] == 128 and not f["causal"]
    assert abs(f["scale"] - 0.125) < 1e-12
    pc = RS.build_attention(256, 64, tile=64, B=1, H=2, dtype="bf16", causal=True)
    qc = R.fuse_softmax_chain(pc, pc.body[-1], with_scores=True)
    fc = _match_flash(qc.body[0], qc)
    assert fc is not None and fc["causal"]


def test_menu_offers_chain_fusion_only_when_needed():
    p = RS.build_attention(64, 16, tile=16)
    labels = [r.label for r in O.enumerate_rewrites(p, O.DEFAULT_RULES)]
    assert "fuse_softmax_chain(O)" in labels and "fuse_attention(O)" in labels
    assert not any(l.startswith("fuse_softmax_chain") for l in
                   (r.label for r in O.enumerate_rewrites(p, O.REFERENCE_RULES)))
    # once fused, neither applies again
    q = R.fuse_softmax_chain(p, p.body[-1], with_scores=True)
    labels = [r.label for r in O.enumerate_rewrites(q, O.DEFAULT_RULES)]
    assert not any(l.startswith(("fuse_softmax_chain", "fuse_attention")) for l in labels)


def test_chain_fusion_rejects_shared_intermediates():
    """If a softmax intermediate is a program output it cannot be dropped."""
    p = RS.build_attention(64, 16, tile=16)
    # read `e` from an extra stage: merge(e, ...) becomes illegal
    from grammar.kernel_ast import Load, Store, ParallelLoop
    eL = Load("e", ["i", "j"])
    c = Compute("mulc", [eL], const=2.0)
    p.body.append(ParallelLoop("e2", (16, 16), ("i", "j"), [eL, c, Store("e2", c, ["i", "j"])]))
    p.tensors["e2"] = (64, 64)
    ok, why = R.can_fuse_softmax_chain(p, p.body[-2])
    assert not ok
