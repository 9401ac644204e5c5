"""Golden vectors from the reference's own search logs (tests/golden/
reference_runs.json, written by tests/golden/make_fixtures.py from
runs/*/log.jsonl): 42 programs the reference's descent committed, each with
the flops, flops_exact and peak_tile_bytes the reference computed for it.

Each program is rebuilt from its structural key and this grammar's
program_flops / peak_tile_bytes must reproduce the logged values; the rebuilt
program's structural key must round-trip; and the interpreter must run each
one to the same attention output as the closed form."""
import json
import os

import numpy as np
import pytest

from grammar.kernel_ast import program_flops, peak_tile_bytes, program_from_key, structural_key, validate

HERE = os.path.dirname(os.path.abspath(__file__))
RECORDS = json.load(open(os.path.join(HERE, "golden", "reference_runs.json")))["records"]


def _tuplify(x):
    return tuple(_tuplify(i) for i in x) if isinstance(x, list) else x


def test_fixture_count():
    assert len(RECORDS) == 42
    assert {r["flops"] for r in RECORDS} == {68681728}


@pytest.mark.parametrize("rec", RECORDS, ids=lambda r: f"{r['run']}-it{r['iter']}")
def test_reference_logged_flops_and_tile_bytes(rec):
    prog = program_from_key(rec["key"])
    validate(prog)
    assert structural_key(prog) == _tuplify(rec["key"])
    assert [[s.out, list(s.tile_shape)] for s in prog.body] == rec["stages"]
    flops, exact = program_flops(prog)
    assert (flops, exact) == (rec["flops"], rec["flops_exact"])
    assert peak_tile_bytes(prog) == rec["peak_tile_bytes"]


@pytest.mark.parametrize("rec", [r for r in RECORDS if r["loss_kind"] == "feasible"][:12],
                         ids=lambda r: f"{r['run']}-it{r['iter']}")
def test_reference_programs_compute_attention(rec):
    from oracle.grammar_interp import run_program
    prog = program_from_key(rec["key"])
    rng = np.random.default_rng(1)
    ins = {"Q": rng.standard_normal((512, 64)).astype(np.float32),
           "KT": rng.standard_normal((64, 512)).astype(np.float32),
           "V": rng.standard_normal((512, 64)).astype(np.float32)}
    out = run_program(prog, ins)["O"]
    s = (ins["Q"].astype(np.float64) @ ins["KT"]) / 8.0
    e = np.exp(s - s.max(-1, keepdims=True))
    ref = (e / e.sum(-1, keepdims=True)) @ ins["V"]
    assert np.allclose(out, ref, rtol=1e-3, atol=1e-3)
