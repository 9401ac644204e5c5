"""The reference's own descent-found programs, rendered by this backend, on the GPU.

tests/golden/reference_runs.json holds the 42 programs the reference's
descent logged (runs/*/log.jsonl `best_key`); the 35 feasible ones are the
reference's own stage structures and tile sizes at its workload (one head,
N = 512, d = 64, fp32). Each is rebuilt from its key, rendered unchanged
(the stages take the GEMM, row and generic lowerings), run once, and checked
against the float64 oracle at the reference's GPU-test bar, rtol = atol =
1e-3 (test_renderer.py:222-223, 287). Every intermediate is allocated
NaN-filled, so a stage that leaves part of its output unwritten fails."""
import json
import os

import numpy as np
import pytest

from oracle import attention as O

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

HERE = os.path.dirname(os.path.abspath(__file__))
RECORDS = [r for r in json.load(open(os.path.join(HERE, "golden", "reference_runs.json")))["records"]
           if r["loss_kind"] == "feasible"]


@pytest.fixture(scope="module")
def compiled():
    """Code objects of all programs, compiled concurrently (hiprtc releases the GIL)."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from concurrent.futures import ThreadPoolExecutor
    from grammar.hip_module import compile_cached
    from grammar.kernel_ast import emit_module, program_from_key
    srcs = [emit_module(program_from_key(r["key"])) for r in RECORDS]
    with ThreadPoolExecutor(max_workers=8) as pool:
        codes = list(pool.map(lambda s: compile_cached(s)[0], srcs))
    return dict(zip((f"{r['run']}-it{r['iter']}" for r in RECORDS), zip(srcs, codes)))


def test_fixture_has_the_reference_finals():
    got = {(r["run"], r["iter"]) for r in RECORDS}
    # the reference's published results/attn-*.json are these runs' final best programs
    assert {("attn_full", 24), ("attn_norev", 36), ("attn_nojump", 28), ("attn_nolocal", 20)} <= got
    assert len(RECORDS) == 35


@pytest.mark.parametrize("rec", RECORDS, ids=lambda r: f"{r['run']}-it{r['iter']}")
def test_reference_program_matches_oracle(rec, compiled):
    from grammar.hip_module import HipModule
    src, code = compiled[f"{rec['run']}-it{rec['iter']}"]
    mod = HipModule(src, code)
    g = torch.Generator("cpu").manual_seed(rec["iter"])
    host = {n: torch.randn(tuple(s), generator=g) for n, s in mod.KERNEL_META["inputs"]}
    out = mod.fn(*[host[n].cuda() for n in mod.inputs])
    torch.cuda.synchronize()
    got = out.double().cpu().numpy()
    want = O.attention(host["Q"].numpy(), host["KT"].numpy(), host["V"].numpy(), k_transposed=True,
                       dtype=np.float64)
    lowering = [s["lowering"] for s in mod.plan["steps"]]
    print(f"[reference program] {rec['run']} it{rec['iter']}: {len(rec['stages'])} stages, "
          f"lowering {lowering}, max|d| {float(np.max(np.abs(got - want))):.2e}", flush=True)
    assert len(lowering) >= len(rec["stages"])
    assert np.all(np.isfinite(got)), "NaN/Inf: incomplete write"
    assert np.allclose(got, want, rtol=1e-3, atol=1e-3)
