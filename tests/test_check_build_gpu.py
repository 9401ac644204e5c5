"""The checking build on the GPU (csrc/gr_check.h): the generic lowering's
programs -- every reference case, and the programs a random walk of legal
rewrites reaches from the atomic attention program -- run with every LDS
access bounds- and race-checked and every global index bounds-checked, and
must report nothing while matching the interpreter; a module with one barrier
taken out of its text must report the race it opens."""
import random

import numpy as np
import pytest

import grammar_cases as C
from grammar.kernel_ast import kernel_meta
from oracle.grammar_interp import run_program
from test_check_build import _generic, fit_for_check

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def _cuda():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _run_checked(src, prog, ins):
    from grammar.hip_module import HipModule
    dev = _cuda()
    mod = HipModule(src)
    tensors = {n: torch.from_numpy(ins[n]).to(dev).to(mod.dtype) for n in mod.inputs}
    tensors.update(mod.allocate(dev))
    mod.bind(tensors).run()
    torch.cuda.synchronize()
    out = tensors[mod.plan["outputs"][0]].float().cpu().numpy()
    return out, mod.check_report(tensors)


def _clean(rep):
    return all(rep[k] == 0 for k in ("lds_range", "global_range", "raw", "war", "waw"))


@pytest.mark.parametrize("name", [n for n in C.REFS if "flash" not in n and n != "mlp_silu"])
def test_reference_cases_run_clean(name):
    build, ref = C.REFS[name]
    prog = _generic(build())
    src = fit_for_check(prog)
    ins = C.inputs_for(prog, 0)
    print(f"[check] {name}: tiles {[tuple(l.tile_shape) for l in prog.body]}", flush=True)
    got, rep = _run_checked(src, prog, ins)
    assert _clean(rep), rep
    want = run_program(prog, ins)[kernel_meta(prog)["output"][0]]
    assert np.allclose(got, want, rtol=1e-3, atol=1e-3)
    assert np.allclose(got, ref(ins), rtol=1e-3, atol=1e-3)


def test_rewrite_walk_runs_clean():
    """Eight steps of a seeded random walk over the descent's rewrite menu from
    the atomic attention program: each program reached runs clean."""
    from grammar.optimization import DEFAULT_RULES, enumerate_rewrites
    build, ref = C.REFS["attention_atomic"]
    prog = _generic(build())
    ins = C.inputs_for(prog, 0)
    want = ref(ins)
    rng = random.Random(0)
    for step in range(8):
        menu = enumerate_rewrites(prog, DEFAULT_RULES)
        rng.shuffle(menu)
        for rw in menu:
            nxt = rw.resolve(prog)
            if nxt is None:
                continue
            try:
                src = fit_for_check(_generic(nxt))
            except Exception:
                continue          # a rewrite the generic lowering cannot render at any tiling
            prog = nxt
            break
        else:
            break
        print(f"[check] walk step {step}: {rw.label}, {len(prog.body)} stage(s)", flush=True)
        got, rep = _run_checked(src, prog, ins)
        assert _clean(rep), (rw.label, rep)
        assert np.allclose(got, want, rtol=1e-3, atol=1e-3), rw.label


def test_a_missing_barrier_is_reported():
    """The matmul's operand tiles are written by one thread mapping and read
    along whole rows by another: without the barrier between the load and the
    product, reads meet other threads' writes of the same interval (or writes
    meet reads). The kernel's indices are unchanged, so it stays in bounds."""
    build, _ = C.REFS["matmul_full_k"]
    prog = _generic(build())
    src = fit_for_check(prog)
    mm = src.index("// matmul: C = A @ B")
    last = src.rindex("GR_SYNC();", 0, mm)       # the barrier between the last load and the product
    racy = src[:last] + src[last + len("GR_SYNC();"):]
    ins = C.inputs_for(prog, 0)
    _, rep = _run_checked(src, prog, ins)
    assert _clean(rep), rep
    _, rep = _run_checked(racy, prog, ins)
    print(f"[check] barrier removed: {rep}", flush=True)
    assert rep["raw"] + rep["war"] + rep["waw"] > 0 and rep["first"] in ("raw", "war", "waw")
    assert rep["lds_range"] == 0 and rep["global_range"] == 0
