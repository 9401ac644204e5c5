"""CPU tests of the grammar: every reference renderer case run through the
numpy tile interpreter (oracle/grammar_interp.py) against its closed-form
reference (test_renderer.py:526-543, rtol = atol = 1e-3), the validate()
reject case, the property checks and the rewrite contracts
(test_renderer.py:554-857), plus the additive rewrites."""
import math

import numpy as np
import pytest

import grammar_cases as C
from grammar import rewrites as R
from grammar.kernel_ast import (
    Load, Compute, ReductionLoop, RenderCache, program_flops, validate, structural_key,
    _infer_program, kernel_meta,
)
from oracle.grammar_interp import run_program


def _run(prog, seed=0):
    ins = C.inputs_for(prog, seed)
    out = kernel_meta(prog)["output"][0]
    return run_program(prog, ins)[out], ins


@pytest.mark.parametrize("name", list(C.REFS))
def test_case_numeric(name):
    build, ref = C.REFS[name]
    got, ins = _run(build())
    want = ref(ins)
    assert got.shape == want.shape
    assert np.all(np.isfinite(got)), "NaN/Inf: incomplete write or bad index"
    assert np.allclose(got, want, rtol=1e-3, atol=1e-3), float(np.max(np.abs(got - want)))


def test_reference_case_list_is_complete():
    assert len(C.REFERENCE_CASES) == 16 and all(n in C.REFS for n in C.REFERENCE_CASES)


def test_validate_rejects_inner_to_outer_flow():
    with pytest.raises(ValueError):
        validate(C.p_inner_escape())


def test_cache_dedup():
    cache = RenderCache()
    k1 = structural_key(C.p_matmul_reduction())
    k2 = structural_key(C.p_matmul_reduction())
    assert k1 == k2
    src, hit = cache.module(C.p_matmul_reduction())          # two separately built, equal programs
    again, hit2 = cache.module(C.p_matmul_reduction())
    assert (hit, hit2) == (False, True) and again == src
    assert cache.result(C.p_matmul_reduction()) is None
    cache.record(C.p_matmul_reduction(), 1.23)
    assert cache.result(C.p_matmul_reduction()) == 1.23


def test_flops_matmul_exact():
    flops, exact = program_flops(C.p_matmul_reduction())
    assert exact and flops == 2 * 256 * 256 * 128


def test_flops_invariant_under_tiling_and_subtile():
    p = C.p_matmul_full_k()
    mm = next(s for s in p.body[0].body if isinstance(s, Compute))
    q = R.subtile_reduction(p, mm, "k", tile=32)
    assert program_flops(p) == program_flops(q)


def _loads(prog):
    return [s for l in prog.body for s in R.statements(l.body) if isinstance(s, Load)]


def _build_red():
    return C.p_matmul_reduction()


def test_hoist_equivalence_and_no_mutation():
    base = _build_red()
    r0, _ = _run(base)
    p = base
    for src in ("x", "y"):
        p = R.hoist(p, [l for l in _loads(p) if l.source == src][0])
    r1, _ = _run(p)
    assert np.allclose(r0, r1, rtol=1e-3, atol=1e-3)
    # loads are now outside the reduction: consumers read per-iteration sub-tiles
    red = next(s for s in p.body[0].body if isinstance(s, ReductionLoop))
    assert not any(isinstance(s, Load) for s in red.body)
    # the input tree is untouched
    rb = next(s for s in base.body[0].body if isinstance(s, ReductionLoop))
    assert any(isinstance(s, Load) for s in rb.body)


def test_sink_roundtrip():
    base = _build_red()
    r0, _ = _run(base)
    p = base
    for src in ("x", "y"):
        p = R.hoist(p, [l for l in _loads(p) if l.source == src][0])
    for src in ("x", "y"):
        red = next(s for s in p.body[0].body if isinstance(s, ReductionLoop))
        p = R.sink(p, [l for l in _loads(p) if l.source == src][0], red)
    r2, _ = _run(p)
    assert np.allclose(r0, r2, rtol=1e-3, atol=1e-3)
    assert structural_key(p) == structural_key(base) or len(_loads(p)) == 2


def test_hoist_precondition():
    p = _build_red()
    p = R.hoist(p, [l for l in _loads(p) if l.source == "x"][0])
    top = [l for l in _loads(p) if l.source == "x"][0]
    assert not R.can_hoist(p, top)[0]


def test_sink_precondition_outside_consumer():
    from grammar.kernel_ast import Program, ParallelLoop, Store
    bx, by = Load("x", ["n", "k"]), Load("y", ["k", "m"])
    bmm = Compute("matmul", [bx, by])
    bred = ReductionLoop("k", 32, [bx, by, bmm], bmm)
    bb = Load("b", ["n", "m"])
    brelu = Compute("relu", [bb])
    bad = Program({"x": (256, 128), "y": (128, 256), "b": (256, 256), "c": (256, 256)},
                  [ParallelLoop("c", (64, 64), ("n", "m"), [bb, brelu, bred, Store("c", bred, ["n", "m"])])])
    assert not R.can_sink(bad, bb, bred)[0]


def _fullk():
    p = C.p_matmul_full_k()
    return p, next(s for s in p.body[0].body if isinstance(s, Compute))


def test_subtile_reduction_equivalence_and_no_mutation():
    full, mm = _fullk()
    r0, _ = _run(full)
    p = R.subtile_reduction(full, mm, "k", tile=32)
    r1, _ = _run(p)
    assert np.allclose(r0, r1, rtol=1e-3, atol=1e-3)
    assert any(isinstance(s, ReductionLoop) for s in p.body[0].body)
    assert any(s is mm for s in full.body[0].body)


def test_subtile_precondition():
    full, mm = _fullk()
    assert not R.can_subtile_reduction(full, mm, "n")[0]
    relu = C.p_relu()
    r = next(s for s in relu.body[0].body if isinstance(s, Compute))
    assert not R.can_subtile_reduction(relu, r, "n")[0]
    p = R.subtile_reduction(full, mm, "k", tile=32)
    rl = next(s for s in p.body[0].body if isinstance(s, ReductionLoop))
    assert not R.can_subtile_reduction(p, rl.partial, "k")[0]


def test_unwrap_is_exact_inverse():
    full, mm = _fullk()
    wrapped = R.subtile_reduction(full, mm, "k", tile=32)
    rl = next(s for s in wrapped.body[0].body if isinstance(s, ReductionLoop))
    back = R.unwrap_reduction(wrapped, rl)
    assert structural_key(back) == structural_key(full)


def test_unwrap_precondition_rejects_sunk_load():
    full, mm = _fullk()
    wrapped = R.subtile_reduction(full, mm, "k", tile=32)
    rl = next(s for s in wrapped.body[0].body if isinstance(s, ReductionLoop))
    lx = [s for s in wrapped.body[0].body if isinstance(s, Load) and s.source == "x"][0]
    w2 = R.sink(wrapped, lx, rl)
    rl2 = next(s for s in w2.body[0].body if isinstance(s, ReductionLoop))
    assert not R.can_unwrap_reduction(w2, rl2)[0]


def _two_stage():
    from grammar.kernel_ast import Program, ParallelLoop, Store
    x, y = Load("x", ["n", "k"]), Load("y", ["k", "m"])
    mm = Compute("matmul", [x, y])
    s1 = ParallelLoop("a", (64, 64), ("n", "m"), [x, y, mm, Store("a", mm, ["n", "m"])])
    a2, b2 = Load("a", ["n", "m"]), Load("b", ["n", "m"])
    add = Compute("add", [a2, b2])
    s2 = ParallelLoop("o", (64, 64), ("n", "m"), [a2, b2, add, Store("o", add, ["n", "m"])])
    return Program({"x": (256, 128), "y": (128, 256), "b": (256, 256), "a": (256, 256), "o": (256, 256)},
                   [s1, s2]), s1, s2


def test_merge_equivalence_and_no_mutation():
    two, s1, s2 = _two_stage()
    r0, _ = _run(two)
    fused = R.merge(two, s1, s2)
    r1, _ = _run(fused)
    assert np.allclose(r0, r1, rtol=1e-3, atol=1e-3)
    assert len(fused.body) == 1 and "a" not in fused.tensors
    assert len(two.body) == 2 and "a" in two.tensors


def test_merge_precondition_shared_intermediate():
    from grammar.kernel_ast import ParallelLoop, Store
    three, t1, t2 = _two_stage()
    a3 = Load("a", ["n", "m"])
    r3 = Compute("relu", [a3])
    three.body.append(ParallelLoop("z", (64, 64), ("n", "m"), [a3, r3, Store("z", r3, ["n", "m"])]))
    three.tensors["z"] = (256, 256)
    assert not R.can_merge(three, t1, t2)[0]


def _two_reductions():
    from grammar.kernel_ast import Program, ParallelLoop, Store
    xa = Load("x", ["n", "k"])
    s1 = Compute("rowsum", [xa], axis="k")
    RL1 = ReductionLoop("k", 64, [xa, s1], s1)
    xb = Load("x", ["n", "k"])
    sq = Compute("mul", [xb, xb])
    s2 = Compute("rowsum", [sq], axis="k")
    RL2 = ReductionLoop("k", 64, [xb, sq, s2], s2)
    comb = Compute("add", [RL1, RL2])
    pl = ParallelLoop("O", (64, 1), ("n", "k"), [RL1, RL2, comb, Store("O", comb, ["n", "k"])])
    return Program({"x": (128, 256), "O": (128, 1)}, [pl]), RL1, RL2


def test_merge_reductions_equivalence_single_load_no_mutation():
    tr, RL1, RL2 = _two_reductions()
    r0, ins = _run(tr)
    want = ins["x"].sum(-1, keepdims=True) + (ins["x"] ** 2).sum(-1, keepdims=True)
    assert np.allclose(r0, want, rtol=1e-3, atol=1e-3)
    fused = R.merge_reductions(tr, RL1, RL2)
    r1, _ = _run(fused)
    assert np.allclose(r0, r1, rtol=1e-3, atol=1e-3)
    reds = [s for s in fused.body[0].body if isinstance(s, ReductionLoop)]
    assert len(reds) == 1 and len(reds[0].partials) == 2
    assert len([l for l in _loads(fused) if l.source == "x"]) == 1
    assert len([s for s in tr.body[0].body if isinstance(s, ReductionLoop)]) == 2


def test_merge_reductions_precondition_dependent():
    from grammar.kernel_ast import Program, ParallelLoop, Store
    xa2 = Load("x", ["n", "k"])
    m1 = Compute("rowmax", [xa2], axis="k")
    D1 = ReductionLoop("k", 64, [xa2, m1], m1)
    xb2 = Load("x", ["n", "k"])
    sb = Compute("sub", [xb2, D1])
    e2 = Compute("exp", [sb])
    s2b = Compute("rowsum", [e2], axis="k")
    D2 = ReductionLoop("k", 64, [xb2, sb, e2, s2b], s2b)
    dep = Program({"x": (128, 256), "O": (128, 1)},
                  [ParallelLoop("O", (64, 1), ("n", "k"), [D1, D2, Store("O", D2, ["n", "k"])])])
    assert not R.can_merge_reductions(dep, D1, D2)[0]


def _three_stage():
    from grammar.kernel_ast import Program, ParallelLoop, Store
    x, y = Load("x", ["n", "k"]), Load("y", ["k", "m"])
    mm = Compute("matmul", [x, y])
    sA = ParallelLoop("a", (64, 64), ("n", "m"), [x, y, mm, Store("a", mm, ["n", "m"])])
    w = Load("w", ["n", "m"])
    rz = Compute("relu", [w])
    sZ = ParallelLoop("z", (64, 64), ("n", "m"), [w, rz, Store("z", rz, ["n", "m"])])
    a2, b2 = Load("a", ["n", "m"]), Load("b", ["n", "m"])
    add = Compute("add", [a2, b2])
    sO = ParallelLoop("o", (64, 64), ("n", "m"), [a2, b2, add, Store("o", add, ["n", "m"])])
    return Program({"x": (256, 128), "y": (128, 256), "w": (256, 256), "b": (256, 256), "a": (256, 256),
                    "z": (256, 256), "o": (256, 256)}, [sA, sZ, sO]), sA, sZ, sO


def test_reorder_enables_merge_and_no_mutation():
    tri, sA, sZ, sO = _three_stage()
    assert not R.can_merge(tri, sA, sO)[0]
    re = R.reorder(tri, sZ, sO)
    sA2 = next(s for s in re.body if s.out == "a")
    sO2 = next(s for s in re.body if s.out == "o")
    assert R.can_merge(re, sA2, sO2)[0]
    assert [s.out for s in re.body] == ["a", "o", "z"]
    assert [s.out for s in tri.body] == ["a", "z", "o"]


def test_reorder_precondition():
    from grammar.kernel_ast import Program, ParallelLoop, Store
    raw, rsA, _, rsO = _three_stage()
    raw2 = Program(dict(raw.tensors), [rsA, rsO])
    assert not R.can_reorder(raw2, rsA, rsO)[0]
    la, lb = Load("a", ["n", "m"]), Load("b", ["n", "m"])
    ad = Compute("add", [la, lb])
    sp = Program({"a": (256, 256), "b": (256, 256), "o": (256, 256)},
                 [ParallelLoop("o", (64, 64), ("n", "m"), [la, lb, ad, Store("o", ad, ["n", "m"])])])
    assert R.can_reorder(sp, la, lb)[0]
    assert not R.can_reorder(sp, lb, ad)[0]


# ---- additive rewrites ----------------------------------------------------
def test_fuse_softmax_then_flash_structure_equivalence():
    """p_attention (S, P, O stages) -> fuse_softmax(P, O) -> subtile over j ->
    sink QK^T and the K/V loads into the loop: every step computes the same
    attention, the final program is the one-stage flash form, and
    program_flops never changes."""
    p = C.p_attention()
    r0, ins = _run(p)
    f0 = program_flops(p)
    sP, sO = p.body[1], p.body[2]
    assert R.can_fuse_softmax(p, sP, sO)[0]
    q = R.fuse_softmax(p, sP, sO)
    assert len(q.body) == 2 and "P" not in q.tensors
    assert np.allclose(_run(q)[0], r0, rtol=1e-3, atol=1e-3)
    assert program_flops(q) == f0
    # the S stage iterates (i, j), the fused stage (i, dd): merge (same index
    # vars only, as in the reference) must therefore run before the fusion
    assert not R.can_merge(q, q.body[0], q.body[1])[0]
    q = R.merge(p, p.body[0], p.body[1])
    q = R.fuse_softmax(q, q.body[0], q.body[1])
    assert len(q.body) == 1
    assert np.allclose(_run(q)[0], r0, rtol=1e-3, atol=1e-3)
    smm = next(s for s in q.body[0].body if isinstance(s, Compute) and s.op == "softmax_matmul")
    q = R.subtile_reduction(q, smm, "j", tile=32)
    assert np.allclose(_run(q)[0], r0, rtol=1e-3, atol=1e-3)
    rl = next(s for s in q.body[0].body if isinstance(s, ReductionLoop))
    S = next(s for s in q.body[0].body if isinstance(s, Compute) and s.op == "matmul")
    assert R.can_sink_compute(q, S, rl)[0]
    q = R.sink_compute(q, S, rl)
    rl = next(s for s in q.body[0].body if isinstance(s, ReductionLoop))
    for src in ("KT", "V"):
        ld = [l for l in _loads(q) if l.source == src][0]
        q = R.sink(q, ld, rl)
        rl = next(s for s in q.body[0].body if isinstance(s, ReductionLoop))
    assert np.allclose(_run(q)[0], r0, rtol=1e-3, atol=1e-3)
    assert program_flops(q) == f0
    srcs = {l.source for l in _loads(q) if any(l is s for s in rl.body)}
    assert srcs == {"KT", "V"}
    # peak tile now bounded by the key tile, not the full row
    shapes = _infer_program(q)
    assert max(math.prod(shapes[id(s)]) for s in rl.body if id(s) in shapes) <= 64 * 64


def test_split_softmax_inverts_fuse():
    p = C.p_attention()
    r0, _ = _run(p)
    q = R.fuse_softmax(p, p.body[1], p.body[2])
    smm = next(s for s in q.body[1].body if isinstance(s, Compute) and s.op == "softmax_matmul")
    assert R.can_split_softmax(q, smm)[0]
    back = R.split_softmax(q, smm)
    assert len(back.body) == 3
    assert np.allclose(_run(back)[0], r0, rtol=1e-3, atol=1e-3)
    assert program_flops(back) == program_flops(p)


def test_fuse_softmax_preconditions():
    p = C.p_attention()
    assert not R.can_fuse_softmax(p, p.body[0], p.body[1])[0]      # S stage stores no softmax
    assert not R.can_fuse_softmax(p, p.body[1], p.body[0])[0]      # not producer -> consumer order
    a = C.p_attention_atomic()
    assert not R.can_fuse_softmax(a, a.body[5], a.body[6])[0]      # P = e/sm split across stages


def test_hoist_compute_inverts_sink_compute():
    q = C.p_flash_attention(B=1, H=1, N=64, d=32, bm=32, bn=16)
    r0, _ = _run(q)
    rl = next(s for s in q.body[0].body if isinstance(s, ReductionLoop))
    kt = next(s for s in rl.body if isinstance(s, Load) and s.source == "KT")
    S = next(s for s in rl.body if isinstance(s, Compute) and s.op == "matmul")
    assert not R.can_hoist_compute(q, S)[0]       # reads KT loaded inside the loop
    q1 = R.hoist(q, kt)
    S1 = next(s for s in R.statements(q1.body[0].body) if isinstance(s, Compute) and s.op == "matmul")
    assert R.can_hoist_compute(q1, S1)[0]
    q2 = R.hoist_compute(q1, S1)
    assert np.allclose(_run(q2)[0], r0, rtol=1e-3, atol=1e-3)
    rl2 = next(s for s in q2.body[0].body if isinstance(s, ReductionLoop))
    S2 = next(s for s in q2.body[0].body if isinstance(s, Compute) and s.op == "matmul")
    q3 = R.sink_compute(q2, S2, rl2)
    assert np.allclose(_run(q3)[0], r0, rtol=1e-3, atol=1e-3)


def test_sink_compute_rejects_loop_axis_reduction():
    p = C.p_softmax()
    red_in = next(s for s in p.body[0].body if isinstance(s, Compute) and s.op == "rowsum")
    p2 = R.subtile_reduction(p, red_in, "m", tile=64)
    rl = next(s for s in p2.body[0].body if isinstance(s, ReductionLoop))
    mx = next(s for s in p2.body[0].body if isinstance(s, Compute) and s.op == "rowmax")
    assert not R.can_sink_compute(p2, mx, rl)[0]


def test_program_from_key_binds_duplicate_loads_by_tile():
    """A stage that reads one tensor twice at different tile shapes (the row
    max over the full row, the subtraction over the tile) rebuilds from its
    structural key with each operand bound to the right load."""
    import run_attention_search as RS
    from grammar import rewrites as Rw
    from grammar.kernel_ast import _infer_program, program_from_key
    p = RS.build_attention(64, 16, tile=16)
    names = [l.out for l in p.body]
    i = names.index("mx")
    q = Rw.merge(p, p.body[i], p.body[i + 1])
    _infer_program(q)
    k = structural_key(q)
    r = program_from_key(k)
    _infer_program(r)
    assert structural_key(r) == k
