"""CPU checks of the HIP renderer: every grammar case renders to a launch plan
and compiles for gfx950 through hiprtc (no device needed), and the emitted
source shows the structure the rewrites produce -- the counterparts of the
reference's source-text checks (test_renderer.py:593-857: ct.extract after
hoist, ct.mma after subtile, identical source after unwrap(subtile), one load
after merge_reductions)."""
import pytest

import grammar_cases as C
from grammar import rewrites as R
from grammar.hip_backend import parse_plan, render_module, UnsupportedProgram, LdsOverflow
from grammar.kernel_ast import emit_module, Compute, ReductionLoop, Load


@pytest.mark.parametrize("name", list(C.REFS))
def test_renders_and_compiles(name):
    from grammar import runtime as rt
    src = emit_module(C.REFS[name][0]())
    plan = parse_plan(src)
    assert plan["steps"] and all(s["lds"] <= 160 * 1024 for s in plan["steps"])
    code = rt.compile_source(src, name + ".hip")
    assert code[:4] == b"\x7fELF"


def test_plan_matches_kernel_meta():
    p = C.p_attention_atomic()
    plan = parse_plan(emit_module(p))
    assert plan["inputs"] == ["KT", "Q", "V"] and plan["outputs"] == ["O"]
    assert plan["meta"]["flops"] == 4 * 128 * 128 * 64 + 5 * 128 * 128 and plan["meta"]["flops_exact"]
    assert [s["kernel"] for s in plan["steps"]] == [f"t_{n}_kernel" for n in ("S", "mx", "sb", "e", "sm", "P", "O")]


def _loads(p):
    return [s for l in p.body for s in R.statements(l.body) if isinstance(s, Load)]


def _generic(p):
    """Pin every stage to the generic LDS-tile lowering (fp32 matmul stages
    otherwise lower to the fp32 MFMA GEMM)."""
    for l in p.body:
        l.knobs["lowering"] = "generic"
    return p


def test_hoist_emits_subtile_reads_and_sink_removes_them():
    p = _generic(C.p_matmul_reduction())
    assert "GR_SUBTILE" not in emit_module(p)
    for src in ("x", "y"):
        p = R.hoist(p, [l for l in _loads(p) if l.source == src][0])
    assert "GR_SUBTILE" in emit_module(p)
    for src in ("x", "y"):
        red = next(s for s in p.body[0].body if isinstance(s, ReductionLoop))
        p = R.sink(p, [l for l in _loads(p) if l.source == src][0], red)
    assert "GR_SUBTILE" not in emit_module(p)


def test_subtile_emits_accumulating_mma():
    p = _generic(C.p_matmul_full_k())
    mm = next(s for s in p.body[0].body if isinstance(s, Compute))
    src_full = emit_module(p)
    q = R.subtile_reduction(p, mm, "k", tile=32)
    src_red = emit_module(q)
    assert "mma: acc += A @ B" in src_red and "mma: acc += A @ B" not in src_full


def test_unwrap_subtile_reproduces_source():
    p = _generic(C.p_matmul_full_k())
    mm = next(s for s in p.body[0].body if isinstance(s, Compute))
    w = R.subtile_reduction(p, mm, "k", tile=32)
    rl = next(s for s in w.body[0].body if isinstance(s, ReductionLoop))
    assert emit_module(R.unwrap_reduction(w, rl)) == emit_module(p)


def test_merge_reductions_single_load():
    from test_grammar import _two_reductions
    tr, a, b = _two_reductions()
    def n_loads(src):
        # generic lowering: scalar LDS fills; row lowering: one vector load per pass
        return src.count("(float)t_x[") + src.count(", t_x + ")
    assert n_loads(emit_module(tr)) == 2
    assert n_loads(emit_module(R.merge_reductions(tr, a, b))) == 1


def test_flash_lowering_selected_for_fp16_flash_structure():
    p = C.p_flash_attention(B=2, H=2, N=256, d=64, bm=128, bn=64, dtype="fp16")
    plan = parse_plan(emit_module(p))
    assert [s["lowering"] for s in plan["steps"]] == ["flash"]
    assert plan["steps"][0]["tiles"] == {"block_m": 128, "block_n": 64, "waves": 4, "qb": 1, "pipe": 0, "causal": False}
    # the same structure in fp32: the fp32 flash kernel, keys split over waves
    # (block_n keys per wave), its partials in module-scope device arrays
    p32 = C.p_flash_attention(B=2, H=2, N=256, d=64, bm=64, bn=32, dtype="fp32")
    src32 = emit_module(p32)
    st, mg = parse_plan(src32)["steps"]
    assert st["lowering"] == "flash" and st["grid"] == [4 * 8 * 4, 1, 1] and st["block"] == [128, 1, 1]
    assert st["tiles"] == {"block_m": 64, "block_n": 32, "waves": 2, "parts": 4}
    assert "gr_flash32_fwd_body<64, 32, 2, true, 4>" in src32 and '#include "gr_flash_f32.h"' in src32
    assert f"__device__ float gr_ws_t_O[{4 * 4 * 256 * 64}];" in src32
    # the second launch merges the 4 partials of each query: one thread per 8 head dims
    assert mg["kernel"] == "t_O_merge_kernel" and mg["merge"] and mg["grid"] == [4 * 256 * 8 // 256, 1, 1]
    assert "gr_flash32_merge_body<64, 4>" in src32
    # one workgroup per query block (every key in its waves): no workspace
    one = parse_plan(emit_module(C.p_flash_attention(B=1, H=1, N=256, d=64, bm=128, bn=64, dtype="fp32")))
    assert one["steps"][0]["tiles"]["parts"] == 1 and len(one["steps"]) == 1
    # causal fp32 stays on the generic lowering; so does a workspace past the cap
    p32c = C.p_flash_attention(B=2, H=2, N=256, d=64, bm=32, bn=32, causal=True, dtype="fp32")
    assert parse_plan(emit_module(p32c))["steps"][0]["lowering"] == "generic"
    pbig = C.p_flash_attention(B=4, H=16, N=1024, d=64, bm=128, bn=32, dtype="fp32")
    assert parse_plan(emit_module(pbig))["steps"][0]["lowering"] == "generic"
    # unsupported query tile -> generic (never a silent mismatch)
    p48 = C.p_flash_attention(B=1, H=1, N=256, d=64, bm=16, bn=64, dtype="fp16")
    assert parse_plan(emit_module(p48))["steps"][0]["lowering"] == "generic"


def test_flash_schedule_knobs_reach_the_renderer_and_the_key():
    """The flash stage's schedule knobs (the two-waves-per-SIMD body, query
    blocks per wave, software pipelining) are descent parameters: they change
    the rendered kernel and the structural key, survive program_from_key, and
    the renderer's default is stored as an absent knob."""
    from grammar import optimization as O
    from grammar.kernel_ast import program_from_key, structural_key
    p = C.p_flash_attention(B=2, H=2, N=512, d=64, bm=256, bn=64, dtype="fp16")
    names = {q.name: q for q in O.parameter_vector(p)}
    # fp16, d 64, non-causal, 256 x 64: the two-wave body is on by default and
    # is then the only flash knob
    assert [n for n in names if n.startswith("SCHED_")] == ["SCHED_O.w2"] and names["SCHED_O.w2"].current == 1
    src = emit_module(p)
    assert "gr_flash_w2_body<true>(a, gr_flash_smem);" in src and '#include "gr_flash_w2.h"' in src
    st = parse_plan(src)["steps"][0]
    assert st["block"] == [512, 1, 1] and st["lds"] == 163840 and st["grid"] == [4 * 2, 1, 1]
    assert st["tiles"] == {"block_m": 256, "block_n": 64, "waves": 8, "qb": 1, "pipe": 0, "causal": False, "w2": 1}
    w2_key, w2_src = structural_key(p), src
    names["SCHED_O.w2"].set(0)
    assert p.body[0].knobs == {"w2": 0} and structural_key(p) != w2_key
    assert "gr_flash_w2" not in emit_module(p)
    names = {q.name: q for q in O.parameter_vector(p)}
    assert {"SCHED_O.qb", "SCHED_O.pipe", "SCHED_O.w2"} <= set(names)
    assert names["SCHED_O.qb"].ladder() == [1, 2] and names["SCHED_O.pipe"].current == 0
    assert names["SCHED_O.w2"].current == 0
    base_key, base_src = structural_key(p), emit_module(p)
    names["SCHED_O.pipe"].set(1)
    names["SCHED_O.qb"].set(2)
    assert p.body[0].knobs == {"w2": 0, "pipe": 1, "qb": 2}
    tiles = parse_plan(emit_module(p))["steps"][0]["tiles"]
    assert tiles == {"block_m": 256, "block_n": 64, "waves": 4, "qb": 2, "pipe": 1, "causal": False}
    assert "gr_flash_fwd_body<_Float16, 64, 64, 4, 2, false, true, true," in emit_module(p)
    key = structural_key(p)
    assert key != base_key and structural_key(program_from_key(key)) == key
    names["SCHED_O.pipe"].set(0)
    names["SCHED_O.qb"].set(1)
    assert p.body[0].knobs == {"w2": 0} and structural_key(p) == base_key and emit_module(p) == base_src
    names["SCHED_O.w2"].set(1)
    assert p.body[0].knobs == {} and structural_key(p) == w2_key and emit_module(p) == w2_src
    # the two-wave body does not apply to other shapes: bf16, causal, other tiles
    for q in (C.p_flash_attention(B=1, H=2, N=512, d=64, bm=256, bn=64, dtype="bf16"),
              C.p_flash_attention(B=1, H=2, N=512, d=64, bm=256, bn=64, causal=True, dtype="fp16"),
              C.p_flash_attention(B=1, H=2, N=512, d=64, bm=256, bn=128, dtype="fp16"),
              C.p_flash_attention(B=1, H=2, N=512, d=64, bm=128, bn=64, dtype="fp16"),
              C.p_flash_attention(B=1, H=2, N=512, d=64, bm=256, bn=64, scale=1.0, dtype="fp16")):
        assert "SCHED_O.w2" not in {x.name for x in O.parameter_vector(q)} and "gr_flash_w2" not in emit_module(q)
    # head dim 128 offers no second query block per wave
    p128 = C.p_flash_attention(B=1, H=2, N=256, d=128, bm=128, bn=64, dtype="bf16")
    assert [q.name for q in O.parameter_vector(p128) if q.name.startswith("SCHED_")] == ["SCHED_O.pipe"]
    # the atomic fp32 program offers no flash knobs; its fp32 GEMM stages (S, O) offer split K
    sched = [q.name for q in O.parameter_vector(C.p_attention_atomic()) if q.name.startswith("SCHED_")]
    assert sched == ["SCHED_S.ksplit", "SCHED_O.ksplit"], sched


def test_flash_head_dim_128_two_wave_body():
    """Head dim 128 at 256 x 64 tiles (fp16 or bf16, causal or not, N a
    multiple of 256) renders the d = 128 two-waves-per-SIMD body
    (gr_flash_w2h.h), on by default and then the only flash knob; off, the
    stage falls back to the flash body with its pipelining knob."""
    from grammar import optimization as O
    for dt, ctype, causal in (("bf16", "__bf16", True), ("fp16", "_Float16", False), ("bf16", "__bf16", False)):
        p = C.p_flash_attention(B=2, H=2, N=512, d=128, bm=256, bn=64, causal=causal, dtype=dt)
        names = {q.name: q for q in O.parameter_vector(p)}
        assert [n for n in names if n.startswith("SCHED_")] == ["SCHED_O.w2"] and names["SCHED_O.w2"].current == 1
        src = emit_module(p)
        assert f"gr_flash_w2h_body<{ctype}, {'true' if causal else 'false'}>(a, gr_flash_smem);" in src
        assert '#include "gr_flash_w2h.h"' in src and '#include "gr_flash_w2.h"' not in src
        st = parse_plan(src)["steps"][0]
        assert st["block"] == [512, 1, 1] and st["lds"] == 163840 and st["grid"] == [4 * 2, 1, 1]
        assert st["tiles"] == {"block_m": 256, "block_n": 64, "waves": 8, "qb": 1, "pipe": 0, "causal": causal,
                               "w2": 1}
        names["SCHED_O.w2"].set(0)
        assert "gr_flash_w2h" not in emit_module(p) and parse_plan(emit_module(p))["steps"][0]["block"] == [512, 1, 1]
        names = {q.name: q for q in O.parameter_vector(p)}
        assert {"SCHED_O.pipe", "SCHED_O.w2"} == {n for n in names if n.startswith("SCHED_")}
    # other tiles keep the flash body
    for q in (C.p_flash_attention(B=1, H=2, N=512, d=128, bm=128, bn=64, causal=True, dtype="bf16"),
              C.p_flash_attention(B=1, H=2, N=512, d=128, bm=256, bn=32, dtype="bf16")):
        assert "SCHED_O.w2" not in {x.name for x in O.parameter_vector(q)} and "gr_flash_w2h" not in emit_module(q)


def test_fp16_flash_with_large_scale_skips_the_q_prescale():
    """The fp16 flash kernel rounds Q * scale * log2(e) to fp16; a module whose
    flash stage has scale * log2(e) > 1 turns that off (GR_FLASH_OPT 0)."""
    big = C.p_flash_attention(B=1, H=2, N=256, d=64, bm=128, bn=64, scale=1.0, dtype="fp16")
    assert emit_module(big).startswith("#define GR_FLASH_OPT 0")
    assert "GR_FLASH_OPT" not in emit_module(C.p_flash_attention(B=1, H=2, N=256, d=64, bm=128, bn=64, dtype="fp16"))
    assert "GR_FLASH_OPT" not in emit_module(C.p_flash_attention(B=1, H=2, N=256, d=64, bm=128, bn=64, scale=1.0,
                                                                 dtype="bf16"))


def test_lds_overflow_is_reported():
    from grammar.kernel_ast import Program, ParallelLoop, Store
    # an fp32 matmul stage (generic lowering) whose operand tiles need 1.5 MiB
    x, w = Load("x", ["n", "k"]), Load("w", ["k", "m"])
    r = Compute("matmul", [x, w])
    big = Program({"x": (512, 512), "w": (512, 512), "o": (512, 512)},
                  [ParallelLoop("o", (256, 512), ("n", "m"), [x, w, r, Store("o", r, ["n", "m"])])])
    with pytest.raises(LdsOverflow):
        render_module(big)
    # a pointwise stage of the same tile needs no LDS: the row lowering streams it
    y = Load("x", ["n", "m"])
    rl = Compute("relu", [y])
    pw = Program({"x": (512, 512), "o": (512, 512)},
                 [ParallelLoop("o", (256, 512), ("n", "m"), [y, rl, Store("o", rl, ["n", "m"])])])
    assert parse_plan(render_module(pw))["steps"][0]["lowering"] == "rows"


def test_residual_add_lowers_to_the_gemm_epilogue():
    """A stage computing A @ B + R (R loaded at the output's indices) lowers to
    the GEMM with the residual epilogue flag (GR_EPI_RES = 4) and R's
    pointer and strides in the argument block; an add of anything else keeps
    the generic lowering."""
    import run_mlp_search as RM
    from grammar import rewrites as R
    for dt, body in (("fp32", "gr_gemm_f32_body<64, 64, 32, 2, 2, false, 4>"),
                     ("fp16", "gr_gemm_body<_Float16, 64, 64, 64, 1, 1, false, 4>")):
        p = RM.build_mlp_ln(256, 512, 1024, tile=64, dtype=dt)
        p = R.merge(p, p.body[2], p.body[3])
        src = emit_module(p)
        st = [s for s in parse_plan(src)["steps"] if s["kernel"] == "t_r_kernel"][0]
        assert st["lowering"] == "gemm" and "t_X" in src.split("void t_r_kernel(")[1].split(")")[0]
        assert "a.r = t_X; a.r_sb = 131072LL; a.r_sm = 512;" in src and body in src, dt


def test_gemm_waves_knob():
    """16-bit GEMM stages with 256 x 256 tiles offer the schedule knob waves:
    4 (the default, kept as an absent knob) renders the one-wave-per-SIMD body
    with its hand-ordered main loop, 8 the two-waves-per-SIMD body. Smaller
    tiles and fp32 programs offer no such knob."""
    import run_mlp_search as RM
    from grammar import rewrites as R
    from grammar.hip_backend import schedule_knobs
    from grammar.kernel_ast import structural_key
    p = RM.build_mlp_silu(512, 256, 512, tile=256, dtype="fp16")
    p = R.merge(p, p.body[0], p.body[1])
    assert [schedule_knobs(s, p) for s in p.body] == [{"waves": ((4, 8), 4)}] * 2
    key0, src0 = structural_key(p), emit_module(p)
    steps = parse_plan(src0)["steps"]
    assert [s["block"] for s in steps] == [[256, 1, 1]] * 2 and [s["lds"] for s in steps] == [131072] * 2
    assert [s["tiles"]["waves"] for s in steps] == [4, 4]
    assert "gr_gemm_w4_body<_Float16, false, 2, 64, 256>(a, gr_gemm_smem);" in src0      # SiLU epilogue
    assert "gr_gemm_w4_body<_Float16, false, 0, 64, 256>(a, gr_gemm_smem);" in src0
    p.body[1].knobs["waves"] = 8
    assert structural_key(p) != key0
    src8 = emit_module(p)
    assert "gr_gemm_body<_Float16, 256, 256, 64, 2, 4, false, 0>(a, gr_gemm_smem);" in src8
    assert parse_plan(src8)["steps"][1]["block"] == [512, 1, 1]
    p.body[1].knobs.pop("waves")
    assert structural_key(p) == key0 and emit_module(p) == src0
    q = RM.build_mlp_silu(512, 256, 512, tile=128, dtype="fp16")
    q = R.merge(q, q.body[0], q.body[1])
    assert [schedule_knobs(s, q) for s in q.body] == [{}, {}]
    f = RM.build_mlp_ln(256, 512, 1024, tile=64)
    assert "waves" not in schedule_knobs(f.body[2], f)


def test_gemm_stage_with_a_part_filled_last_round_splits_its_columns():
    """A one-wave 256 x 256 GEMM stage whose last round of workgroups would
    leave more than half of the 256 CUs idle (X W1 of the C4 MLP: 1,376
    tiles, a sixth round of 96) renders two launches, as the library's
    gr_gemm does: the first 10,240 columns on 256 x 256 tiles, the last 768
    on 256 x 128 tiles with B, C (and R) offset by the first launch's
    columns. H W2 (512 tiles, two whole rounds) stays one launch."""
    import run_mlp_search as RM
    from grammar import rewrites as R
    from grammar import runtime as rt
    from grammar.hip_backend import _gemm_w4_split
    assert _gemm_w4_split(8192, 11008, 1) == (10240, 1280, 192)
    assert _gemm_w4_split(8192, 4096, 1) is None                 # 512 tiles: whole rounds
    assert _gemm_w4_split(8192, 11008, 2) is None                # batched launches stay whole
    assert _gemm_w4_split(4096, 4416, 1) == (4096, 256, 48)      # ragged tail: 320 columns
    p = RM.build_mlp_silu(8192, 4096, 11008, tile=256, subtile_k=64, dtype="fp16")
    p = R.merge(p, p.body[0], p.body[1])
    src = emit_module(p)
    steps = parse_plan(src)["steps"]
    assert [(s["kernel"], s["grid"][0], s["lds"], s.get("tail", False)) for s in steps] == [
        ("t_a_kernel", 1280, 131072, False), ("t_a_tail_kernel", 192, 98304, True), ("t_y_kernel", 512, 131072, False)]
    assert steps[1]["tiles"]["block_n"] == 128 and steps[1]["tiles"]["col0"] == 10240
    assert "a.M = 8192; a.N = 10240; a.K = 4096;" in src and "a.M = 8192; a.N = 768; a.K = 4096;" in src
    assert "a.b = t_W1 + 10240LL; a.c = t_a + 10240LL;" in src
    assert "gr_gemm_w4_body<_Float16, false, 2, 64, 128>(a, gr_gemm_smem);" in src
    code = rt.compile_source(src, "c4_split.hip")
    assert code[:4] == b"\x7fELF"


def test_fp32_gemm_split_k_knob():
    """fp32 GEMM stages offer the schedule knob ksplit: the K loop split over
    workgroups (grid z), the partials in a module-scope workspace, and a
    second launch that sums them and applies alpha, the activation and the
    residual. With no activation and only row-lowered readers of the same
    shape there is no second launch: the first part adds the residual and
    the reader sums the partials as it loads them. A split that does not
    divide K into whole k tiles keeps one part."""
    import run_mlp_search as RM
    from grammar import rewrites as R
    from grammar.hip_backend import schedule_knobs
    from grammar.kernel_ast import structural_key
    p = RM.build_mlp_ln(256, 512, 1024, tile=64)
    p = R.merge(p, p.body[2], p.body[3])
    r = p.body[2]
    assert r.out == "r" and schedule_knobs(r, p) == {"ksplit": ((1, 2, 4, 8), 1)}
    key0 = structural_key(p)
    r.knobs["ksplit"] = 4
    assert structural_key(p) != key0
    # r = a @ W2 + X, read only by the LayerNorm rows: the sum moves into the reader
    src = emit_module(p)
    steps = [s for s in parse_plan(src)["steps"] if s["kernel"].startswith("t_r_")]
    assert [s["kernel"] for s in steps] == ["t_r_kernel"] and steps[0]["tiles"]["sum_in_consumer"]
    assert steps[0]["grid"] == [(256 // 64) * (512 // 64), 1, 4] and steps[0]["tiles"]["ksplit"] == 4
    body = src.split("void t_r_kernel(")[1].split("}\n")[0]
    assert "if (blockIdx.z != 0) a.r = nullptr;" in body and "gr_gemm_f32_body<64, 64, 32" in body
    assert body.rstrip().endswith("4>(a, gr_gemm_smem);")         # the residual epilogue, no activation
    assert "__device__ float gr_ws_t_r[524288];" in src and "gr_gemm_f32_reduce_body" not in src
    reader = src.split("void t_out_kernel(")[1]
    assert "gr_row_load_parts<" in reader and "gr_ws_t_r + " in reader and "131072LL, 4)" in reader
    r.knobs["ksplit"] = 8                       # 1024 / 8 = 128: whole 32-deep k tiles
    assert [s for s in parse_plan(emit_module(p))["steps"] if s["kernel"] == "t_r_kernel"][0]["tiles"]["ksplit"] == 8
    # a = relu(X @ W1): an activation keeps the second launch
    q = RM.build_mlp_ln(256, 512, 1024, tile=64)
    q = R.merge(q, q.body[0], q.body[1])
    q.body[0].knobs["ksplit"] = 4
    src = emit_module(q)
    steps = [s for s in parse_plan(src)["steps"] if s["kernel"].startswith("t_a_")]
    assert [s["kernel"] for s in steps] == ["t_a_kernel", "t_a_reduce_kernel"]
    assert steps[1]["merge"] and steps[1]["grid"] == [256 * 1024 // 4 // 256, 1, 1]
    assert "__device__ float gr_ws_t_a[1048576];" in src and "gr_gemm_f32_reduce_body<1>(a, gr_ws_t_a, 4" in src
    p16 = RM.build_mlp_ln(256, 512, 1024, tile=64, dtype="fp16")
    assert schedule_knobs(p16.body[2], p16) == {}   # fp16 GEMMs take no split
