"""GPU parity of grammar programs rendered to HIP and run through the C ABI.

fp32 programs: the rendered module's output must match the numpy tile
interpreter on the same inputs (the reference's own bar, rtol = atol = 1e-3,
test_renderer.py:222-223, 287) and every intermediate/output must be fully
written (NaN-filled allocation). fp16/bf16 attention programs (flash
lowering): max-abs <= 2e-2, mean-abs <= 2e-3 against the fp32 oracle on the
rounded inputs."""
import numpy as np
import pytest

import grammar_cases as C
from grammar import rewrites as R
from grammar.kernel_ast import emit_module, kernel_meta, Compute, ReductionLoop, Load
from oracle import attention as O
from oracle.grammar_interp import run_program

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def _cuda():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _gpu_run(prog, ins):
    from grammar.hip_module import load_module
    mod = load_module(emit_module(prog))
    args = [torch.from_numpy(ins[n]).to(_cuda()).to(mod.dtype) for n in mod.inputs]
    out = mod.fn(*args)
    torch.cuda.synchronize()
    return out.float().cpu().numpy(), mod


@pytest.mark.parametrize("name", list(C.REFS))
def test_rendered_case_matches_interpreter(name):
    build, ref = C.REFS[name]
    prog = build()
    ins = C.inputs_for(prog, 0)
    got, mod = _gpu_run(prog, ins)
    want = run_program(prog, ins)[kernel_meta(prog)["output"][0]]
    print(f"[renderer] {name}: lowering {[s['lowering'] for s in mod.plan['steps']]} "
          f"max|d| {float(np.max(np.abs(got - want))):.2e}", flush=True)
    assert np.all(np.isfinite(got)), "NaN/Inf: incomplete write"
    assert np.allclose(got, want, rtol=1e-3, atol=1e-3)
    assert np.allclose(got, ref(ins), rtol=1e-3, atol=1e-3)


def test_rewrites_preserve_results_on_gpu():
    p = C.p_matmul_reduction()
    ins = C.inputs_for(p, 0)
    gemm_out, mod = _gpu_run(p, ins)                  # fp32 matmul stage: the fp32 MFMA GEMM
    assert [s["lowering"] for s in mod.plan["steps"]] == ["gemm"]
    for l in p.body:                                  # the same program on the generic lowering
        l.knobs["lowering"] = "generic"
    base, mod = _gpu_run(p, ins)
    assert [s["lowering"] for s in mod.plan["steps"]] == ["generic"]
    assert np.allclose(gemm_out, base, rtol=1e-3, atol=1e-3)
    h = p
    for src in ("x", "y"):
        ld = [s for l in h.body for s in R.statements(l.body) if isinstance(s, Load) and s.source == src][0]
        h = R.hoist(h, ld)
    assert "GR_SUBTILE" in emit_module(h)
    assert np.allclose(_gpu_run(h, ins)[0], base, rtol=1e-3, atol=1e-3)
    t = C.p_attention()
    ti = C.inputs_for(t, 0)
    r0, _ = _gpu_run(t, ti)
    q = R.merge(t, t.body[0], t.body[1])
    q = R.fuse_softmax(q, q.body[0], q.body[1])
    smm = next(s for s in q.body[0].body if isinstance(s, Compute) and s.op == "softmax_matmul")
    q = R.subtile_reduction(q, smm, "j", tile=32)
    assert np.allclose(_gpu_run(q, ti)[0], r0, rtol=1e-3, atol=1e-3)


FLASH = [
    # B, H, N, d, bm, bn, causal, dtype
    (2, 2, 256, 64, 128, 64, False, "fp16"),
    (2, 2, 256, 64, 64, 32, True, "fp16"),
    (1, 4, 512, 64, 256, 64, False, "bf16"),
    (1, 2, 256, 128, 128, 64, True, "bf16"),
    (1, 2, 256, 64, 32, 128, False, "fp16"),
    # schedule knobs (descent parameters SCHED_O.pipe / SCHED_O.qb)
    (1, 4, 512, 64, 256, 128, False, "fp16", {"pipe": 1}),
    (1, 4, 512, 64, 256, 64, False, "fp16", {"qb": 2, "w2": 0}),
    (1, 4, 512, 64, 256, 64, True, "bf16", {"qb": 2, "pipe": 1}),
    (1, 2, 256, 128, 128, 64, True, "bf16", {"pipe": 1}),
    (2, 2, 256, 64, 128, 128, False, "bf16", {"qb": 2}),
    # scale 1 in fp16: no Q pre-scale (scale * log2(e) > 1)
    (1, 2, 256, 64, 128, 64, True, "fp16", {}, 1.0),
    # fp16 d 64 non-causal 256 x 64: the two-waves-per-SIMD body (knob w2, on
    # by default); 40 tiles leave seven steps after the groups of eight
    (1, 4, 512, 64, 256, 64, False, "fp16"),
    (2, 2, 1024, 64, 256, 64, False, "fp16", {"w2": 1}),
    (1, 2, 2560, 64, 256, 64, False, "fp16"),
    # head dim 128 at 256 x 64: the d = 128 two-wave body (gr_flash_w2h.h),
    # causal or not; off (w2 0), the flash body
    (1, 2, 256, 128, 256, 64, True, "bf16"),
    (2, 4, 1024, 128, 256, 64, True, "bf16"),
    (1, 2, 512, 128, 256, 64, False, "fp16"),
    (1, 2, 768, 128, 256, 64, True, "fp16"),
    (1, 2, 512, 128, 256, 64, True, "bf16", {"w2": 0}),
]


@pytest.mark.parametrize("case", FLASH, ids=lambda c: "-".join(map(str, c)))
def test_flash_lowered_program_parity(case):
    dev = _cuda()
    from grammar.hip_module import load_module
    from grammar.workloads import AttnConfig, attention_inputs
    B, H, N, d, bm, bn, causal, dt = case[:8]
    knobs = case[8] if len(case) > 8 else {}
    scale = case[9] if len(case) > 9 else 1.0 / d ** 0.5
    prog = C.p_flash_attention(B=B, H=H, N=N, d=d, bm=bm, bn=bn, causal=causal, scale=scale, dtype=dt)
    prog.body[0].knobs.update(knobs)
    print(f"[case] flash-lowered {case}", flush=True)
    mod = load_module(emit_module(prog))
    assert [s["lowering"] for s in mod.plan["steps"]] == ["flash"]
    tiles = mod.plan["steps"][0]["tiles"]
    w2 = (bm, bn) == (256, 64) and N % 256 == 0 and knobs.get("w2", 1) == 1 and (
        (dt == "fp16" and d == 64 and not causal and scale * 1.4426950408889634 <= 1.0) or d == 128)
    assert tiles.get("w2", 0) == int(w2)
    if not w2:
        assert tiles["qb"] == knobs.get("qb", 1) and tiles["pipe"] == knobs.get("pipe", 0)
    q, kt, v = attention_inputs(AttnConfig("t", B, H, N, d, dt, causal), seed=3, k_transposed=True)
    o = mod.fn(kt.to(dev), q.to(dev), v.to(dev))          # sorted input names: KT, Q, V
    torch.cuda.synchronize()
    ref = O.attention(q.float().numpy(), kt.float().numpy(), v.float().numpy(), causal=causal, k_transposed=True,
                      scale=scale)
    mx, mn = O.errors(o.float().cpu().numpy(), ref)
    print(f"[flash-lowered] {case}: max-abs {mx:.2e} mean-abs {mn:.2e}", flush=True)
    assert mx <= O.MAX_ABS_TOL and mn <= O.MEAN_ABS_TOL


FLASH32 = [
    # B, H, N, d, bm, bn: fp32 flash stage (gr_flash_f32.h): bm / 32 waves per
    # workgroup, bn keys per wave, N / (bm / 32 * bn) workgroups per query block
    (1, 1, 512, 64, 128, 32),      # the reference's own workload: 4 parts
    (1, 1, 512, 64, 128, 128),     # one workgroup per query block: no workspace
    (1, 1, 512, 64, 32, 32),       # 16 parts of one wave each
    (2, 3, 256, 64, 64, 64),
    (1, 2, 256, 128, 256, 32),     # 8 waves, d = 128
    (4, 1, 128, 64, 32, 128),
]


@pytest.mark.parametrize("case", FLASH32, ids=lambda c: "-".join(map(str, c)))
def test_fp32_flash_stage_parity_and_relaunch(case):
    """fp32 attention as one flash stage on the fp32 matrix cores, its keys
    split over the waves of a workgroup and, with several workgroups per
    query block, over workgroups whose partials a second launch merges --
    three launches on new and on repeated inputs agree with the fp64 closed
    form at fp32 tolerance (and repeat bit for bit)."""
    dev = _cuda()
    from grammar.hip_module import load_module
    B, H, N, d, bm, bn = case
    prog = C.p_flash_attention(B=B, H=H, N=N, d=d, bm=bm, bn=bn, dtype="fp32")
    print(f"[case] fp32 flash {case}", flush=True)
    mod = load_module(emit_module(prog))
    parts = N // (bm // 32 * bn)
    assert mod.plan["steps"][0]["tiles"]["parts"] == parts
    # with several workgroups per query block a second launch merges their partials
    assert [s["lowering"] for s in mod.plan["steps"]] == ["flash"] * (1 if parts == 1 else 2)
    g = torch.Generator("cpu").manual_seed(5)
    for rep in range(3):
        q = torch.randn((B, H, N, d), generator=g)
        kt = torch.randn((B, H, d, N), generator=g)
        v = torch.randn((B, H, N, d), generator=g)
        if rep == 2:
            q, kt, v = prev
        o = mod.fn(kt.to(dev), q.to(dev), v.to(dev))
        torch.cuda.synchronize()
        ref = O.attention(q.double().numpy(), kt.double().numpy(), v.double().numpy(), k_transposed=True,
                          scale=1.0 / d ** 0.5)
        err = float(np.max(np.abs(o.cpu().numpy() - ref)))
        print(f"[flash32] {case} launch {rep}: max-abs {err:.2e}", flush=True)
        assert err <= 1e-3
        if rep == 0:
            prev, first = (q, kt, v), o.clone()
        if rep == 2:
            assert torch.equal(o, first)      # the same inputs give the same bits on a later launch


def test_generic_fp16_attention_matches_rounded_interpreter():
    dev = _cuda()
    from grammar.hip_module import load_module
    prog = C.p_attention()
    prog.dtype = "fp16"
    ins = C.inputs_for(prog, 0)
    rnd = lambda x: np.asarray(x, dtype=np.float16).astype(np.float32)
    ins16 = {k: rnd(v) for k, v in ins.items()}
    mod = load_module(emit_module(prog))
    out = mod.fn(*[torch.from_numpy(ins16[n]).to(dev).half() for n in mod.inputs]).float().cpu().numpy()
    want = run_program(prog, ins16, storage_round=rnd)["O"]
    assert np.allclose(out, want, rtol=2e-3, atol=2e-3)


def test_gemm_lowered_attention_stages():
    """The atomic attention program at fp16: its two matmul stages lower to the
    MFMA GEMM (S with K given transposed as [d, N], O with V as [N, d]); the
    softmax stages stay generic. Output against the fp32 oracle."""
    dev = _cuda()
    from grammar.hip_module import load_module
    from grammar.workloads import AttnConfig, attention_inputs
    import run_attention_search as RS
    prog = RS.build_attention(256, 64, tile=64, B=2, H=2, dtype="fp16")
    mod = load_module(emit_module(prog))
    low = {s["kernel"]: s["lowering"] for s in mod.plan["steps"]}
    print(f"[gemm-lowered] attention stages {low}", flush=True)
    assert low["t_S_kernel"] == "gemm" and low["t_O_kernel"] == "gemm"
    q, kt, v = attention_inputs(AttnConfig("t", 2, 2, 256, 64, "fp16", False), seed=4, k_transposed=True)
    o = mod.fn(kt.to(dev), q.to(dev), v.to(dev))
    torch.cuda.synchronize()
    ref = O.attention(q.float().numpy(), kt.float().numpy(), v.float().numpy(), k_transposed=True)
    mx, mn = O.errors(o.float().cpu().numpy(), ref)
    print(f"[gemm-lowered] attention: max-abs {mx:.2e} mean-abs {mn:.2e}", flush=True)
    assert mx <= O.MAX_ABS_TOL and mn <= O.MEAN_ABS_TOL


@pytest.mark.parametrize("dt", ["fp16", "bf16"])
def test_gemm_lowered_mlp_program(dt):
    """Y = SiLU(X W1) W2 from the grammar: after merge(h, a) both stages lower
    to the GEMM, the first with its SiLU epilogue."""
    dev = _cuda()
    from grammar.hip_module import load_module
    import run_mlp_search as RM
    prog = RM.build_mlp_silu(256, 128, 256, tile=128, subtile_k=64, dtype=dt)
    prog = R.merge(prog, prog.body[0], prog.body[1])
    mod = load_module(emit_module(prog))
    assert [s["lowering"] for s in mod.plan["steps"]] == ["gemm", "gemm"]
    ins = RM.mlp_inputs(256, 128, 256, dt, seed=2, device=str(dev))
    y = mod.fn(*[ins[n] for n in mod.inputs])
    torch.cuda.synchronize()
    ref = O.mlp_silu(ins["X"].float().cpu().numpy(), ins["W1"].float().cpu().numpy(),
                     ins["W2"].float().cpu().numpy(), dtype=np.float64)
    mx, mn = O.errors(y.float().cpu().numpy(), ref)
    print(f"[gemm-lowered] mlp {dt}: max-abs {mx:.2e} mean-abs {mn:.2e}", flush=True)
    assert mx <= O.MAX_ABS_TOL and mn <= O.MEAN_ABS_TOL
    assert np.allclose(RM.verify(prog, "silu"), True)


def test_gemm_lowered_batched_with_shared_weight():
    """A batched [2, 128, 64] operand against one [64, 128] weight (batch
    stride 0), with a mulc + relu epilogue."""
    dev = _cuda()
    from grammar.hip_module import load_module
    from grammar.kernel_ast import Program, ParallelLoop, Store
    A, W = Load("A", ["b", "i", "k"]), Load("W", ["k", "j"])
    mm = Compute("matmul", [A, W])
    sc = Compute("mulc", [mm], const=0.5)
    rl = Compute("relu", [sc])
    prog = Program({"A": (2, 128, 64), "W": (64, 128), "C": (2, 128, 128)},
                   [ParallelLoop("C", (1, 128, 128), ("b", "i", "j"), [A, W, mm, sc, rl, Store("C", rl, ["b", "i", "j"])])],
                   "fp16")
    mod = load_module(emit_module(prog))
    assert [s["lowering"] for s in mod.plan["steps"]] == ["gemm"]
    g = torch.Generator("cpu").manual_seed(9)
    a = torch.randn((2, 128, 64), generator=g).half()
    w = (torch.randn((64, 128), generator=g) / 8).half()
    c = mod.fn(a.to(dev), w.to(dev))
    torch.cuda.synchronize()
    ref = np.maximum(0.5 * (a.double().numpy() @ w.double().numpy()), 0.0)
    mx, mn = O.errors(c.float().cpu().numpy(), ref)
    assert mx <= O.MAX_ABS_TOL and mn <= O.MEAN_ABS_TOL


@pytest.mark.parametrize("dt,causal", [("fp16", False), ("bf16", True)])
def test_fuse_attention_from_atomic_program_runs_flash(dt, causal):
    """The atomic 8/9-stage attention, fused by fuse_attention into one stage
    (scores over the full key range, no key loop), renders to the flash
    kernel and matches the fp32 oracle."""
    dev = _cuda()
    from grammar.hip_module import load_module
    from grammar.workloads import AttnConfig, attention_inputs
    import run_attention_search as RS
    p = RS.build_attention(512, 64, tile=128, B=2, H=2, dtype=dt, causal=causal)
    q = R.fuse_softmax_chain(p, p.body[-1], with_scores=True)
    mod = load_module(emit_module(q))
    assert [s["lowering"] for s in mod.plan["steps"]] == ["flash"]
    qq, kt, v = attention_inputs(AttnConfig("t", 2, 2, 512, 64, dt, causal), seed=6, k_transposed=True)
    o = mod.fn(kt.to(dev), qq.to(dev), v.to(dev))
    torch.cuda.synchronize()
    ref = O.attention(qq.float().numpy(), kt.float().numpy(), v.float().numpy(), causal=causal, k_transposed=True)
    mx, mn = O.errors(o.float().cpu().numpy(), ref)
    print(f"[fuse_attention] {dt} causal={causal}: max-abs {mx:.2e} mean-abs {mn:.2e}", flush=True)
    assert mx <= O.MAX_ABS_TOL and mn <= O.MEAN_ABS_TOL


@pytest.mark.parametrize("tile,sk", [(32, 32), (32, None), (16, 64)])
def test_ln_mlp_block_on_gpu(tile, sk):
    """The reference's MLP block (relu + residual + LayerNorm,
    run_mlp_search.py:42-127) rendered to HIP (fp32, generic lowering) matches
    the closed form (run_mlp_search.py:138-149) at the reference's tolerance."""
    _cuda()
    import run_mlp_search as RM
    p = RM.build_mlp_ln(256, 256, 512, tile=tile, subtile_k=sk)
    assert RM.verify(p, "ln")
    ins = {k: v.cpu().numpy() for k, v in RM.mlp_inputs(256, 256, 512, "fp32", seed=3).items()}
    got, mod = _gpu_run(p, ins)
    want = run_program(p, ins)["out"]
    print(f"[ln-block] tile={tile} sk={sk}: max|d| {float(np.max(np.abs(got - want))):.2e}", flush=True)
    assert np.allclose(got, want, rtol=1e-3, atol=1e-3)


@pytest.mark.parametrize("dt", ["fp32", "fp16", "bf16"])
def test_residual_add_fuses_into_the_gemm(dt):
    """The LN block with its second matmul and the residual add merged into one
    stage (r = a @ W2 + X) and the first with its relu (a = relu(X @ W1)):
    both lower to the GEMM, the residual read in its epilogue (GR_EPI_RES)
    and added in fp32 before the output is rounded. Against the tile
    interpreter on the same (rounded) inputs."""
    _cuda()
    import run_mlp_search as RM
    from grammar import rewrites as R
    from grammar.hip_module import load_module
    p = RM.build_mlp_ln(256, 256, 512, tile=64, dtype=dt)
    p = R.merge(p, p.body[2], p.body[3])
    p = R.merge(p, p.body[0], p.body[1])
    mod = load_module(emit_module(p))
    assert [s["lowering"] for s in mod.plan["steps"]] == ["gemm", "gemm", "rows"]
    ins = {k: v.float().cpu().numpy() for k, v in RM.mlp_inputs(256, 256, 512, dt, seed=3).items()}
    args = [torch.from_numpy(ins[n]).to(_cuda()).to(mod.dtype) for n in mod.inputs]
    tensors = mod.run_with(args)
    torch.cuda.synchronize()
    if dt == "fp32":
        want = run_program(p, ins)
        tol = 1e-3
    else:
        rnd = (lambda x: np.asarray(x, dtype=np.float16).astype(np.float32)) if dt == "fp16" else \
            (lambda x: torch.from_numpy(np.asarray(x, dtype=np.float32)).bfloat16().float().numpy())
        want = run_program(p, ins, storage_round=rnd)
        tol = 2e-2 if dt == "bf16" else 5e-3
    for name in ("r", "out"):
        got = tensors[name].float().cpu().numpy()
        err = float(np.max(np.abs(got - want[name])))
        print(f"[residual-gemm] {dt} {name}: max|d| {err:.2e}", flush=True)
        assert np.isfinite(got).all() and err <= tol * max(1.0, float(np.max(np.abs(want[name]))))


@pytest.mark.parametrize("dt", ["fp16", "bf16"])
def test_gemm_waves_knob_schedules_agree(dt):
    """The LN block's two GEMM stages (a = relu(X @ W1), r = a @ W2 + X) at
    256 x 256 tiles under both values of the schedule knob waves: the
    one-wave-per-SIMD body (4, the default) and the two-waves-per-SIMD body
    (8) accumulate every output in the same k order, so r and out agree bit
    for bit; both against the tile interpreter on the same rounded inputs."""
    _cuda()
    import run_mlp_search as RM
    from grammar import rewrites as R
    from grammar.hip_module import load_module
    M, Dm, H = 512, 256, 512
    p = RM.build_mlp_ln(M, Dm, H, tile=256, dtype=dt)
    p = R.merge(p, p.body[2], p.body[3])
    p = R.merge(p, p.body[0], p.body[1])
    ins = {k: v.float().cpu().numpy() for k, v in RM.mlp_inputs(M, Dm, H, dt, seed=5).items()}
    rnd = (lambda x: np.asarray(x, dtype=np.float16).astype(np.float32)) if dt == "fp16" else \
        (lambda x: torch.from_numpy(np.asarray(x, dtype=np.float32)).bfloat16().float().numpy())
    want = run_program(p, ins, storage_round=rnd)
    tol = 2e-2 if dt == "bf16" else 5e-3
    runs = {}
    for waves in (4, 8):
        for st in p.body[:2]:
            st.knobs.pop("waves", None)
            if waves != 4:
                st.knobs["waves"] = waves
        mod = load_module(emit_module(p))
        gemm_steps = [s for s in mod.plan["steps"] if s["lowering"] == "gemm"]
        assert [s["block"][0] for s in gemm_steps] == [256 if waves == 4 else 512] * 2
        print(f"[case] LN block {dt} M={M} Dm={Dm} H={H} waves={waves}", flush=True)
        args = [torch.from_numpy(ins[n]).to(_cuda()).to(mod.dtype) for n in mod.inputs]
        tensors = mod.run_with(args)
        torch.cuda.synchronize()
        runs[waves] = {n: tensors[n].float().cpu().numpy() for n in ("r", "out")}
        for name in ("r", "out"):
            got = runs[waves][name]
            err = float(np.max(np.abs(got - want[name])))
            print(f"[waves] {dt} waves={waves} {name}: max|d| {err:.2e}", flush=True)
            assert np.isfinite(got).all() and err <= tol * max(1.0, float(np.max(np.abs(want[name]))))
    for name in ("r", "out"):
        assert np.array_equal(runs[4][name], runs[8][name]), name


@pytest.mark.parametrize("dt,H", [("fp16", 4352), ("bf16", 4416)])
def test_gemm_stage_split_into_two_launches(dt, H):
    """Y = SiLU(X W1) W2 with X W1 at 4096 x H x 128 on 256 x 256 tiles: a
    second round of 16 or 18 workgroups, so the stage renders two launches
    (the first 4,096 columns on 256 x 256 tiles, the rest on 256 x 128; at
    H = 4,416 the last of those is ragged). The intermediate a and Y against
    the float64 closed form on the same rounded inputs."""
    dev = _cuda()
    import run_mlp_search as RM
    from grammar import rewrites as R
    from grammar.hip_module import load_module
    M, Dm = 4096, 128
    p = RM.build_mlp_silu(M, Dm, H, tile=256, subtile_k=64, dtype=dt)
    p = R.merge(p, p.body[0], p.body[1])
    mod = load_module(emit_module(p))
    steps = [(s["kernel"], s["grid"][0]) for s in mod.plan["steps"]]
    assert steps[:2] == [("t_a_kernel", 256), ("t_a_tail_kernel", 16 * ((H - 4096 + 127) // 128))], steps
    print(f"[case] split GEMM stage {dt} M={M} Dm={Dm} H={H}: {steps}", flush=True)
    ins = RM.mlp_inputs(M, Dm, H, dt, seed=3, device=str(dev))
    tensors = mod.run_with([ins[n] for n in mod.inputs])
    torch.cuda.synchronize()
    x, w1, w2 = (ins[n].double().cpu().numpy() for n in ("X", "W1", "W2"))
    a_ref = O.silu(x @ w1)
    mx, mn = O.errors(tensors["a"].float().cpu().numpy(), a_ref)
    print(f"[split] {dt} a: max-abs {mx:.2e} mean-abs {mn:.2e}", flush=True)
    assert mx <= O.MAX_ABS_TOL and mn <= O.MEAN_ABS_TOL
    tail = tensors["a"][:, 4096:].float().cpu().numpy()
    assert np.isfinite(tail).all() and float(np.abs(tail - a_ref[:, 4096:]).max()) <= O.MAX_ABS_TOL
    ref = O.mlp_silu(x, w1, w2, dtype=np.float64)
    mx, mn = O.errors(tensors["y"].float().cpu().numpy(), ref)
    print(f"[split] {dt} y: max-abs {mx:.2e} mean-abs {mn:.2e}", flush=True)
    assert mx <= O.MAX_ABS_TOL and mn <= O.MEAN_ABS_TOL


@pytest.mark.parametrize("ks_a,ks_r", [(2, 4), (8, 8), (4, 1)])
def test_fp32_split_k_gemm_stages(ks_a, ks_r):
    """fp32 GEMM stages with K split over workgroups (schedule knob ksplit):
    the ReLU stage (two launches: the sum applies the activation) and the
    residual stage of the merged LN block against the tile interpreter; two
    runs of the bound plan give the same bits. The residual stage, read only
    by the LayerNorm rows, leaves its sum to them: r is then not materialised
    and the output carries its check."""
    _cuda()
    import run_mlp_search as RM
    from grammar import rewrites as R
    from grammar.hip_module import load_module
    p = RM.build_mlp_ln(256, 256, 512, tile=64)
    p = R.merge(p, p.body[2], p.body[3])
    p = R.merge(p, p.body[0], p.body[1])
    p.body[0].knobs["ksplit"] = ks_a
    p.body[1].knobs["ksplit"] = ks_r
    mod = load_module(emit_module(p))
    tiles = [s.get("tiles", {}).get("ksplit", 1) for s in mod.plan["steps"] if not s.get("merge")]
    assert tiles[:2] == [ks_a, ks_r], tiles
    ins = {k: v.cpu().numpy() for k, v in RM.mlp_inputs(256, 256, 512, "fp32", seed=4).items()}
    args = [torch.from_numpy(ins[n]).to(_cuda()) for n in mod.inputs]
    tensors = {n: t for n, t in zip(mod.inputs, args)}
    tensors.update(mod.allocate(args[0].device))
    plan = mod.bind(tensors)
    plan.run()
    torch.cuda.synchronize()
    summed_by_reader = [s for s in mod.plan["steps"] if s.get("tiles", {}).get("sum_in_consumer")]
    assert [s["kernel"] for s in summed_by_reader] == (["t_r_kernel"] if ks_r > 1 else [])
    names = ("a", "out") if ks_r > 1 else ("a", "r", "out")
    first = {n: tensors[n].clone() for n in names}
    plan.run()
    torch.cuda.synchronize()
    want = run_program(p, ins)
    for name in names:
        got = tensors[name].cpu().numpy()
        err = float(np.max(np.abs(got - want[name])))
        print(f"[split-k] ksplit {ks_a}/{ks_r} {name}: max|d| {err:.2e}", flush=True)
        assert err <= 1e-3 * max(1.0, float(np.max(np.abs(want[name]))))
        assert torch.equal(tensors[name], first[name])


@pytest.mark.parametrize("dt,causal,merges", [("fp16", False, 0), ("bf16", True, 0), ("fp16", False, 3)])
def test_row_lowered_softmax_stages(dt, causal, merges):
    """The softmax stages of the atomic attention program (scale, causal
    mask, row max, subtract/exp, row sum, divide) lower to one-wave-per-row
    kernels; after merges that gather them, the fused row stage computes
    exp(x - rowmax x) / rowsum(...) in passes over the row. Output against the
    fp32 oracle."""
    dev = _cuda()
    from grammar.hip_module import load_module
    from grammar.workloads import AttnConfig, attention_inputs
    import run_attention_search as RS
    p = RS.build_attention(512, 64, tile=64, B=2, H=2, dtype=dt, causal=causal)
    for l in p.body[1:-1]:
        l.tile_shape = (1, 1, 64, 512)        # full rows, so merged stages keep one tile per value
    for _ in range(merges):
        names = [l.out for l in p.body]
        i = names.index("sm") if "sm" in names else names.index("P") - 1
        a = p.body[i]
        b = p.body[i + 1]
        if not R.can_merge(p, a, b)[0]:
            break
        p = R.merge(p, a, b)
    mod = load_module(emit_module(p))
    low = [s["lowering"] for s in mod.plan["steps"]]
    print(f"[rows] {dt} causal={causal} merges={merges}: {[l.out for l in p.body]} {low}", flush=True)
    assert low[0] == "gemm" and low[-1] == "gemm" and all(x == "rows" for x in low[1:-1])
    q, kt, v = attention_inputs(AttnConfig("t", 2, 2, 512, 64, dt, causal), seed=8, k_transposed=True)
    o = mod.fn(kt.to(dev), q.to(dev), v.to(dev))
    torch.cuda.synchronize()
    ref = O.attention(q.float().numpy(), kt.float().numpy(), v.float().numpy(), causal=causal, k_transposed=True)
    mx, mn = O.errors(o.float().cpu().numpy(), ref)
    print(f"[rows] max-abs {mx:.2e} mean-abs {mn:.2e}", flush=True)
    assert mx <= O.MAX_ABS_TOL and mn <= O.MEAN_ABS_TOL


def test_kernel_handle_keeps_its_module_loaded():
    """A kernel looked up on a temporary Module stays launchable: the handle
    (and a Plan built from it) keeps the code object loaded."""
    import gc
    from grammar import runtime as rt
    dev = _cuda()
    code = rt.compile_source('extern "C" __global__ void fill(float* x, float v) { x[threadIdx.x] = v; }\n',
                             "fill.hip")
    kern = rt.Module(code).kernel("fill")
    gc.collect()
    x = torch.zeros(64, device=dev)
    import struct
    plan = rt.Plan([(kern, (1, 1, 1), (64, 1, 1), 0, [x.data_ptr(), struct.unpack("<I", struct.pack("<f", 2.5))[0]])])
    del kern
    gc.collect()
    plan.run()
    torch.cuda.synchronize()
    assert torch.all(x == 2.5)
