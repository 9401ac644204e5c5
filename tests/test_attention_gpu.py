"""GPU parity of the hand-written CDNA4 attention forward (gr_attn_fwd) against
the fp32 CPU oracle, on the same seeded inputs.

Bar: max-abs <= 2e-2 and mean-abs <= 2e-3 against
softmax(QK^T/sqrt(d))V computed in fp32 on the CPU from the fp16/bf16-rounded
inputs. Full-size configs add size-independent properties (finiteness,
convex hull of V, bitwise layout/stride invariance, determinism)."""
import math

import numpy as np
import pytest

from oracle import attention as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _cuda():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _run(q, k, v, **kw):
    from grammar.attention import flash_attention_fwd
    o = flash_attention_fwd(q, k, v, **kw)
    torch.cuda.synchronize()
    return o


def _check(o_gpu, ref, label):
    got = o_gpu.float().cpu().numpy()
    mx, mn = O.errors(got, ref)
    print(f"[parity] {label}: max-abs {mx:.3e} mean-abs {mn:.3e}", flush=True)
    assert np.isfinite(got).all(), label
    assert mx <= O.MAX_ABS_TOL and mn <= O.MEAN_ABS_TOL, (label, mx, mn)
    return mx, mn


def test_mfma32_layout_selftest():
    dev = _cuda()
    from grammar.attention import mfma32_selftest
    g = torch.Generator("cpu").manual_seed(3)
    a = torch.randn(32, 16, generator=g).half()
    b = torch.randn(16, 32, generator=g).half()
    d = mfma32_selftest(a.to(dev), b.to(dev)).cpu()
    ref = a.double() @ b.double()
    assert torch.allclose(d.double(), ref, atol=1e-3, rtol=1e-3), (d - ref).abs().max()


SMALL = [
    # B, H, N, D, dtype, causal, k_transposed, block_m, block_n
    (1, 2, 256, 64, "fp16", False, False, 128, 64),
    (1, 2, 256, 64, "bf16", False, False, 128, 64),
    (1, 2, 256, 64, "fp16", True, False, 128, 64),
    (1, 2, 256, 64, "fp16", False, True, 128, 64),
    (1, 2, 256, 64, "bf16", True, True, 128, 64),
    (2, 3, 256, 128, "fp16", False, False, 128, 64),
    (2, 3, 256, 128, "bf16", True, False, 128, 64),
    (1, 2, 512, 64, "fp16", False, False, 128, 32),
    (1, 2, 512, 64, "fp16", True, False, 128, 128),
    (1, 2, 512, 64, "bf16", False, False, 128, 128),
    (1, 2, 512, 64, "fp16", False, False, 64, 64),
    (1, 2, 512, 64, "fp16", True, False, 256, 64),
    (1, 2, 512, 64, "bf16", False, True, 256, 32),
    (1, 2, 512, 64, "fp16", False, True, 256, 128),
    (1, 2, 512, 64, "bf16", True, True, 256, 128),
    (2, 3, 512, 128, "fp16", False, True, 256, 64),
    (1, 2, 512, 128, "bf16", True, False, 256, 32),
    (1, 2, 256, 64, "fp16", True, True, 64, 32),
    (1, 2, 384, 64, "fp16", False, False, 0, 0),
    (1, 2, 320, 128, "bf16", True, True, 0, 0),
    (1, 2, 512, 128, "bf16", True, True, 128, 32),
    (1, 1, 128, 64, "fp16", True, False, 128, 64),
    # block_m 129 / 257: the software-pipelined schedule (next tile's scores
    # interleaved with this tile's softmax), 128 / 256 queries per workgroup
    (1, 2, 512, 64, "fp16", False, True, 129, 64),
    (1, 2, 512, 64, "bf16", True, False, 129, 128),
    (1, 2, 512, 64, "fp16", True, True, 257, 64),
    (1, 2, 512, 64, "bf16", False, False, 257, 32),
    (1, 2, 512, 128, "fp16", True, True, 129, 32),
    (1, 2, 512, 128, "bf16", False, True, 257, 64),
    (1, 1, 128, 64, "fp16", False, False, 129, 128),
    # fp16 d 64 non-causal 256 x 64: the two-waves-per-SIMD body (gr_flash_w2.h),
    # from the fewest tiles (4) to 36 and 40 tiles (three and seven steps after
    # the groups of eight)
    (1, 2, 256, 64, "fp16", False, False, 256, 64),
    (1, 2, 512, 64, "fp16", False, True, 256, 64),
    (2, 3, 1024, 64, "fp16", False, False, 256, 64),
    (1, 2, 2304, 64, "fp16", False, True, 256, 64),
    (1, 1, 2560, 64, "fp16", False, False, 256, 64),
    # d 128, K^T, 256 x 64: the d = 128 two-wave body (gr_flash_w2h.h), causal
    # (the diagonal block alone at N 256) or not; 6 heads take the grid-wide
    # causal order, 8 the per-XCD one
    (1, 2, 256, 128, "bf16", True, True, 256, 64),
    (1, 2, 256, 128, "fp16", False, True, 256, 64),
    (1, 2, 512, 128, "bf16", True, True, 256, 64),
    (2, 3, 1024, 128, "fp16", True, True, 256, 64),
    (1, 8, 1024, 128, "bf16", True, True, 256, 64),
    (1, 2, 2304, 128, "bf16", False, True, 256, 64),
    (1, 1, 1280, 128, "fp16", True, True, 0, 0),
]


@pytest.mark.parametrize("case", SMALL, ids=lambda c: "-".join(map(str, c)))
def test_attention_small_parity(case):
    dev = _cuda()
    from grammar.workloads import AttnConfig, attention_inputs
    B, H, N, D, dt, causal, kt, bm, bn = case
    cfg = AttnConfig("t", B, H, N, D, dt, causal)
    q, k, v = attention_inputs(cfg, seed=11, k_transposed=kt)
    ref = O.attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), causal=causal, k_transposed=kt)
    o = _run(q.to(dev), k.to(dev), v.to(dev), causal=causal, k_transposed=kt, block_m=bm, block_n=bn)
    _check(o, ref, str(case))


def test_c1_shape_fp16():
    # C1 is the CPU plumbing config (fp32); its shape also runs on the GPU in fp16.
    dev = _cuda()
    from grammar.workloads import C1, attention_inputs
    q, k, v = attention_inputs(C1, seed=0, dtype="fp16")
    ref = O.attention(q.float().numpy(), k.float().numpy(), v.float().numpy())
    _check(_run(q.to(dev), k.to(dev), v.to(dev)), ref, "C1@fp16")


def test_c1_fp32_as_configured():
    """C1 exactly as BASELINE.json gives it (B1 H4 N256 d64 fp32) through
    gr_attn_fwd's fp32 path, at the fp32 bar against the float64 oracle."""
    dev = _cuda()
    from grammar.workloads import C1, attention_inputs
    q, k, v = attention_inputs(C1, seed=0)
    assert q.dtype == torch.float32
    ref = O.attention(q.numpy(), k.numpy(), v.numpy(), dtype=np.float64)
    got = _run(q.to(dev), k.to(dev), v.to(dev)).double().cpu().numpy()
    print(f"[parity] C1@fp32: max-abs {np.abs(got - ref).max():.2e}", flush=True)
    assert np.allclose(got, ref, rtol=1e-3, atol=1e-3)


def test_c2_full_parity_and_layout_invariance():
    dev = _cuda()
    from grammar.workloads import C2, attention_inputs
    q, k, v = attention_inputs(C2, seed=0)
    ref = O.attention(q.float().numpy(), k.float().numpy(), v.float().numpy())
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    o = _run(qd, kd, vd)
    _check(o, ref, "C2")
    # KT layout stages the same LDS tile -> bitwise identical output.
    o_kt = _run(qd, kd.transpose(-1, -2).contiguous(), vd, k_transposed=True)
    assert torch.equal(o, o_kt)
    # Strided views ([B, N, H, D] memory) give the bitwise same result.
    qs, ks, vs = (t.transpose(1, 2).contiguous().transpose(1, 2) for t in (qd, kd, vd))
    assert qs.stride() != qd.stride()
    assert torch.equal(_run(qs, ks, vs), o)
    # Deterministic across launches.
    assert torch.equal(_run(qd, kd, vd), o)


def test_c2_two_wave_body_layouts_and_strides():
    """The two-waves-per-SIMD body (fp16, d 64, non-causal, 256 x 64 tiles;
    gr_flash_w2.h) at the C2 shape: parity with the oracle; the K^T layout and
    strided [B, N, H, D] views give the bitwise same output (the same operands
    reach the same MFMAs); deterministic across launches."""
    dev = _cuda()
    from grammar.workloads import C2, attention_inputs
    q, k, v = attention_inputs(C2, seed=0)
    ref = O.attention(q.float().numpy(), k.float().numpy(), v.float().numpy())
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    kw = dict(block_m=256, block_n=64)
    o = _run(qd, kd, vd, **kw)
    _check(o, ref, "C2 two-wave body")
    assert torch.equal(_run(qd, kd.transpose(-1, -2).contiguous(), vd, k_transposed=True, **kw), o)
    qs, ks, vs = (t.transpose(1, 2).contiguous().transpose(1, 2) for t in (qd, kd, vd))
    assert qs.stride() != qd.stride()
    assert torch.equal(_run(qs, ks, vs, **kw), o)
    assert torch.equal(_run(qd, kd, vd, **kw), o)


def test_d128_two_wave_body_rescales_a_growing_row_max():
    """The d = 128 two-wave body takes its softmax base from the first tile it
    visits (for causal, the diagonal block) and moves it only when a step's
    row sum leaves the P type's range. Keys past the first 256 scaled up make
    later scores far larger: by 12 (p up to about 2^40, past fp16's 2^16) in
    fp16, by 40 (past fp32's 2^128, so the row sum overflows) in bf16, where V
    is halved to keep the bf16 rounding of p and of O inside the bar. The
    rescaling path runs in both; parity with the oracle."""
    dev = _cuda()
    from grammar.workloads import AttnConfig, attention_inputs
    for dt, causal, grow in (("fp16", False, 12.0), ("fp16", True, 12.0), ("bf16", False, 40.0), ("bf16", True, 40.0)):
        q, kt, v = attention_inputs(AttnConfig("t", 1, 2, 1024, 128, dt, causal), seed=7, k_transposed=True)
        kt = kt.clone()
        kt[..., 256:] = (kt[..., 256:].float() * grow).to(kt.dtype)
        if dt == "bf16":
            v = (v.float() * 0.5).to(v.dtype)
        ref = O.attention(q.float().numpy(), kt.float().numpy(), v.float().numpy(), causal=causal, k_transposed=True)
        o = _run(q.to(dev), kt.to(dev), v.to(dev), causal=causal, k_transposed=True, block_m=256, block_n=64)
        _check(o, ref, f"d128 two-wave growing max {dt} causal={causal} x{grow:g}")


def test_c3_two_wave_body_kt_full_size():
    """C3 (B2 H32 N4096 d128 bf16 causal) with K given transposed, as the
    grammar's programs hand it over: the d = 128 two-wave body. Finite, inside
    each head's V hull, row 0 equal to V row 0, the oracle on sampled heads,
    strided views bitwise equal, deterministic."""
    dev = _cuda()
    from grammar.workloads import C3, attention_inputs
    q, kt, v = attention_inputs(C3, seed=0, k_transposed=True)
    qd, kd, vd = q.to(dev), kt.to(dev), v.to(dev)
    kw = dict(causal=True, k_transposed=True, block_m=256, block_n=64)
    o = _run(qd, kd, vd, **kw)
    of = o.float().cpu()
    assert torch.isfinite(of).all()
    vf = v.float()
    assert bool(((of >= vf.amin(dim=2, keepdim=True) - 1e-2) & (of <= vf.amax(dim=2, keepdim=True) + 1e-2)).all())
    assert (of[:, :, 0] - vf[:, :, 0]).abs().max().item() <= 1e-2
    for b, h in ((0, 0), (1, 31), (0, 17)):
        ref = O.attention(q[b, h].float().numpy(), kt[b, h].float().numpy(), v[b, h].float().numpy(), causal=True,
                          k_transposed=True)
        _check(of[b, h], ref, f"C3 K^T head ({b},{h})")
    qs, vs = (t.transpose(1, 2).contiguous().transpose(1, 2) for t in (qd, vd))
    assert torch.equal(_run(qs, kd, vs, **kw), o)
    assert torch.equal(_run(qd, kd, vd, **kw), o)


def test_c2_key_permutation_property():
    dev = _cuda()
    from grammar.workloads import C2, attention_inputs
    q, k, v = (t.to(dev) for t in attention_inputs(C2, seed=5))
    perm = torch.randperm(C2.N, generator=torch.Generator("cpu").manual_seed(1)).to(dev)
    a = _run(q, k, v).float()
    b = _run(q, k[:, :, perm].contiguous(), v[:, :, perm].contiguous()).float()
    assert (a - b).abs().max().item() <= 2e-3


def test_c3_causal_bf16_full_size():
    dev = _cuda()
    from grammar.workloads import C3, attention_inputs
    q, k, v = attention_inputs(C3, seed=0)
    o = _run(q.to(dev), k.to(dev), v.to(dev), causal=True).float().cpu()
    assert torch.isfinite(o).all()
    # O[i] is a convex combination of V[0..i]: inside each head's V hull.
    vf = v.float()
    lo = vf.amin(dim=2, keepdim=True) - 1e-2
    hi = vf.amax(dim=2, keepdim=True) + 1e-2
    assert bool(((o >= lo) & (o <= hi)).all())
    # Row 0 attends only to key 0: O[.,.,0] == V[.,.,0] up to bf16 rounding.
    assert (o[:, :, 0] - vf[:, :, 0]).abs().max().item() <= 1e-2
    # Oracle on a sample of heads (each is a 4096x4096 fp32 problem on the CPU).
    for b, h in ((0, 0), (1, 31), (0, 17)):
        ref = O.attention(q[b, h].float().numpy(), k[b, h].float().numpy(), v[b, h].float().numpy(), causal=True)
        _check(o[b, h], ref, f"C3 head ({b},{h})")


F32 = [
    # B, H, N, D, k_transposed: waves per workgroup 4 (N % 128 == 0), 2 (N % 64), 1
    (1, 1, 512, 64, True),                   # the reference's own workload
    (2, 3, 256, 128, False),
    (1, 2, 192, 64, True),
    (1, 1, 96, 128, False),
    (2, 1, 32, 64, False),
    # the keys of each query block also split over workgroups when the query
    # blocks would leave CUs idle: 4 parts, 2 parts (above), 8 parts, 2 parts
    # at 128 query blocks, and 512 query blocks without a split
    (1, 1, 1024, 64, False),
    (1, 2, 2048, 128, True),
    (4, 8, 512, 64, False),
]


@pytest.mark.parametrize("case", F32, ids=lambda c: "-".join(map(str, c)))
def test_attention_fp32_parity(case):
    """fp32 throughout (the reference's dtype) against the float64 oracle at
    the reference's fp32 bar, rtol = atol = 1e-3 (test_renderer.py:222-223)."""
    dev = _cuda()
    B, H, N, D, kt = case
    g = torch.Generator("cpu").manual_seed(5)
    q = torch.randn(B, H, N, D, generator=g)
    k = torch.randn(B, H, D, N, generator=g) if kt else torch.randn(B, H, N, D, generator=g)
    v = torch.randn(B, H, N, D, generator=g)
    ref = O.attention(q.numpy(), k.numpy(), v.numpy(), k_transposed=kt, dtype=np.float64)
    o = _run(q.to(dev), k.to(dev), v.to(dev), k_transposed=kt)
    got = o.double().cpu().numpy()
    print(f"[parity] fp32 {case}: max-abs {np.abs(got - ref).max():.2e}", flush=True)
    assert np.allclose(got, ref, rtol=1e-3, atol=1e-3)


def test_attention_fp32_key_split_workspace_per_stream():
    """The fp32 key split keeps its partials in a library workspace per
    (device, stream) that grows on demand: a split call, a larger one queued
    behind it on the same stream (the workspace grows while the first may
    still run), and a split call on a second stream, with no synchronisation
    in between; each against the float64 oracle."""
    dev = _cuda()
    from grammar.attention import flash_attention_fwd
    cases = [(1, 1, 512, 64), (2, 2, 1024, 128), (1, 1, 256, 64)]
    g = torch.Generator("cpu").manual_seed(9)
    ins = [tuple(torch.randn(B, H, N, D, generator=g) for _ in range(3)) for B, H, N, D in cases]
    dev_ins = [tuple(t.to(dev) for t in x) for x in ins]
    torch.cuda.synchronize()
    outs = [flash_attention_fwd(*dev_ins[0]), flash_attention_fwd(*dev_ins[1])]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        outs.append(flash_attention_fwd(*dev_ins[2]))
    torch.cuda.synchronize()
    for (q, k, v), o, c in zip(ins, outs, cases):
        ref = O.attention(q.numpy(), k.numpy(), v.numpy(), dtype=np.float64)
        got = o.double().cpu().numpy()
        print(f"[parity] fp32 split {c}: max-abs {np.abs(got - ref).max():.2e}", flush=True)
        assert np.allclose(got, ref, rtol=1e-3, atol=1e-3), c


@pytest.mark.parametrize("B,H,n", [(1, 2, 512), (2, 8, 2048)])
def test_attention_fp32_strided_heads(B, H, n):
    """fp32 with Q, K, V and O read and written through [B, N, H, D] storage
    (head stride D, sequence stride H * D), split (32 query blocks: 4 key
    parts) and unsplit with 16 32-key blocks per wave (1,024 query blocks),
    against the float64 oracle."""
    dev = _cuda()
    from grammar.attention import flash_attention_fwd
    D = 64
    g = torch.Generator("cpu").manual_seed(13)
    q, k, v = (torch.randn(B, n, H, D, generator=g) for _ in range(3))
    qd, kd, vd = (t.to(dev).transpose(1, 2) for t in (q, k, v))
    out = torch.empty(B, n, H, D, device=dev).transpose(1, 2)
    o = flash_attention_fwd(qd, kd, vd, out=out)
    torch.cuda.synchronize()
    ref = O.attention(*(t.transpose(1, 2).numpy() for t in (q, k, v)), dtype=np.float64)
    got = o.double().cpu().numpy()
    print(f"[parity] fp32 strided N={n}: max-abs {np.abs(got - ref).max():.2e}", flush=True)
    assert np.allclose(got, ref, rtol=1e-3, atol=1e-3)


def test_attention_fp32_rejects_what_it_does_not_cover():
    dev = _cuda()
    from grammar import runtime as rt
    from grammar.attention import flash_attention_fwd_train
    q = torch.zeros(1, 1, 128, 64, dtype=torch.float32, device=dev)
    with pytest.raises(rt.GrError, match="non-causal"):
        _run(q, q, q, causal=True)
    with pytest.raises(rt.GrError, match="training"):
        flash_attention_fwd_train(q, q, q)
    q = torch.zeros(1, 1, 100, 64, dtype=torch.float32, device=dev)
    with pytest.raises(rt.GrError, match="multiple of 32"):
        _run(q, q, q)


def test_rejects_bad_shapes():
    dev = _cuda()
    from grammar import runtime as rt
    q = torch.zeros(1, 1, 200, 64, dtype=torch.float16, device=dev)
    with pytest.raises(rt.GrError):
        _run(q, q, q)                        # N not a multiple of the tile
    q = torch.zeros(1, 1, 256, 96, dtype=torch.float16, device=dev)
    with pytest.raises(rt.GrError):
        _run(q, q, q)                        # unsupported head dim
    with pytest.raises(ValueError):
        from grammar.attention import flash_attention_fwd
        flash_attention_fwd(q.cpu(), q.cpu(), q.cpu())   # no CPU path
    q = torch.zeros(1, 1, 256, 64, dtype=torch.float16, device=dev)
    with pytest.raises(rt.GrError, match="64 x 32"):
        _run(q, q, q, scale=1.0, block_m=256, block_n=128)   # scale log2(e) > 1 in fp16: one tile only


@pytest.mark.parametrize("causal,kt", [(False, False), (True, True), (False, True)])
def test_fp16_scale_above_one_keeps_q_as_given(causal, kt):
    """fp16 with scale log2(e) > 1 (scale 1, a pre-scaled q): Q * scale log2(e)
    could overflow fp16, so these calls keep Q as given and scale every score
    (as torch SDPA accepts any scale). Includes entries of q that the fp16
    pre-scale would have turned into inf."""
    dev = _cuda()
    g = torch.Generator("cpu").manual_seed(41)
    B, H, N, D = 1, 2, 256, 64
    q = (torch.randn((B, H, N, D), generator=g) / 8).half()
    q[0, 0, 5, :4] = 60000.0 / 64           # q * log2(e) * 64 would pass fp16's 65504 if pre-scaled by 64
    k = torch.randn((B, H, N, D), generator=g).half()
    v = torch.randn((B, H, N, D), generator=g).half()
    print(f"[case] fp16 scale 1.0 causal={causal} k_transposed={kt}", flush=True)
    kk = k.transpose(-1, -2).contiguous() if kt else k
    o = _run(q.to(dev), kk.to(dev), v.to(dev), scale=1.0, causal=causal, k_transposed=kt)
    ref = O.attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), causal=causal, scale=1.0)
    _check(o, ref, f"fp16 scale 1 causal={causal} kt={kt}")


def test_fp16_scale_above_one_training_and_decode():
    """The same path through the training forward (lse) and the decode
    launch with more than four queries (the flash body), split and not."""
    dev = _cuda()
    from grammar.attention import flash_attention_decode, flash_attention_fwd_train
    g = torch.Generator("cpu").manual_seed(42)
    q = (torch.randn((1, 2, 128, 64), generator=g) / 8).half()
    k = torch.randn((1, 2, 128, 64), generator=g).half()
    v = torch.randn((1, 2, 128, 64), generator=g).half()
    print("[case] fp16 scale 1.0 training forward", flush=True)
    o, lse = flash_attention_fwd_train(q.to(dev), k.to(dev), v.to(dev), scale=1.0)
    torch.cuda.synchronize()
    ref = O.attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), scale=1.0)
    _check(o, ref, "fp16 scale 1 training forward")
    lref = O.attention_lse(q.float().numpy(), k.float().numpy(), scale=1.0)
    assert np.abs(lse.cpu().numpy() - lref).max() <= 2e-3
    kd = torch.randn((1, 2, 1024, 64), generator=g).half()
    vd = torch.randn((1, 2, 1024, 64), generator=g).half()
    qd = (torch.randn((1, 2, 40, 64), generator=g) / 8).half()
    dref = O.attention(qd.float().numpy(), kd.float().numpy(), vd.float().numpy(), scale=1.0)
    for splits in (1, 3):
        print(f"[case] fp16 scale 1.0 decode Nq40 N1024 splits {splits}", flush=True)
        od = flash_attention_decode(qd.to(dev), kd.to(dev), vd.to(dev), scale=1.0, splits=splits)
        torch.cuda.synchronize()
        _check(od, dref, f"fp16 scale 1 decode splits {splits}")


DECODE = [
    # B, H, Nq, N, D, dtype, splits (0 = chosen by decode_splits)
    (2, 3, 1, 256, 64, "fp16", 0),
    (1, 4, 7, 512, 128, "bf16", 3),
    (2, 2, 64, 1024, 64, "fp16", 1),
    (1, 2, 100, 2048, 128, "fp16", 0),
    (1, 2, 33, 96, 64, "fp16", 2),           # 96 keys: 32-key tiles
    (4, 16, 1, 8192, 128, "bf16", 0),
    (4, 2, 1024, 1024, 64, "fp16", 4),       # C2 at 8 heads, keys split four ways
    # up to 4 queries: the streaming kernel
    (1, 3, 2, 160, 64, "bf16", 1),           # one part, keys past the last full iteration
    (2, 2, 3, 96, 128, "fp16", 2),           # 3 queries on the 4-query kernel
    (1, 2, 4, 4096, 64, "fp16", 0),
    (3, 1, 1, 32, 128, "bf16", 0),           # a single 32-key part
    (1, 1, 1, 8192, 64, "fp16", 64),         # many parts
]


@pytest.mark.parametrize("case", DECODE, ids=lambda c: "-".join(map(str, c)))
def test_decode_parity(case):
    """Nq queries against N keys (non-causal), with and without the key split,
    against the oracle on the same rounded inputs."""
    dev = _cuda()
    from grammar.attention import flash_attention_decode
    B, H, Nq, N, D, dt, splits = case
    print(f"[case] decode {case}", flush=True)
    g = torch.Generator("cpu").manual_seed(5)
    tdt = {"fp16": torch.float16, "bf16": torch.bfloat16}[dt]
    q = torch.randn((B, H, Nq, D), generator=g).to(tdt)
    k = torch.randn((B, H, N, D), generator=g).to(tdt)
    v = torch.randn((B, H, N, D), generator=g).to(tdt)
    o = flash_attention_decode(q.to(dev), k.to(dev), v.to(dev), splits=splits)
    torch.cuda.synchronize()
    ref = O.attention(q.float().numpy(), k.float().numpy(), v.float().numpy())
    _check(o, ref, f"decode {case}")


def test_decode_split_matches_unsplit_and_square_path():
    """The key split only regroups the sum: split and unsplit agree to float
    rounding, and Nq == N reproduces gr_attn_fwd at the same tiles."""
    dev = _cuda()
    from grammar.attention import flash_attention_decode
    g = torch.Generator("cpu").manual_seed(6)
    q, k, v = (torch.randn((2, 4, 512, 64), generator=g).half().to(dev) for _ in range(3))
    one = flash_attention_decode(q, k, v, splits=1)
    four = flash_attention_decode(q, k, v, splits=4)
    torch.cuda.synchronize()
    assert float((one.float() - four.float()).abs().max()) <= 2e-3
    sq = _run(q, k, v, block_m=128, block_n=64)
    assert torch.equal(one, sq)


def test_decode_rejects_bad_arguments():
    dev = _cuda()
    from grammar import runtime as rt
    from grammar.attention import flash_attention_decode
    q = torch.zeros(1, 1, 4, 64, dtype=torch.float16, device=dev)
    k = torch.zeros(1, 1, 100, 64, dtype=torch.float16, device=dev)
    with pytest.raises(rt.GrError):
        flash_attention_decode(q, k, k)                  # keys not a multiple of 32
    k = torch.zeros(1, 1, 1024, 64, dtype=torch.float16, device=dev)
    small = torch.empty(16, dtype=torch.uint8, device=dev)
    with pytest.raises(ValueError):
        flash_attention_decode(q, k, k, splits=4, workspace=small)   # workspace too small
    # the C-ABI itself refuses it too (4 key parts need 4*4*(64+2)*4 bytes)
    import ctypes
    st = (ctypes.c_longlong * 3)(64 * 4, 64 * 4, 64)
    stk = (ctypes.c_longlong * 3)(64 * 1024, 64 * 1024, 64)
    o = torch.empty_like(q)
    assert rt.lib().gr_attn_decode_workspace(1, 1, 4, 64, 4) == 4 * 4 * 66 * 4
    rc = rt.lib().gr_attn_decode(q.data_ptr(), k.data_ptr(), k.data_ptr(), o.data_ptr(), rt.dtype_code(q.dtype),
                                 1, 1, 4, 1024, 64, st, stk, stk, st, 0.125, 4, small.data_ptr(), 16, None)
    assert rc != 0 and "workspace" in rt.last_error()


@pytest.mark.parametrize("dt,causal,D", [("fp16", False, 64), ("bf16", True, 128), ("fp16", True, 64)])
def test_growing_row_max_takes_the_rebase_path(dt, causal, D):
    """Keys drifting along the queries make each row's max grow tile after
    tile, past what an fp16 P holds with the first tile's base: the kernel
    must notice the overflow and redo those tiles with a moved base."""
    dev = _cuda()
    g = torch.Generator("cpu").manual_seed(9)
    B, H, N = 1, 4, 1024
    tdt = {"fp16": torch.float16, "bf16": torch.bfloat16}[dt]
    # q has a common component along (1, ..., 1) and the keys climb along it,
    # so a row's scores grow by about 3 sqrt(D) from the first to the last key
    q = torch.randn((B, H, N, D), generator=g) + 1.0
    k = torch.randn((B, H, N, D), generator=g) + 3.0 * (torch.arange(N).float() / N).view(1, 1, N, 1)
    v = torch.randn((B, H, N, D), generator=g)
    q, k, v = q.to(tdt), k.to(tdt), v.to(tdt)
    s = (q.float() @ k.float().transpose(-1, -2)) / math.sqrt(D)
    grow = s.amax(-1) - s[..., :64].amax(-1)
    assert float(grow.median()) > 16 * math.log(2), "inputs must force a rebase"
    ref = O.attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), causal=causal)
    # 129 / 257: the pipelined schedule, whose next-tile scores were computed
    # from the base before the move
    for bm, bn in ((128, 64), (256, 64), (129, 64), (257, 64)):
        o = _run(q.to(dev), k.to(dev), v.to(dev), causal=causal, block_m=bm, block_n=bn)
        _check(o, ref, f"growing max {dt} causal={causal} D={D} {bm}x{bn}")


BWD = [
    # B, H, N, D, dtype, causal
    (1, 2, 256, 64, "fp16", False),
    (2, 2, 256, 64, "bf16", True),
    (1, 3, 512, 128, "fp16", True),
    (1, 2, 256, 128, "bf16", False),
    (2, 4, 1024, 64, "fp16", True),
    (1, 2, 384, 64, "bf16", True),      # N not a multiple of 256: 4-wave dQ workgroups
    (1, 2, 640, 128, "fp16", False),
    (1, 2, 2048, 128, "bf16", True),
    # fp16 d 64 non-causal, N a multiple of 256: the training forward (and its
    # lse) on the two-wave body at the default tile, 16 key tiles
    (1, 2, 1024, 64, "fp16", False),
]


@pytest.mark.parametrize("case", BWD, ids=lambda c: "-".join(map(str, c)))
def test_backward_parity(case):
    """lse of the training forward and dQ, dK, dV of gr_attn_bwd against the
    float64 oracle (itself pinned by finite differences) on the same rounded
    inputs. Bar: the attention bar on gradients scaled to unit size
    (max-abs <= 2e-2 and mean-abs <= 2e-3 of max(1, max|ref|))."""
    dev = _cuda()
    from grammar.attention import flash_attention_bwd, flash_attention_fwd_train
    B, H, N, D, dt, causal = case
    print(f"[case] backward {case}", flush=True)
    g = torch.Generator("cpu").manual_seed(13)
    tdt = {"fp16": torch.float16, "bf16": torch.bfloat16}[dt]
    q, k, v, do = (torch.randn((B, H, N, D), generator=g).to(tdt) for _ in range(4))
    o, lse = flash_attention_fwd_train(q.to(dev), k.to(dev), v.to(dev), causal=causal)
    dq, dk, dv = flash_attention_bwd(q.to(dev), k.to(dev), v.to(dev), o, do.to(dev), lse, causal=causal)
    torch.cuda.synchronize()
    qf, kf, vf, dof = (t.double().numpy() for t in (q, k, v, do))
    ref_lse = O.attention_lse(qf, kf, causal=causal)
    assert float(np.abs(lse.cpu().numpy() - ref_lse).max()) <= 2e-3, "lse"
    rdq, rdk, rdv = O.attention_backward(qf, kf, vf, dof, causal=causal)
    for name, got, ref in (("dq", dq, rdq), ("dk", dk, rdk), ("dv", dv, rdv)):
        got = got.float().cpu().numpy()
        unit = max(1.0, float(np.abs(ref).max()))
        mx, mn = O.errors(got / unit, ref / unit)
        print(f"[parity] backward {case} {name}: max-abs {mx:.3e} mean-abs {mn:.3e} (unit {unit:.2f})", flush=True)
        assert np.isfinite(got).all(), name
        assert mx <= O.MAX_ABS_TOL and mn <= O.MEAN_ABS_TOL, (name, mx, mn)


@pytest.mark.parametrize("dt,causal", [("bf16", True), ("fp16", False)])
def test_backward_full_length_d128_against_torch_fp32(dt, causal):
    """dQ, dK, dV at N = 4,096, d = 128 (C3's length and head size, two heads)
    against gradients that torch autograd takes through attention computed
    in float32 on the GPU, from the same rounded inputs. At this length the
    d = 128 dK/dV kernel runs 32 query tiles per key block (one masked, the
    rest on the unmasked path). Bar: the attention bar on gradients scaled
    to unit size."""
    dev = _cuda()
    from grammar.attention import flash_attention_bwd, flash_attention_fwd_train
    B, H, N, D = 1, 2, 4096, 128
    print(f"[case] backward B{B} H{H} N{N} d{D} {dt} causal={causal} against torch fp32", flush=True)
    g = torch.Generator("cpu").manual_seed(29)
    tdt = {"fp16": torch.float16, "bf16": torch.bfloat16}[dt]
    q, k, v, do = (torch.randn((B, H, N, D), generator=g).to(tdt).to(dev) for _ in range(4))
    o, lse = flash_attention_fwd_train(q, k, v, causal=causal)
    dq, dk, dv = flash_attention_bwd(q, k, v, o, do, lse, causal=causal)
    qf, kf, vf = (t.float().requires_grad_() for t in (q, k, v))
    s = (qf @ kf.transpose(-1, -2).contiguous()) / math.sqrt(D)
    if causal:
        s = s.masked_fill(torch.ones(N, N, dtype=torch.bool, device=dev).triu(1), float("-inf"))
    (torch.softmax(s, dim=-1) @ vf).backward(do.float())
    torch.cuda.synchronize()
    for name, got, ref in (("dq", dq, qf.grad), ("dk", dk, kf.grad), ("dv", dv, vf.grad)):
        unit = max(1.0, float(ref.abs().max()))
        d = (got.float() - ref).abs() / unit
        mx, mn = float(d.max()), float(d.mean())
        print(f"[parity] backward N{N} d{D} {dt} causal={causal} {name}: max-abs {mx:.3e} mean-abs {mn:.3e}",
              flush=True)
        assert torch.isfinite(got).all(), name
        assert mx <= O.MAX_ABS_TOL and mn <= O.MEAN_ABS_TOL, (name, mx, mn)


def test_bound_training_launchers_repeat_and_validate():
    """bind_flash_attention_train / bind_flash_attention_bwd: repeated launches
    give bit-identical results (no state carried between calls, delta is
    rewritten each time), and malformed operands are rejected before any
    launch."""
    dev = _cuda()
    from grammar.attention import bind_flash_attention_bwd, bind_flash_attention_train
    g = torch.Generator("cpu").manual_seed(15)
    q, k, v, do = (torch.randn((2, 2, 512, 128), generator=g).to(torch.bfloat16).to(dev) for _ in range(4))
    fwd, o, lse = bind_flash_attention_train(q, k, v, causal=True)
    fwd()
    bwd, grads = bind_flash_attention_bwd(q, k, v, o, do, lse, causal=True)
    bwd()
    torch.cuda.synchronize()
    first = [t.clone() for t in (o, lse, *grads)]
    fwd()
    bwd()
    torch.cuda.synchronize()
    for a, b in zip(first, (o, lse, *grads)):
        assert torch.equal(a, b)
    with pytest.raises(ValueError):
        bind_flash_attention_bwd(q, k, v, o, do.transpose(2, 3), lse)            # not [B, H, N, D]
    with pytest.raises(ValueError):
        bind_flash_attention_bwd(q, k, v, o, do[:, :, ::2].repeat(1, 1, 2, 1).transpose(1, 2).contiguous()
                                 .transpose(1, 2), lse)                           # non-contiguous
    with pytest.raises(ValueError):
        bind_flash_attention_bwd(q, k, v, o, do, lse.half())                       # lse must be fp32
    with pytest.raises(ValueError):
        bind_flash_attention_bwd(q, k, v, o, do, lse, workspace=torch.empty(16, dtype=torch.uint8, device=dev))


def test_autograd_training_step_matches_oracle():
    """flash_attention as a torch.autograd function: loss.backward() gives the
    oracle's gradients."""
    dev = _cuda()
    from grammar.attention import flash_attention
    g = torch.Generator("cpu").manual_seed(14)
    q, k, v = (torch.randn((1, 2, 256, 64), generator=g).half() for _ in range(3))
    w = torch.randn((1, 2, 256, 64), generator=g).half()
    qd, kd, vd = (t.to(dev).requires_grad_() for t in (q, k, v))
    out = flash_attention(qd, kd, vd, causal=True)
    (out.float() * w.to(dev).float()).sum().backward()
    torch.cuda.synchronize()
    rdq, rdk, rdv = O.attention_backward(q.double().numpy(), k.double().numpy(), v.double().numpy(),
                                         w.double().numpy(), causal=True)
    for got, ref in ((qd.grad, rdq), (kd.grad, rdk), (vd.grad, rdv)):
        mx, mn = O.errors(got.float().cpu().numpy(), ref)
        assert mx <= O.MAX_ABS_TOL and mn <= O.MEAN_ABS_TOL, (mx, mn)
