"""GPU parity of the hand-written CDNA4 GEMM with fused epilogue (gr_gemm) and
of the two-GEMM MLP block (gr_mlp_fwd) against CPU oracles on the same seeded,
fp16/bf16-rounded inputs.

Bar: max-abs <= 2e-2 and mean-abs <= 2e-3. Small
shapes compare every element against float64 products; the full C4 MLP
(X[8192,4096] W1[4096,11008] W2[11008,4096]) compares 256 sampled rows,
which the row-wise structure of Y = SiLU(X W1) W2 makes exact oracles."""
import numpy as np
import pytest

from oracle import attention as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _cuda():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _td(name):
    return {"fp16": torch.float16, "bf16": torch.bfloat16}[name]


def _check(got, ref, label):
    got = got.float().cpu().numpy()
    mx, mn = O.errors(got, ref)
    print(f"[parity] {label}: max-abs {mx:.3e} mean-abs {mn:.3e}", flush=True)
    assert np.isfinite(got).all(), label
    assert mx <= O.MAX_ABS_TOL and mn <= O.MEAN_ABS_TOL, (label, mx, mn)


def _act(x, epi):
    if epi == "relu":
        return np.maximum(x, 0.0)
    if epi == "silu":
        return O.silu(x)
    return x


CASES = [
    # batch, M, N, K, dtype, epilogue, alpha, b_kmajor, tile
    (1, 256, 256, 128, "fp16", "none", 1.0, False, (128, 128)),
    (1, 256, 256, 128, "fp16", "none", 1.0, False, (256, 128)),
    (1, 256, 256, 128, "fp16", "none", 1.0, False, (128, 256)),
    (1, 256, 256, 128, "fp16", "none", 1.0, False, (256, 256)),
    (1, 256, 512, 192, "bf16", "silu", 0.5, False, (128, 128)),
    (1, 512, 256, 256, "fp16", "relu", 1.0, True, (256, 256)),
    (1, 256, 256, 128, "bf16", "none", 0.125, True, (128, 256)),
    (3, 128, 256, 64, "fp16", "silu", 1.0, False, (128, 128)),
    # ragged M / N (edge tiles store only their valid part), K a multiple of 32 only
    (1, 200, 136, 96, "fp16", "none", 1.0, False, (128, 128)),
    (1, 300, 1376, 1376, "fp16", "silu", 1.0, False, (256, 256)),
    (2, 72, 40, 64, "bf16", "relu", 1.0, True, (256, 256)),
    (1, 1000, 264, 160, "fp16", "none", 0.5, True, (128, 256)),
    (1, 33, 8, 32, "bf16", "silu", 1.0, False, (256, 128)),
    # the 256 x 256 tile's one-wave body: one k tile, three 32-deep tiles (only
    # the loop's tail runs), bf16 with a [K, N] B, a batch with a K-major B
    (1, 256, 256, 64, "bf16", "none", 1.0, False, (256, 256)),
    (1, 512, 512, 96, "fp16", "silu", 1.0, False, (256, 256)),
    (2, 256, 512, 192, "bf16", "relu", 0.5, True, (256, 256)),
    # a last round of at most half the CUs (256 on MI355X): the columns past
    # the whole rounds run as 256 x 128 tiles in a second launch (ragged in
    # the second and third case: 320 columns there)
    (1, 4096, 4352, 128, "fp16", "silu", 1.0, False, (256, 256)),
    (1, 4096, 4416, 64, "bf16", "relu", 1.0, True, (256, 256)),
    (1, 4096, 4416, 96, "fp16", "none", 0.5, False, (256, 256)),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(map(str, c)))
def test_gemm_small_parity(case):
    dev = _cuda()
    from grammar.gemm import gemm
    z, M, N, K, dt, epi, alpha, km, (bm, bn) = case
    print(f"[case] gemm z={z} M={M} N={N} K={K} {dt} {epi} alpha={alpha} kmajor={km} tile={bm}x{bn}", flush=True)
    g = torch.Generator("cpu").manual_seed(11)
    a = torch.randn((z, M, K), generator=g).to(_td(dt))
    b = (torch.randn((z, N, K) if km else (z, K, N), generator=g) / np.sqrt(K)).to(_td(dt))
    c = gemm(a.to(dev), b.to(dev), epilogue=epi, alpha=alpha, b_kmajor=km, block_m=bm, block_n=bn)
    torch.cuda.synchronize()
    a64 = a.double().numpy()
    b64 = b.double().numpy()
    if km:
        b64 = b64.transpose(0, 2, 1)
    ref = _act(alpha * (a64 @ b64), epi)
    _check(c, ref, f"gemm {case}")


@pytest.mark.parametrize("dt,N,km", [("fp16", 4352, False), ("bf16", 4416, True)])
def test_split_launch_matches_the_whole_grid(dt, N, km):
    """A batch-1 launch whose last round is part-filled runs as two launches
    (the tail on 256 x 128 tiles); a batch-2 launch of the same matrices
    runs as one grid. Each output keeps its k order, so the two agree bit
    for bit."""
    dev = _cuda()
    from grammar.gemm import gemm
    print(f"[case] split vs whole grid {dt} M=4096 N={N} K=128 kmajor={km}", flush=True)
    g = torch.Generator("cpu").manual_seed(21)
    a = torch.randn((1, 4096, 128), generator=g).to(_td(dt)).to(dev)
    b = (torch.randn((N, 128) if km else (128, N), generator=g) / np.sqrt(128)).to(_td(dt)).to(dev)
    one = gemm(a, b, epilogue="silu", b_kmajor=km, block_m=256, block_n=256)
    two = gemm(a.expand(2, -1, -1).contiguous(), b, epilogue="silu", b_kmajor=km, block_m=256, block_n=256)
    torch.cuda.synchronize()
    assert torch.equal(one[0], two[0]) and torch.equal(one[0], two[1])


F32_CASES = [
    # batch, M, N, K, epilogue, alpha, b_kmajor, tile: the fp32 matrix-core GEMM (gr_gemm_f32.h)
    (1, 128, 128, 64, "none", 1.0, False, (64, 64)),
    (1, 256, 512, 96, "silu", 0.5, False, (128, 128)),
    (2, 64, 256, 136, "relu", 1.0, True, (32, 128)),
    (1, 512, 64, 512, "none", 0.125, False, (128, 32)),
    (3, 96, 32, 40, "none", 1.0, True, (32, 32)),
    (1, 384, 256, 1024, "silu", 1.0, False, (0, 0)),
]


@pytest.mark.parametrize("case", F32_CASES, ids=lambda c: "-".join(map(str, c)))
def test_gemm_fp32_parity(case):
    """fp32 in, fp32 out, fp32 products and sums on v_mfma_f32_32x32x2_f32:
    against float64 at 1e-4 relative to the output's scale."""
    dev = _cuda()
    from grammar.gemm import gemm
    z, M, N, K, epi, alpha, km, (bm, bn) = case
    print(f"[case] gemm fp32 z={z} M={M} N={N} K={K} {epi} alpha={alpha} kmajor={km} tile={bm}x{bn}", flush=True)
    g = torch.Generator("cpu").manual_seed(13)
    a = torch.randn((z, M, K), generator=g)
    b = torch.randn((z, N, K) if km else (z, K, N), generator=g) / np.sqrt(K)
    c = gemm(a.to(dev), b.to(dev), epilogue=epi, alpha=alpha, b_kmajor=km, block_m=bm, block_n=bn)
    torch.cuda.synchronize()
    b64 = b.double().numpy()
    if km:
        b64 = b64.transpose(0, 2, 1)
    ref = _act(alpha * (a.double().numpy() @ b64), epi)
    got = c.double().cpu().numpy()
    err = np.abs(got - ref).max() / max(1.0, np.abs(ref).max())
    print(f"[parity] gemm fp32 {case}: max rel {err:.2e}", flush=True)
    assert c.dtype == torch.float32 and np.isfinite(got).all() and err <= 1e-4


def test_gemm_fp32_rejects_ragged_tiles():
    dev = _cuda()
    from grammar import runtime as rt
    from grammar.gemm import gemm
    a = torch.zeros((100, 64), device=dev)
    b = torch.zeros((64, 64), device=dev)
    with pytest.raises(rt.GrError):
        gemm(a, b, block_m=64, block_n=64)


def test_gemm_broadcast_b_and_batch_views():
    """A [2,3,M,K] against one shared B [K,N] (batch stride 0), and a
    non-contiguous batch view of A (every other matrix)."""
    dev = _cuda()
    from grammar.gemm import gemm
    g = torch.Generator("cpu").manual_seed(5)
    a = torch.randn((2, 3, 128, 64), generator=g).half()
    b = (torch.randn((64, 256), generator=g) / 8).half()
    c = gemm(a.to(dev), b.to(dev), block_m=128, block_n=128)
    torch.cuda.synchronize()
    _check(c, a.double().numpy() @ b.double().numpy(), "broadcast b")
    a6 = torch.randn((6, 128, 64), generator=g).half().to(dev)
    sub = a6[::2]
    c2 = gemm(sub, b.to(dev), block_m=128, block_n=128)
    torch.cuda.synchronize()
    _check(c2, sub.double().cpu().numpy() @ b.double().numpy(), "strided batch")


def test_gemm_matches_triple_loop_tiny():
    """Pins the product against the unvectorised float64 loop (not BLAS)."""
    dev = _cuda()
    from grammar.gemm import gemm
    g = torch.Generator("cpu").manual_seed(2)
    a = torch.randn((128, 64), generator=g).half()
    b = (torch.randn((64, 128), generator=g) / 8).half()
    c = gemm(a.to(dev), b.to(dev), block_m=128, block_n=128)
    torch.cuda.synchronize()
    _check(c, O.matmul_loop(a.numpy(), b.numpy()), "triple loop")


def test_gemm_rejects_bad_shapes():
    dev = _cuda()
    from grammar.gemm import gemm
    from grammar.runtime import GrError
    a = torch.zeros((200, 64), dtype=torch.float16, device=dev)
    b = torch.zeros((64, 128), dtype=torch.float16, device=dev)
    with pytest.raises(GrError):
        gemm(a[:, :48], b[:48], block_m=128, block_n=128)   # K not a multiple of 32
    with pytest.raises(GrError):
        gemm(a, b[:, :100], block_m=128, block_n=128)       # N not a multiple of 8
    with pytest.raises(GrError):
        gemm(a[:128], b, block_m=64, block_n=64)       # tile not compiled in
    with pytest.raises(ValueError):
        gemm(a[:128], b.t(), block_m=128, block_n=128)  # non-unit inner stride


@pytest.mark.parametrize("dt", ["fp16", "bf16"])
def test_mlp_small_parity(dt):
    dev = _cuda()
    from grammar.gemm import mlp_fwd
    g = torch.Generator("cpu").manual_seed(7)
    M, D, F = 256, 256, 512
    x = torch.randn((M, D), generator=g).to(_td(dt))
    w1 = (torch.randn((D, F), generator=g) / np.sqrt(D)).to(_td(dt))
    w2 = (torch.randn((F, D), generator=g) / np.sqrt(F)).to(_td(dt))
    y = mlp_fwd(x.to(dev), w1.to(dev), w2.to(dev), block_m=128, block_n=128)
    torch.cuda.synchronize()
    ref = O.mlp_silu(x.float().numpy(), w1.float().numpy(), w2.float().numpy(), dtype=np.float64)
    _check(y, ref, f"mlp {dt}")


def test_mlp_c4_tensor_parallel_shard():
    """One GPU's share of C4 split eight ways (W1 by columns, W2 by rows:
    F = 11008 / 8 = 1376, not a multiple of the 256 tile); sampled rows."""
    dev = _cuda()
    from grammar.gemm import mlp_fwd
    from grammar.workloads import C4, mlp_inputs
    print("[case] mlp C4 shard F=1376", flush=True)
    x, w1, w2 = mlp_inputs(C4, seed=0)
    w1s, w2s = w1[:, :1376].contiguous(), w2[:1376].contiguous()
    y = mlp_fwd(x.to(dev), w1s.to(dev), w2s.to(dev))
    torch.cuda.synchronize()
    rows = np.random.default_rng(1).choice(C4.M, 128, replace=False)
    ref = O.mlp_silu(x[rows].float().numpy(), w1s.float().numpy(), w2s.float().numpy(), dtype=np.float32)
    _check(y[torch.as_tensor(rows, device=dev)], ref, "mlp C4 shard rows")


def test_mlp_c4_sampled_rows():
    """Full C4 shape; Y's rows depend only on the same rows of X."""
    dev = _cuda()
    from grammar.gemm import mlp_fwd
    from grammar.workloads import C4, mlp_inputs
    print("[case] mlp C4 full shape", flush=True)
    x, w1, w2 = mlp_inputs(C4, seed=0)
    y = mlp_fwd(x.to(dev), w1.to(dev), w2.to(dev))
    torch.cuda.synchronize()
    rows = np.random.default_rng(0).choice(C4.M, 256, replace=False)
    ref = O.mlp_silu(x[rows].float().numpy(), w1.float().numpy(), w2.float().numpy(), dtype=np.float32)
    _check(y[torch.as_tensor(rows, device=dev)], ref, "mlp C4 rows")
    y2 = mlp_fwd(x.to(dev), w1.to(dev), w2.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(y, y2), "MLP is not deterministic"
