"""Pins the CPU oracle (oracle/attention.py, oracle/naive_torch.py) before any
GPU result is compared with it. Each check is chosen so that a plausible
mistake -- a missing max shift, a wrong scale, a transposed operand, a
row/column mix-up in the broadcasts, a wrong mask direction, a dropped term in
SiLU -- fails at least one of them."""
import math

import numpy as np
import pytest

from oracle import attention as O


def _rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape)


@pytest.mark.parametrize("causal", [False, True])
def test_attention_matches_float64_bruteforce(causal):
    q, k, v = (_rand((2, 3, 7, 5), s) for s in (1, 2, 3))
    ref = O.attention_bruteforce(q, k, v, causal=causal)
    got = O.attention(q, k, v, causal=causal, dtype=np.float64)
    assert np.allclose(got, ref, rtol=1e-12, atol=1e-12)
    got32 = O.attention(q, k, v, causal=causal)
    assert np.allclose(got32, ref, rtol=1e-5, atol=1e-5)


def test_fewer_queries_than_keys_are_rows_of_the_square_problem():
    # the decode shape (Nq != N, non-causal) is the same closed form: its rows
    # equal the square problem's rows for those queries
    q, k, v = (_rand((2, 3, 11, 5), s) for s in (7, 8, 9))
    full = O.attention(q, k, v, dtype=np.float64)
    rows = [0, 4, 10]
    part = O.attention(q[:, :, rows], k, v, dtype=np.float64)
    assert part.shape == (2, 3, 3, 5)
    assert np.allclose(part, full[:, :, rows], rtol=1e-13, atol=1e-13)


def test_kt_layout_equals_k_layout():
    q, k, v = (_rand((1, 2, 9, 4), s) for s in (4, 5, 6))
    a = O.attention(q, k, v, dtype=np.float64)
    b = O.attention(q, np.swapaxes(k, -1, -2), v, k_transposed=True, dtype=np.float64)
    assert np.allclose(a, b, rtol=0, atol=1e-14)


def test_scale_is_one_over_sqrt_d():
    # With d = 4 the default scale is 0.5; an explicit 0.5 must agree and 1.0 must not.
    q, k, v = (_rand((1, 1, 6, 4), s) for s in (7, 8, 9))
    a = O.attention(q, k, v, dtype=np.float64)
    b = O.attention(q, k, v, scale=0.5, dtype=np.float64)
    c = O.attention(q, k, v, scale=1.0, dtype=np.float64)
    assert np.allclose(a, b, atol=1e-14) and not np.allclose(a, c, atol=1e-3)


def test_invariants_rows_sum_to_one_and_convex_hull():
    q, k, v = (_rand((2, 2, 16, 8), s) for s in (10, 11, 12))
    st = O.attention_staged(q, np.swapaxes(k, -1, -2), v, dtype=np.float64)
    assert np.allclose(st["P"].sum(-1), 1.0, atol=1e-12)
    o = st["O"]
    lo = v.min(axis=-2, keepdims=True)
    hi = v.max(axis=-2, keepdims=True)
    assert np.all(o >= lo - 1e-12) and np.all(o <= hi + 1e-12)


@pytest.mark.parametrize("causal", [False, True])
def test_zero_query_gives_mean_or_prefix_mean(causal):
    n = 12
    k, v = _rand((1, 1, n, 4), 13), _rand((1, 1, n, 4), 14)
    q = np.zeros((1, 1, n, 4))
    o = O.attention(q, k, v, causal=causal, dtype=np.float64)
    if causal:
        want = np.cumsum(v, axis=-2) / np.arange(1, n + 1)[:, None]
    else:
        want = np.broadcast_to(v.mean(axis=-2, keepdims=True), v.shape)
    assert np.allclose(o, want, atol=1e-12)


def test_single_key_returns_v():
    q, k, v = (_rand((2, 1, 1, 3), s) for s in (15, 16, 17))
    assert np.allclose(O.attention(q, k, v, dtype=np.float64), v, atol=1e-14)


def test_key_value_permutation_invariance():
    q, k, v = (_rand((1, 2, 10, 4), s) for s in (18, 19, 20))
    perm = np.random.default_rng(21).permutation(10)
    a = O.attention(q, k, v, dtype=np.float64)
    b = O.attention(q, k[..., perm, :], v[..., perm, :], dtype=np.float64)
    assert np.allclose(a, b, atol=1e-13)


def test_row_shift_invariance_guards_the_max_shift():
    # Adding a per-row constant to the scores leaves softmax unchanged. Large
    # shifts also exercise the max shift: without it exp() overflows to inf.
    s = _rand((4, 6), 22) * 3.0
    shift = np.array([[0.0], [500.0], [-700.0], [1000.0]])
    a = O.softmax_rows(s)
    b = O.softmax_rows(s + shift)
    assert np.all(np.isfinite(b)) and np.allclose(a, b, atol=1e-12)


def test_causal_mask_direction():
    # Row i may only see keys j <= i: making V[j] huge for j > i must not move O[i].
    n = 8
    q, k, v = (_rand((1, 1, n, 4), s) for s in (23, 24, 25))
    v2 = v.copy()
    v2[..., n - 1, :] = 1e6
    a = O.attention(q, k, v, causal=True, dtype=np.float64)
    b = O.attention(q, k, v2, causal=True, dtype=np.float64)
    assert np.allclose(a[..., : n - 1, :], b[..., : n - 1, :], atol=1e-12)
    assert not np.allclose(a[..., n - 1, :], b[..., n - 1, :])


@pytest.mark.parametrize("causal", [False, True])
def test_staged_equals_fused(causal):
    q, k, v = (_rand((2, 2, 24, 8), s) for s in (26, 27, 28))
    st = O.attention_staged(q, np.swapaxes(k, -1, -2), v, causal=causal, dtype=np.float64)
    assert np.allclose(st["O"], O.attention(q, k, v, causal=causal, dtype=np.float64), atol=1e-12)
    assert st["mx"].shape[-1] == 1 and st["sm"].shape[-1] == 1


def test_torch_staged_baseline_matches_oracle():
    torch = pytest.importorskip("torch")
    from oracle.naive_torch import staged_attention
    q, k, v = (_rand((1, 4, 64, 16), s).astype(np.float32) for s in (29, 30, 31))
    kt = np.ascontiguousarray(np.swapaxes(k, -1, -2))
    got = staged_attention(torch.from_numpy(q), torch.from_numpy(kt), torch.from_numpy(v)).numpy()
    ref = O.attention(q, k, v, dtype=np.float64)
    assert np.allclose(got, ref, atol=1e-5)
    got_c = staged_attention(torch.from_numpy(q), torch.from_numpy(kt), torch.from_numpy(v), causal=True).numpy()
    assert np.allclose(got_c, O.attention(q, k, v, causal=True, dtype=np.float64), atol=1e-5)


def test_silu_closed_form_points():
    x = np.array([0.0, 1.0, -1.0, 20.0, -20.0])
    want = np.array([0.0, 1.0 / (1.0 + math.exp(-1.0)), -1.0 / (1.0 + math.e), 20.0, 0.0])
    assert np.allclose(O.silu(x), want, atol=1e-7)


def test_mlp_matches_loop_gemm():
    x, w1, w2 = _rand((5, 6), 32), _rand((6, 7), 33), _rand((7, 6), 34)
    h = O.matmul_loop(x, w1)
    a = h / (1.0 + np.exp(-h))
    ref = O.matmul_loop(a, w2)
    assert np.allclose(O.mlp_silu(x, w1, w2, dtype=np.float64), ref, atol=1e-12)
    assert np.allclose(O.matmul_loop(x, w1), x @ w1, atol=1e-12)


def test_tolerance_helper():
    ref = np.zeros((10, 10))
    assert O.within_tolerance(ref + 1e-3, ref)
    assert not O.within_tolerance(ref + 3e-3, ref)          # mean-abs fails
    bad = ref.copy(); bad[0, 0] = 0.05
    assert not O.within_tolerance(bad, ref)                  # max-abs fails
    nan = ref.copy(); nan[1, 1] = np.nan
    assert not O.within_tolerance(nan, ref)


def test_reference_flop_counts():
    # Values held by the reference: 4*N^2*d at N=512, d=64 is the pure-GEMM
    # part of KERNEL_META.flops = 68,681,728 (pytorch-naive.py:67); six
    # pointwise/row-reduce passes over [512,512] make up the rest.
    from grammar.workloads import C2, C3
    assert 4 * 512 * 512 * 64 + 6 * 512 * 512 == 68681728
    assert C2.flops == 17179869184
    assert C3.flops == 274877906944


@pytest.mark.parametrize("causal", [False, True])
def test_backward_matches_finite_differences(causal):
    # d/dx of f = sum(O * dO) by central differences in float64, every element
    rng = np.random.default_rng(3)
    q, k, v, do = (rng.standard_normal((2, 5, 4)) for _ in range(4))
    dq, dk, dv = O.attention_backward(q, k, v, do, causal=causal)

    def f(q_, k_, v_):
        return float((O.attention(q_, k_, v_, causal=causal, dtype=np.float64) * do).sum())
    eps = 1e-6
    for x, g in ((q, dq), (k, dk), (v, dv)):
        num = np.zeros_like(x)
        for idx in np.ndindex(*x.shape):
            xp, xm = x.copy(), x.copy()
            xp[idx] += eps
            xm[idx] -= eps
            args_p = [xp if x is t else t for t in (q, k, v)]
            args_m = [xm if x is t else t for t in (q, k, v)]
            num[idx] = (f(*args_p) - f(*args_m)) / (2 * eps)
        assert np.allclose(g, num, rtol=1e-6, atol=1e-7)
    if causal:   # the first query attends to one key only: its softmax is constant, its gradient zero
        assert np.allclose(dq[:, 0], 0.0, atol=1e-12)


def test_lse_matches_finite_difference_and_closed_form():
    rng = np.random.default_rng(4)
    q, k = rng.standard_normal((3, 6, 4)), rng.standard_normal((3, 6, 4))
    lse = O.attention_lse(q, k)
    s = (q @ np.swapaxes(k, -1, -2)) / 2.0
    assert np.allclose(lse, np.log(np.exp(s).sum(-1)), rtol=1e-13)
    # softmax rows are exp(s - lse)
    assert np.allclose(np.exp(s - lse[..., None]), O.softmax_rows(s), rtol=1e-12)
    lc = O.attention_lse(q, k, causal=True)
    assert np.allclose(lc[:, 0], s[:, 0, 0])     # the first query sees one key
