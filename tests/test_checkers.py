"""CPU pins of the closed-form checkers every descent variant is scored
against (the product-side `reference` callables handed to the Evaluator):
run_attention_search.attention_reference and run_mlp_search.mlp_reference
against the numpy oracle on the same inputs (reference checkers:
run_attention_search.py:169-181, run_mlp_search.py:138-149).

A mistake that would let a wrong kernel pass -- a missing scale, the mask on
the wrong side of the diagonal or missing, the softmax over the wrong axis,
relu in place of SiLU -- makes one of these fail."""
import math

import numpy as np
import pytest
import torch

from oracle import attention as O


def _attn_inputs(shape, d, seed):
    g = torch.Generator("cpu").manual_seed(seed)
    q = torch.randn(shape + (d,), generator=g)
    k = torch.randn(shape + (d,), generator=g)
    v = torch.randn(shape + (d,), generator=g)
    return q, k, v


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("lead", [(), (2, 3)])
def test_attention_reference_matches_oracle(causal, lead):
    import run_attention_search as RS
    n, d = 96, 32
    q, k, v = _attn_inputs(lead + (n,), d, seed=4)
    scale = 1.0 / math.sqrt(d)
    got = RS.attention_reference(scale, causal)({"Q": q, "KT": k.transpose(-1, -2).contiguous(), "V": v})
    ref = O.attention(q.numpy(), k.numpy(), v.numpy(), causal=causal, scale=scale, dtype=np.float64)
    assert np.abs(got.double().numpy() - ref).max() < 1e-5
    # and against the float64 brute force on one head
    bf = O.attention_bruteforce(q.reshape(-1, n, d)[0].double().numpy(), k.reshape(-1, n, d)[0].double().numpy(),
                                v.reshape(-1, n, d)[0].double().numpy(), causal=causal, scale=scale)
    assert np.abs(got.reshape(-1, n, d)[0].double().numpy() - bf).max() < 1e-5


def _softmax_over_queries(q, k, v, scale):
    s = (q @ k.T) * scale
    s = np.where(np.triu(np.ones(s.shape, dtype=bool), 1), -np.inf, s)
    return O.softmax_rows(s.T).T @ v


def test_attention_reference_detects_planted_mistakes():
    """The checker disagrees with each plausible wrong kernel by far more than
    the tolerance."""
    import run_attention_search as RS
    n, d = 64, 16
    q, k, v = _attn_inputs((n,), d, seed=9)
    scale = 1.0 / math.sqrt(d)
    good = RS.attention_reference(scale, True)({"Q": q, "KT": k.t().contiguous(), "V": v}).numpy()
    wrong = {
        "unscaled": O.attention(q.numpy(), k.numpy(), v.numpy(), causal=True, scale=1.0),
        "mask transposed": np.flip(O.attention(q.numpy()[::-1].copy(), k.numpy()[::-1].copy(),
                                               v.numpy()[::-1].copy(), causal=True, scale=scale), 0),
        "not causal": O.attention(q.numpy(), k.numpy(), v.numpy(), causal=False, scale=scale),
        "softmax over queries": _softmax_over_queries(q.numpy(), k.numpy(), v.numpy(), scale),
    }
    for name, w in wrong.items():
        assert np.abs(good - w).max() > 10 * O.MAX_ABS_TOL, name


def test_mlp_reference_silu_matches_oracle():
    import run_mlp_search as MS
    ins = MS.mlp_inputs(48, 64, 96, "fp32", seed=2, device="cpu")
    got = MS.mlp_reference("silu")(ins).double().numpy()
    ref = O.mlp_silu(ins["X"].numpy(), ins["W1"].numpy(), ins["W2"].numpy(), dtype=np.float64)
    assert np.abs(got - ref).max() < 1e-4
    relu = np.maximum(ins["X"].double().numpy() @ ins["W1"].double().numpy(), 0) @ ins["W2"].double().numpy()
    assert np.abs(got - relu).max() > 0.05        # relu in place of SiLU would be caught


def test_mlp_reference_layernorm_block():
    """relu MLP + residual + LayerNorm: rows of the result have mean 0 and
    variance 1 (no affine), and before the normalisation the block equals
    relu(X W1) W2 + X computed by the oracle's loop GEMM."""
    import run_mlp_search as MS
    ins = MS.mlp_inputs(8, 16, 24, "fp32", seed=5, device="cpu")
    got = MS.mlp_reference("ln")(ins).double().numpy()
    assert np.abs(got.mean(1)).max() < 1e-6
    assert np.abs(got.var(1) - 1.0).max() < 1e-3
    x, w1, w2 = (ins[n].double().numpy() for n in ("X", "W1", "W2"))
    r = O.matmul_loop(np.maximum(O.matmul_loop(x, w1), 0), w2) + x
    want = (r - r.mean(1, keepdims=True)) / np.sqrt(r.var(1, keepdims=True) + 1e-5)
    assert np.abs(got - want).max() < 1e-4
