"""Attention / MLP oracle (numpy, CPU) -- test infrastructure only.

Reference math restated here:
  * softmax(Q K^T / sqrt(d)) V with a row-max shift:
      run_attention_search.py:176-180 (verify), test_renderer.py:512-523
      (_np_softmax / _attention_ref). K may be passed transposed (KT[d, N]) as
      the reference's programs take it (run_attention_search.py:82-84).
  * causal variant: the same with -inf above the diagonal (key > query).
  * the 8-stage atomic decomposition S, Ss, mx, sb, e, sm, P, O of
      run_attention_search.py:49-85 / pytorch-naive.py:23-65 -- with the two
      pytorch-naive bugs fixed (pytorch-naive.py:48 uses a row SUM where a row
      MAX is meant, and :51/:60 broadcast a keepdim-less [N] vector along the
      wrong axis). Stage structure is kept; the math is the intended one.
  * SiLU MLP Y = SiLU(X W1) W2, SiLU(x) = x / (1 + e^-x) (
      the reference MLP driver's relu/residual/LayerNorm variant is
      run_mlp_search.py:138-149).

Pinning (tests/test_oracle.py): float64 brute force on tiny shapes; row sums
of P equal 1; O within the per-column [min V, max V] hull; Q = 0 gives the
column mean of V (prefix mean for causal); N = 1 gives O = V; key/value
permutation invariance; per-row score shift invariance; staged == fused;
MLP against a float64 loop GEMM and the closed-form SiLU at known points.
The backward (attention_backward, attention_lse) is pinned against central
finite differences of sum(O * dO) and of the log-sum-exp in float64.
"""
from __future__ import annotations

import math

import numpy as np


def softmax_rows(s: np.ndarray) -> np.ndarray:
    """Row softmax over the last axis with the max shift (test_renderer.py:512-514)."""
    m = s.max(axis=-1, keepdims=True)
    e = np.exp(s - m)
    return e / e.sum(axis=-1, keepdims=True)


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, *, causal: bool = False,
              scale: float | None = None, k_transposed: bool = False,
              dtype=np.float32) -> np.ndarray:
    """O = softmax(scale * Q K^T [causal]) V over the last two axes.

    q, v: [..., N, d]; k: [..., N, d] (or [..., d, N] if k_transposed).
    Computed in `dtype` (float32 by default; float64 for pinning), one
    leading-index slice at a time to bound memory at large N."""
    q = np.asarray(q, dtype=dtype)
    k = np.asarray(k, dtype=dtype)
    v = np.asarray(v, dtype=dtype)
    d = q.shape[-1]
    n = q.shape[-2]
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    kt = k if k_transposed else np.swapaxes(k, -1, -2)
    lead = q.shape[:-2]
    out = np.empty(lead + (n, v.shape[-1]), dtype=dtype)
    mask = np.triu(np.ones((n, n), dtype=bool), k=1) if causal else None
    for idx in np.ndindex(*lead):
        s = (q[idx] @ kt[idx]) * dtype(scale)
        if mask is not None:
            s = np.where(mask, -np.inf, s)
        out[idx] = softmax_rows(s) @ v[idx]
    return out


def attention_bruteforce(q, k, v, *, causal: bool = False, scale: float | None = None) -> np.ndarray:
    """Scalar-loop float64 attention for tiny shapes: every dot product,
    exponential and normalisation spelled out, with no max shift (exact
    arithmetic makes the shift irrelevant)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    n, d = q.shape[-2], q.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    out = np.zeros(q.shape[:-1] + (v.shape[-1],))
    for idx in np.ndindex(*q.shape[:-2]):
        for i in range(n):
            w = []
            for j in range(n):
                if causal and j > i:
                    w.append(0.0)
                    continue
                dot = 0.0
                for t in range(d):
                    dot += q[idx + (i, t)] * k[idx + (j, t)]
                w.append(math.exp(scale * dot))
            z = sum(w)
            for c in range(v.shape[-1]):
                acc = 0.0
                for j in range(n):
                    acc += w[j] * v[idx + (j, c)]
                out[idx + (i, c)] = acc / z
    return out


def attention_staged(q, kt, v, *, scale: float | None = None, causal: bool = False,
                     dtype=np.float32) -> dict:
    """The eight materialised stages of run_attention_search.py:49-85 (and the
    intended pytorch-naive.py:23-65), each a full tensor. Returns every stage
    so tests can check intermediate tensors of grammar programs too."""
    q = np.asarray(q, dtype=dtype)
    kt = np.asarray(kt, dtype=dtype)
    v = np.asarray(v, dtype=dtype)
    d = q.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    S = q @ kt                                        # S  = Q @ KT       [N,N]
    Ss = S * dtype(scale)                             # Ss = S * 1/sqrt(d)
    if causal:
        n = Ss.shape[-1]
        Ss = np.where(np.triu(np.ones((n, n), dtype=bool), k=1), -np.inf, Ss)
    mx = Ss.max(axis=-1, keepdims=True)               # mx = rowmax_j(Ss) [N,1]
    sb = Ss - mx                                      # sb = Ss - mx (broadcast)
    e = np.exp(sb)                                    # e  = exp(sb)
    sm = e.sum(axis=-1, keepdims=True)                # sm = rowsum_j(e)  [N,1]
    P = e / sm                                        # P  = e / sm (broadcast)
    O = P @ v                                         # O  = P @ V        [N,d]
    return {"S": S, "Ss": Ss, "mx": mx, "sb": sb, "e": e, "sm": sm, "P": P, "O": O}


def attention_lse(q, k, *, causal: bool = False, scale: float | None = None, dtype=np.float64) -> np.ndarray:
    """Row log-sum-exp of the scaled (masked) scores, natural log: the
    per-query statistic a training forward keeps for the backward pass.
    (No counterpart in the reference, which has no backward.)"""
    q = np.asarray(q, dtype=dtype)
    k = np.asarray(k, dtype=dtype)
    d, n = q.shape[-1], q.shape[-2]
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    s = (q @ np.swapaxes(k, -1, -2)) * scale
    if causal:
        s = np.where(np.triu(np.ones((n, k.shape[-2]), dtype=bool), k=1), -np.inf, s)
    m = s.max(axis=-1, keepdims=True)
    return (m + np.log(np.exp(s - m).sum(axis=-1, keepdims=True)))[..., 0]


def attention_backward(q, k, v, do, *, causal: bool = False, scale: float | None = None,
                       dtype=np.float64) -> tuple:
    """Gradients (dQ, dK, dV) of sum(O * dO) for O = softmax(scale Q K^T
    [causal]) V, from the closed form: P = softmax(S), dV = P^T dO,
    dP = dO V^T, dS = P * (dP - rowsum(dP * P)), dQ = scale dS K,
    dK = scale dS^T Q. rowsum(dP * P) equals rowsum(dO * O). (No
    counterpart in the reference, which has no backward.)"""
    q, k, v, do = (np.asarray(t, dtype=dtype) for t in (q, k, v, do))
    d, n = q.shape[-1], q.shape[-2]
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    s = (q @ np.swapaxes(k, -1, -2)) * scale
    if causal:
        s = np.where(np.triu(np.ones((n, k.shape[-2]), dtype=bool), k=1), -np.inf, s)
    p = softmax_rows(s)
    o = p @ v
    dv = np.swapaxes(p, -1, -2) @ do
    dp = do @ np.swapaxes(v, -1, -2)
    delta = (do * o).sum(axis=-1, keepdims=True)
    ds = p * (dp - delta)
    dq = scale * (ds @ k)
    dk = scale * (np.swapaxes(ds, -1, -2) @ q)
    return dq, dk, dv


def silu(x):
    x = np.asarray(x)
    return x / (1.0 + np.exp(-x))


def mlp_silu(x, w1, w2, dtype=np.float32) -> np.ndarray:
    """Y = SiLU(X @ W1) @ W2, computed in `dtype`."""
    x = np.asarray(x, dtype=dtype)
    h = x @ np.asarray(w1, dtype=dtype)
    return silu(h).astype(dtype) @ np.asarray(w2, dtype=dtype)


def matmul_loop(a, b) -> np.ndarray:
    """Triple-loop float64 GEMM for tiny shapes (pins the BLAS path)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    out = np.zeros((m, n))
    for i in range(m):
        for j in range(n):
            acc = 0.0
            for t in range(k):
                acc += a[i, t] * b[t, j]
            out[i, j] = acc
    return out


def errors(got, ref) -> tuple[float, float]:
    """(max-abs, mean-abs) error of `got` against `ref`, in float64."""
    g = np.asarray(got, dtype=np.float64)
    r = np.asarray(ref, dtype=np.float64)
    d = np.abs(g - r)
    return float(d.max()), float(d.mean())


# Tolerance of every fp16/bf16 variant against the fp32 oracle (BASELINE.json
# north_star): max-abs <= 2e-2 and mean-abs <= 2e-3.
MAX_ABS_TOL = 2e-2
MEAN_ABS_TOL = 2e-3


def within_tolerance(got, ref, max_abs: float = MAX_ABS_TOL, mean_abs: float = MEAN_ABS_TOL) -> bool:
    mx, mn = errors(got, ref)
    return bool(np.isfinite(np.asarray(got, dtype=np.float64)).all() and mx <= max_abs and mn <= mean_abs)
