"""Staged naive attention on the CPU in torch fp32 -- the reported CPU baseline.
Test infrastructure only (imported by tests/ and bench.py's cpu_baseline leg).

Follows the stage structure of pytorch-naive.py:23-65 -- every intermediate
materialised as a full tensor -- with the intended math (row MAX at :48,
keepdim broadcasts at :51/:60), batched over B and H. Pinned against the
numpy oracle's fused attention in tests/test_oracle.py.
"""
from __future__ import annotations

import math


def staged_attention(q, kt, v, scale: float | None = None, causal: bool = False):
    """q, v: [B, H, N, d] fp32 CPU tensors; kt: [B, H, d, N]."""
    import torch
    d = q.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    scores = q @ kt                                   # S  = Q @ KT
    scores = scores * scale                           # Ss = S * 1/sqrt(d)
    if causal:
        n = scores.shape[-1]
        scores = scores.masked_fill(torch.triu(torch.ones(n, n, dtype=torch.bool), 1), float("-inf"))
    mx = torch.amax(scores, dim=-1, keepdim=True)     # mx = rowmax_j(Ss)
    sb = scores - mx                                  # sb = Ss - mx
    e = torch.exp(sb)                                 # e  = exp(sb)
    sm = torch.sum(e, dim=-1, keepdim=True)           # sm = rowsum_j(e)
    P = e / sm                                        # P  = e / sm
    return P @ v                                      # O  = P @ V
