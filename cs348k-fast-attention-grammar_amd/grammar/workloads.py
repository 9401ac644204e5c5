"""The benchmark configurations (BASELINE.json `configs`) and their seeded
synthetic inputs.

Inputs are drawn with torch.Generator('cpu').manual_seed(seed) as fp32 N(0,1),
scaled, rounded to the storage dtype, and only then moved to the GPU, so the
CPU oracle and the GPU kernels see bit-identical values.
"""
from __future__ import annotations

import math
from dataclasses import dataclass


@dataclass(frozen=True)
class AttnConfig:
    name: str
    B: int
    H: int
    N: int
    D: int
    dtype: str            # "fp32" | "fp16" | "bf16"
    causal: bool = False
    input_scale: float = 1.0

    @property
    def flops(self) -> int:
        """4*B*H*N^2*D, halved when causal (old/benchmark.py:354-355)."""
        f = 4 * self.B * self.H * self.N * self.N * self.D
        return f // 2 if self.causal else f

    @property
    def io_bytes(self) -> int:
        eb = 4 if self.dtype == "fp32" else 2
        return 4 * self.B * self.H * self.N * self.D * eb


@dataclass(frozen=True)
class MlpConfig:
    name: str
    M: int
    Dm: int
    Hd: int
    dtype: str = "fp16"

    @property
    def flops(self) -> int:
        return 2 * self.M * self.Dm * self.Hd * 2

    @property
    def io_bytes(self) -> int:
        return 2 * (self.M * self.Dm * 2 + 2 * self.Dm * self.Hd)


C1 = AttnConfig("C1", 1, 4, 256, 64, "fp32")
C2 = AttnConfig("C2", 4, 16, 1024, 64, "fp16")
C3 = AttnConfig("C3", 2, 32, 4096, 128, "bf16", causal=True, input_scale=0.5)
C4 = MlpConfig("C4", 8192, 4096, 11008, "fp16")
CONFIGS = {c.name: c for c in (C1, C2, C3, C4)}


def torch_dtype(name: str):
    import torch
    return {"fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}[name]


def attention_inputs(cfg: AttnConfig, seed: int = 0, device: str | None = None, dtype: str | None = None,
                     k_transposed: bool = False):
    """(q, k, v) of shape [B, H, N, D] (k as [B, H, D, N] if k_transposed),
    drawn Q, K, V in that order from one seeded CPU generator."""
    import torch
    g = torch.Generator("cpu").manual_seed(seed)
    shape = (cfg.B, cfg.H, cfg.N, cfg.D)
    td = torch_dtype(dtype or cfg.dtype)
    out = []
    for _ in range(3):
        t = torch.randn(shape, generator=g, dtype=torch.float32)
        if cfg.input_scale != 1.0:
            t = t * cfg.input_scale
        out.append(t.to(td))
    q, k, v = out
    if k_transposed:
        k = k.transpose(-1, -2).contiguous()
    if device is not None:
        q, k, v = q.to(device), k.to(device), v.to(device)
    return q, k, v


def mlp_inputs(cfg: MlpConfig, seed: int = 0, device: str | None = None):
    """(x, w1, w2): X ~ N(0,1) [M, Dm]; W1 ~ N(0,1)/sqrt(Dm) [Dm, Hd];
    W2 ~ N(0,1)/sqrt(Hd) [Hd, Dm] (std = 1/sqrt(fan_in)), rounded to fp16."""
    import torch
    g = torch.Generator("cpu").manual_seed(seed)
    td = torch_dtype(cfg.dtype)
    x = torch.randn((cfg.M, cfg.Dm), generator=g, dtype=torch.float32).to(td)
    w1 = (torch.randn((cfg.Dm, cfg.Hd), generator=g, dtype=torch.float32) / math.sqrt(cfg.Dm)).to(td)
    w2 = (torch.randn((cfg.Hd, cfg.Dm), generator=g, dtype=torch.float32) / math.sqrt(cfg.Hd)).to(td)
    if device is not None:
        x, w1, w2 = x.to(device), w1.to(device), w2.to(device)
    return x, w1, w2
