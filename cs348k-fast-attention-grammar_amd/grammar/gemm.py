"""Python face of the hand-written CDNA4 GEMM with fused epilogue (gr_gemm)
and the two-GEMM MLP block (gr_mlp_fwd).

`gemm(a, b)` computes act(alpha * a @ b) for fp16/bf16 GPU tensors (fp32
accumulate) or fp32 ones (on the fp32 matrix cores; M and N multiples of 32),
batched over leading dimensions -- the grammar's matmul stage with its mulc and
relu/silu epilogue (grammar/kernel_ast.py:168-223). `mlp_fwd(x, w1, w2)` is
Y = SiLU(X W1) W2, the MLP block of run_mlp_search.py:42-127 with silu as
its activation.

There is no CPU path: CPU tensors or a missing library raise.
"""
from __future__ import annotations

import ctypes

from . import runtime as rt

EPILOGUES = {"none": 0, "relu": 1, "silu": 2}
TILES = ((128, 128), (256, 128), (128, 256), (256, 256))
K_TILE = {(128, 128): 64, (256, 128): 32, (128, 256): 32, (256, 256): 64}


def _batch_view(t, name):
    """(batch, rows, cols, batch stride, row stride) of a >=2-D tensor whose
    leading dims collapse into one uniformly strided batch axis."""
    if t.dim() < 2:
        raise ValueError(f"gemm: {name} must be at least 2-D")
    if t.stride(-1) != 1:
        raise ValueError(f"gemm: {name} must have unit stride on its last dimension")
    lead = t.shape[:-2]
    batch = 1
    for n in lead:
        batch *= int(n)
    if t.dim() == 2 or batch == 1:
        sb = 0
    else:
        sb = int(t.stride(t.dim() - 3))
        # all leading dims must collapse onto a single stride
        expect = sb
        for d in range(t.dim() - 3, -1, -1):
            if t.shape[d] != 1 and t.stride(d) != expect:
                raise ValueError(f"gemm: leading dimensions of {name} do not collapse into one batch axis")
            expect *= int(t.shape[d])
    return batch, int(t.shape[-2]), int(t.shape[-1]), sb, int(t.stride(-2))


def gemm(a, b, *, epilogue: str = "none", alpha: float = 1.0, b_kmajor: bool = False,
         block_m: int = 0, block_n: int = 0, out=None, stream=None):
    """act(alpha * a @ b) on the MI355X, fp32 accumulate.

    a: [..., M, K]; b: [..., K, N], or [..., N, K] with b_kmajor=True (b used
    transposed). Leading dims are a batch (b may have none: broadcast).
    Returns [..., M, N] in a's dtype (or writes `out`)."""
    import torch
    for name, t in (("a", a), ("b", b)):
        if not t.is_cuda:
            raise ValueError(f"gemm: {name} must be a GPU tensor (no CPU path)")
    if a.dtype != b.dtype:
        raise ValueError("gemm: a and b must share a dtype")
    if epilogue not in EPILOGUES:
        raise ValueError(f"gemm: epilogue must be one of {sorted(EPILOGUES)}")
    za, M, K, a_sb, a_sm = _batch_view(a, "a")
    zb, r, c, b_sb, b_s = _batch_view(b, "b")
    Kb, N = (c, r) if b_kmajor else (r, c)
    if Kb != K:
        raise ValueError(f"gemm: contraction mismatch {tuple(a.shape)} x {tuple(b.shape)}")
    if zb not in (1, za):
        raise ValueError("gemm: b's batch must be 1 or match a's")
    if zb == 1:
        b_sb = 0
    shape = tuple(a.shape[:-2]) + (M, N)
    if out is None:
        out = torch.empty(shape, dtype=a.dtype, device=a.device)
    elif tuple(out.shape) != shape or out.dtype != a.dtype:
        raise ValueError("gemm: bad `out` tensor")
    zc, _, _, c_sb, c_sm = _batch_view(out, "out")
    rc = rt.lib().gr_gemm(
        ctypes.c_void_p(a.data_ptr()), ctypes.c_void_p(b.data_ptr()), ctypes.c_void_p(out.data_ptr()),
        rt.dtype_code(a.dtype), za, M, N, K, rt._ll2(a_sb, a_sm), rt._ll2(b_sb, b_s), rt._ll2(c_sb, c_sm),
        int(bool(b_kmajor)), EPILOGUES[epilogue], float(alpha), int(block_m), int(block_n),
        rt._stream_ptr(stream))
    rt.check(rc, "gr_gemm")
    return out


def mlp_fwd(x, w1, w2, *, block_m: int = 0, block_n: int = 0, h=None, out=None, stream=None):
    """Y = SiLU(X @ W1) @ W2 with X [M, D], W1 [D, F], W2 [F, D] contiguous
    fp16/bf16 GPU tensors. `h` ([M, F]) is the intermediate buffer (allocated
    if not given). Returns Y [M, D]."""
    import torch
    for name, t in (("x", x), ("w1", w1), ("w2", w2)):
        if not t.is_cuda:
            raise ValueError(f"mlp_fwd: {name} must be a GPU tensor (no CPU path)")
        if t.dim() != 2 or not t.is_contiguous() or t.dtype != x.dtype:
            raise ValueError(f"mlp_fwd: {name} must be a contiguous 2-D tensor of x's dtype")
    M, D = x.shape
    F = w1.shape[1]
    if tuple(w1.shape) != (D, F) or tuple(w2.shape) != (F, D):
        raise ValueError(f"mlp_fwd: shapes x{tuple(x.shape)} w1{tuple(w1.shape)} w2{tuple(w2.shape)}")
    if h is None:
        h = torch.empty((M, F), dtype=x.dtype, device=x.device)
    if out is None:
        out = torch.empty((M, D), dtype=x.dtype, device=x.device)
    for name, t, shp in (("h", h, (M, F)), ("out", out, (M, D))):
        if tuple(t.shape) != shp or not t.is_contiguous() or t.dtype != x.dtype:
            raise ValueError(f"mlp_fwd: bad `{name}` tensor")
    rc = rt.lib().gr_mlp_fwd(
        ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(w1.data_ptr()), ctypes.c_void_p(w2.data_ptr()),
        ctypes.c_void_p(h.data_ptr()), ctypes.c_void_p(out.data_ptr()), rt.dtype_code(x.dtype),
        M, D, F, int(block_m), int(block_n), rt._stream_ptr(stream))
    rt.check(rc, "gr_mlp_fwd")
    return out


def gemm_flops(M: int, N: int, K: int, batch: int = 1) -> int:
    return 2 * batch * M * N * K


def mlp_flops(M: int, D: int, F: int) -> int:
    """Two GEMMs: 2*M*D*F each."""
    return 4 * M * D * F
