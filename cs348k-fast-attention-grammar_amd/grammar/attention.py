"""Python face of the hand-written CDNA4 attention forward (gr_attn_fwd).

`flash_attention_fwd(q, k, v)` computes softmax(scale * q k^T [causal]) v for
[B, H, N, D] fp16/bf16 tensors (or fp32 ones, non-causal, on the fp32 matrix
cores) on the GPU -- the same math as the reference's
attention module contract `fn(KT, Q, V)` (pytorch-naive.py:23-65,
run_attention_search.py:169-181) and its SDPA reference point
(flash-attn2-sota.py:41-62), batched over B and H.

There is no CPU path: CPU tensors or a missing library raise.
"""
from __future__ import annotations

import ctypes
import math

from . import runtime as rt


def _strides3(t, dims=(0, 1, 2)) -> "ctypes.Array":
    return rt._ll3(*(int(t.stride(d)) for d in dims))


def default_tiles(N: int, D: int, dtype: str | None = None, causal: bool = False) -> tuple:
    """(block_m, block_n) of the flash body's largest tiles: the largest query
    tile of 256 / 128 / 64 dividing N, and 128 keys per tile at D = 64 when
    they divide N, else 64 or 32. With the dtype given, what gr_attn_fwd
    picks for block_m = block_n = 0: the same, except 256 x 64 where the
    two-wave body applies (fp16, D = 64, non-causal, N a multiple of 256)."""
    bm = 256 if N % 256 == 0 else 128 if N % 128 == 0 else 64
    if dtype == "fp16" and D == 64 and not causal and N % 256 == 0:
        return bm, 64
    bn = 128 if (D == 64 and N % 128 == 0) else 64 if N % 64 == 0 else 32
    return bm, bn


def bind_flash_attention(q, k, v, *, causal: bool = False, scale: float | None = None,
                         k_transposed: bool = False, block_m: int = 0, block_n: int = 0,
                         out=None, stream=None):
    """Validate the operands once and return (launch, out): launch() enqueues
    gr_attn_fwd with the pre-packed C arguments (no per-call checks or
    allocation, for launch-bound loops such as a timing loop); out is the
    [B, H, N, D] result tensor it writes. Arguments as flash_attention_fwd."""
    import torch
    for name, t in (("q", q), ("k", k), ("v", v)):
        if not t.is_cuda:
            raise ValueError(f"flash_attention_fwd: {name} must be a GPU tensor (no CPU path)")
        if t.dtype != q.dtype:
            raise ValueError("flash_attention_fwd: q, k, v must share a dtype")
        if t.dim() != 4:
            raise ValueError(f"flash_attention_fwd: {name} must be 4-D")
    B, H, N, D = q.shape
    if tuple(v.shape) != (B, H, N, D):
        raise ValueError(f"flash_attention_fwd: v shape {tuple(v.shape)} != q shape {tuple(q.shape)}")
    want_k = (B, H, D, N) if k_transposed else (B, H, N, D)
    if tuple(k.shape) != want_k:
        raise ValueError(f"flash_attention_fwd: k shape {tuple(k.shape)} != {want_k}")
    if q.stride(3) != 1 or v.stride(3) != 1 or k.stride(3) != 1:
        raise ValueError("flash_attention_fwd: innermost dimension must be contiguous")
    if out is None:
        out = torch.empty((B, H, N, D), dtype=q.dtype, device=q.device)
    elif tuple(out.shape) != (B, H, N, D) or out.dtype != q.dtype or out.stride(3) != 1:
        raise ValueError("flash_attention_fwd: bad `out` tensor")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    fn = rt.lib().gr_attn_fwd
    args = (ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(k.data_ptr()), ctypes.c_void_p(v.data_ptr()),
            ctypes.c_void_p(out.data_ptr()), rt.dtype_code(q.dtype), B, H, N, D,
            _strides3(q), _strides3(k), _strides3(v), _strides3(out),
            int(bool(k_transposed)), int(bool(causal)), float(scale), int(block_m), int(block_n),
            rt._stream_ptr(stream))
    keep = (q, k, v, out)   # the tensors stay alive as long as the launcher

    def launch():
        rt.check(fn(*args), "gr_attn_fwd")
        return keep[3]
    return launch, out


def flash_attention_fwd(q, k, v, *, causal: bool = False, scale: float | None = None,
                        k_transposed: bool = False, block_m: int = 0, block_n: int = 0,
                        out=None, stream=None):
    """O = softmax(scale * Q K^T [+ causal mask]) V on the MI355X.

    q, v: [B, H, N, D]; k: [B, H, N, D], or [B, H, D, N] when k_transposed.
    All three share dtype (float16 or bfloat16) and live on the GPU. Returns a
    new [B, H, N, D] tensor (or writes `out`)."""
    launch, out = bind_flash_attention(q, k, v, causal=causal, scale=scale, k_transposed=k_transposed,
                                       block_m=block_m, block_n=block_n, out=out, stream=stream)
    launch()
    return out


def bind_flash_attention_train(q, k, v, *, causal: bool = False, scale: float | None = None,
                               block_m: int = 0, block_n: int = 0, out=None, lse=None, stream=None):
    """bind_flash_attention for gr_attn_fwd_train: returns (launch, out, lse),
    launch() enqueueing the forward that also writes the row log-sum-exp of
    the scaled scores ([B, H, N] fp32, natural log). K in [B, H, N, D]."""
    import torch
    _, out = bind_flash_attention(q, k, v, causal=causal, scale=scale, block_m=block_m, block_n=block_n,
                                  out=out, stream=stream)
    B, H, N, D = q.shape
    if lse is None:
        lse = torch.empty((B, H, N), dtype=torch.float32, device=q.device)
    elif tuple(lse.shape) != (B, H, N) or lse.dtype != torch.float32 or not lse.is_contiguous():
        raise ValueError("flash_attention_fwd_train: bad `lse` tensor")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    fn = rt.lib().gr_attn_fwd_train
    args = (ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(k.data_ptr()), ctypes.c_void_p(v.data_ptr()),
            ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(lse.data_ptr()), rt.dtype_code(q.dtype), B, H, N, D,
            _strides3(q), _strides3(k), _strides3(v), _strides3(out), 0, int(bool(causal)), float(scale),
            int(block_m), int(block_n), rt._stream_ptr(stream))
    keep = (q, k, v, out, lse)

    def launch():
        rt.check(fn(*args), "gr_attn_fwd_train")
        return keep[3], keep[4]
    return launch, out, lse


def flash_attention_fwd_train(q, k, v, *, causal: bool = False, scale: float | None = None,
                              block_m: int = 0, block_n: int = 0, out=None, lse=None, stream=None):
    """flash_attention_fwd that also returns the row log-sum-exp of the scaled
    scores ([B, H, N] fp32, natural log), kept for flash_attention_bwd.
    K in [B, H, N, D] layout. Returns (out, lse)."""
    launch, out, lse = bind_flash_attention_train(q, k, v, causal=causal, scale=scale, block_m=block_m,
                                                  block_n=block_n, out=out, lse=lse, stream=stream)
    launch()
    return out, lse


def bind_flash_attention_bwd(q, k, v, o, do, lse, *, causal: bool = False, scale: float | None = None,
                             workspace=None, grads=None, stream=None):
    """Validate once and return (launch, (dq, dk, dv)): launch() enqueues
    gr_attn_bwd with pre-packed C arguments. q, k, v, o, do: contiguous
    [B, H, N, D] fp16/bf16 GPU tensors of one dtype (the kernels take one
    stride set); lse: [B, H, N] float32 from the training forward; grads: an
    optional (dq, dk, dv) triple of such tensors to write."""
    import torch
    B, H, N, D = q.shape
    for name, t in (("q", q), ("k", k), ("v", v), ("o", o), ("do", do)):
        if tuple(t.shape) != (B, H, N, D) or t.dtype != q.dtype or not t.is_cuda:
            raise ValueError(f"flash_attention_bwd: {name} must match q ({tuple(q.shape)}, {q.dtype}, GPU)")
        if not t.is_contiguous():
            raise ValueError(f"flash_attention_bwd: {name} must be contiguous")
    if tuple(lse.shape) != (B, H, N) or lse.dtype != torch.float32 or not lse.is_contiguous():
        raise ValueError("flash_attention_bwd: lse must be a contiguous [B, H, N] float32 tensor")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    L = rt.lib()
    need = int(L.gr_attn_bwd_workspace(B, H, N, D))
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    elif workspace.numel() * workspace.element_size() < need:
        raise ValueError(f"flash_attention_bwd: workspace of {need} bytes needed")
    if grads is None:
        grads = (torch.empty_like(q), torch.empty_like(q), torch.empty_like(q))
    for t in grads:
        if tuple(t.shape) != (B, H, N, D) or t.dtype != q.dtype or not t.is_contiguous():
            raise ValueError("flash_attention_bwd: bad gradient tensor")
    dq, dk, dv = grads
    fn = L.gr_attn_bwd
    args = (ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(k.data_ptr()), ctypes.c_void_p(v.data_ptr()),
            ctypes.c_void_p(o.data_ptr()), ctypes.c_void_p(do.data_ptr()), ctypes.c_void_p(lse.data_ptr()),
            ctypes.c_void_p(dq.data_ptr()), ctypes.c_void_p(dk.data_ptr()), ctypes.c_void_p(dv.data_ptr()),
            rt.dtype_code(q.dtype), B, H, N, D, _strides3(q), int(bool(causal)), float(scale),
            ctypes.c_void_p(workspace.data_ptr()), need, rt._stream_ptr(stream))
    keep = (q, k, v, o, do, lse, workspace, grads)

    def launch():
        rt.check(fn(*args), "gr_attn_bwd")
        return keep[7]
    return launch, grads


def flash_attention_bwd(q, k, v, o, do, lse, *, causal: bool = False, scale: float | None = None,
                        workspace=None, stream=None):
    """dQ, dK, dV of sum(O * dO) for the attention forward that produced o and
    lse (flash_attention_fwd_train). q, k, v, o, do: [B, H, N, D] fp16/bf16
    on the GPU (made contiguous here: the kernel takes one stride set)."""
    q, k, v, o, do, lse = (t.contiguous() for t in (q, k, v, o, do, lse))
    launch, grads = bind_flash_attention_bwd(q, k, v, o, do, lse, causal=causal, scale=scale,
                                             workspace=workspace, stream=stream)
    launch()
    return grads


def _autograd_function():
    import torch

    class FlashAttention(torch.autograd.Function):
        @staticmethod
        def forward(ctx, q, k, v, causal, scale):
            q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
            o, lse = flash_attention_fwd_train(q, k, v, causal=causal, scale=scale)
            ctx.save_for_backward(q, k, v, o, lse)
            ctx.causal, ctx.scale = causal, scale
            return o

        @staticmethod
        def backward(ctx, do):
            q, k, v, o, lse = ctx.saved_tensors
            dq, dk, dv = flash_attention_bwd(q, k, v, o, do, lse, causal=ctx.causal, scale=ctx.scale)
            return dq, dk, dv, None, None
    return FlashAttention


_FLASH_FN = None


def flash_attention(q, k, v, *, causal: bool = False, scale: float | None = None):
    """Differentiable attention on the MI355X kernels: forward through
    gr_attn_fwd_train, backward through gr_attn_bwd (torch.autograd)."""
    global _FLASH_FN
    if _FLASH_FN is None:
        _FLASH_FN = _autograd_function()
    return _FLASH_FN.apply(q, k, v, causal, scale)


def decode_splits(B: int, H: int, Nq: int, N: int, cu_count: int = 256) -> int:
    """Key parts per query tile for gr_attn_decode. Up to 4 queries (the
    streaming kernel, 4 waves per workgroup): one workgroup per compute unit,
    each part keeping at least 512 keys. More (the flash body): enough
    workgroups for two per compute unit, each part keeping at least four
    64-key tiles."""
    if Nq <= 4:
        return max(1, min(-(-cu_count // (B * H)), N // 512))
    nw = 1 if Nq <= 32 else 2 if Nq <= 64 else 4
    tiles_q = B * H * -(-Nq // (32 * nw))
    want = -(-2 * cu_count // tiles_q)
    return max(1, min(want, N // 256 if N >= 256 else 1))


def decode_splits_noalloc(B: int, H: int, Nq: int, N: int, D: int, cu_count: int = 256) -> int:
    """decode_splits, lowered until the key parts' partials fit the library's
    scratch array (rt.DECODE_SCRATCH_BYTES), which gr_attn_decode_noalloc
    cannot grow. One part needs no scratch."""
    L = rt.lib()
    s = decode_splits(B, H, Nq, N, cu_count)
    while s > 1 and int(L.gr_attn_decode_workspace(B, H, Nq, D, s)) > rt.DECODE_SCRATCH_BYTES:
        s -= 1
    return s


def bind_flash_attention_decode(q, k, v, *, scale: float | None = None, splits: int = 0, out=None,
                                workspace=None, stream=None):
    """Validate once and return (launch, out) for gr_attn_decode, arguments
    pre-packed (as bind_flash_attention); see flash_attention_decode."""
    import torch
    for name, t in (("q", q), ("k", k), ("v", v)):
        if not t.is_cuda:
            raise ValueError(f"flash_attention_decode: {name} must be a GPU tensor (no CPU path)")
        if t.dtype != q.dtype or t.dim() != 4 or t.stride(3) != 1:
            raise ValueError(f"flash_attention_decode: {name} must be 4-D, q's dtype, unit stride on D")
    B, H, Nq, D = q.shape
    N = k.shape[2]
    if tuple(k.shape) != (B, H, N, D) or tuple(v.shape) != (B, H, N, D):
        raise ValueError(f"flash_attention_decode: k {tuple(k.shape)} / v {tuple(v.shape)} do not match q {tuple(q.shape)}")
    if out is None:
        out = torch.empty((B, H, Nq, D), dtype=q.dtype, device=q.device)
    elif tuple(out.shape) != (B, H, Nq, D) or out.dtype != q.dtype or out.stride(3) != 1:
        raise ValueError("flash_attention_decode: bad `out` tensor")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    L = rt.lib()
    if splits <= 0:
        splits = decode_splits(B, H, Nq, N, rt.device_info(q.device.index or 0)["cu_count"])
    need = int(L.gr_attn_decode_workspace(B, H, Nq, D, splits))
    if need and workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    elif need and workspace.numel() * workspace.element_size() < need:
        raise ValueError(f"flash_attention_decode: workspace of {need} bytes needed")
    fn = L.gr_attn_decode
    args = (ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(k.data_ptr()), ctypes.c_void_p(v.data_ptr()),
            ctypes.c_void_p(out.data_ptr()), rt.dtype_code(q.dtype), B, H, Nq, N, D,
            _strides3(q), _strides3(k), _strides3(v), _strides3(out), float(scale), int(splits),
            ctypes.c_void_p(workspace.data_ptr() if need else None), need, rt._stream_ptr(stream))
    keep = (q, k, v, out, workspace)

    def launch():
        rt.check(fn(*args), "gr_attn_decode")
        return keep[3]
    return launch, out


def bind_flash_attention_decode_noalloc(q, k, v, *, scale: float | None = None, splits: int = 0, out=None,
                                        stream=None):
    """(launch, out) for gr_attn_decode_noalloc: the decode launch with its
    key-split partials in the library's per-device scratch array, so neither
    the binding (given `out`) nor a launch allocates device memory. Launches
    that overlap on one device race on that array. Raises if the split needs
    more than rt.DECODE_SCRATCH_BYTES; splits = 0 picks the largest split
    decode_splits allows that fits it (decode_splits_noalloc)."""
    import torch
    for name, t in (("q", q), ("k", k), ("v", v)):
        if not t.is_cuda:
            raise ValueError(f"flash_attention_decode_noalloc: {name} must be a GPU tensor (no CPU path)")
        if t.dtype != q.dtype or t.dim() != 4 or t.stride(3) != 1:
            raise ValueError(f"flash_attention_decode_noalloc: {name} must be 4-D, q's dtype, unit stride on D")
    B, H, Nq, D = q.shape
    N = k.shape[2]
    if tuple(k.shape) != (B, H, N, D) or tuple(v.shape) != (B, H, N, D):
        raise ValueError("flash_attention_decode_noalloc: k / v do not match q")
    if out is None:
        out = torch.empty((B, H, Nq, D), dtype=q.dtype, device=q.device)
    elif tuple(out.shape) != (B, H, Nq, D) or out.dtype != q.dtype or out.stride(3) != 1:
        raise ValueError("flash_attention_decode_noalloc: bad `out` tensor")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    L = rt.lib()
    if splits <= 0:
        splits = decode_splits_noalloc(B, H, Nq, N, D, rt.device_info(q.device.index or 0)["cu_count"])
    fn = L.gr_attn_decode_noalloc
    args = (ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(k.data_ptr()), ctypes.c_void_p(v.data_ptr()),
            ctypes.c_void_p(out.data_ptr()), rt.dtype_code(q.dtype), B, H, Nq, N, D,
            _strides3(q), _strides3(k), _strides3(v), _strides3(out), float(scale), int(splits),
            rt._stream_ptr(stream))
    keep = (q, k, v, out)

    def launch():
        rt.check(fn(*args), "gr_attn_decode_noalloc")
        return keep[3]
    return launch, out


def flash_attention_decode(q, k, v, *, scale: float | None = None, splits: int = 0, out=None,
                           workspace=None, stream=None):
    """O = softmax(scale * Q K^T) V for Nq queries against N keys (non-causal):
    q [B, H, Nq, D], k and v [B, H, N, D] (N a multiple of 32), fp16/bf16 on
    the GPU. splits = 0 picks the key split (decode_splits); the workspace
    it needs is allocated here unless given."""
    launch, out = bind_flash_attention_decode(q, k, v, scale=scale, splits=splits, out=out,
                                              workspace=workspace, stream=stream)
    launch()
    return out


def attention_flops(B: int, H: int, N: int, D: int, causal: bool = False) -> int:
    """Algorithmic FLOPs of attention forward: 4*B*H*N^2*D (two GEMMs), halved
    for a causal mask (old/benchmark.py:354-355 defines the 4*B*H*S^2*D count)."""
    f = 4 * B * H * N * N * D
    return f // 2 if causal else f


def attention_io_bytes(B: int, H: int, N: int, D: int, elem_bytes: int = 2) -> int:
    """Minimal HBM traffic: read Q, K, V once and write O once."""
    return 4 * B * H * N * D * elem_bytes


def mfma32_selftest(a, b):
    """D = A[32,16] @ B[16,32] through one 32x32x16 MFMA with the operand and
    accumulator layout the kernels assume (fp16 in, fp32 out)."""
    import torch
    if a.shape != (32, 16) or b.shape != (16, 32) or a.dtype != torch.float16 or b.dtype != torch.float16:
        raise ValueError("mfma32_selftest: need fp16 A[32,16] and B[16,32]")
    a = a.contiguous()
    b = b.contiguous()
    d = torch.empty((32, 32), dtype=torch.float32, device=a.device)
    rt.check(rt.lib().gr_selftest_mfma32(ctypes.c_void_p(a.data_ptr()), ctypes.c_void_p(b.data_ptr()),
                                         ctypes.c_void_p(d.data_ptr()), rt._stream_ptr(None)),
             "gr_selftest_mfma32")
    return d
