"""gr_attn_decode_noalloc -- the decode launch with its key-split partials in
the library's per-device scratch array instead of a caller workspace (no
counterpart in the reference; for callers that cannot allocate). Called
through the C ABI, two calls in a row (the second on a smaller input), each
compared bit for bit with gr_attn_decode on the same inputs; a split larger
than the scratch array is refused before anything is launched."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import attention as O

pytestmark = pytest.mark.gpu


def _cuda():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    return torch.device("cuda:0")


def _inputs(B, H, Nq, N, D, dtype, seed):
    g = torch.Generator("cpu").manual_seed(seed)
    q = torch.randn((B, H, Nq, D), generator=g).to(dtype)
    k = torch.randn((B, H, N, D), generator=g).to(dtype)
    v = torch.randn((B, H, N, D), generator=g).to(dtype)
    return q, k, v


def _s3(t):
    from grammar import runtime as rt
    return rt._ll3(t.stride(0), t.stride(1), t.stride(2))


def _call(noalloc, q, k, v, o, splits, ws=None):
    """One launch through the C ABI; returns the status code."""
    from grammar import runtime as rt
    L = rt.lib()
    B, H, Nq, D = q.shape
    N = k.shape[2]
    head = (ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(k.data_ptr()), ctypes.c_void_p(v.data_ptr()),
            ctypes.c_void_p(o.data_ptr()), rt.dtype_code(q.dtype), B, H, Nq, N, D, _s3(q), _s3(k), _s3(v), _s3(o),
            ctypes.c_float(1.0 / D ** 0.5), splits)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if noalloc:
        return L.gr_attn_decode_noalloc(*head, stream)
    need = int(L.gr_attn_decode_workspace(B, H, Nq, D, splits))
    return L.gr_attn_decode(*head, ctypes.c_void_p(ws.data_ptr() if need else None), need, stream)


CASES = [
    # B, H, Nq, N, D, dtype, splits: the first is the larger input
    (4, 16, 1, 8192, 128, torch.bfloat16, 4),      # streaming kernel, 4 key parts
    (1, 2, 3, 1024, 64, torch.float16, 2),         # smaller: 3 queries, 2 parts
]


def test_noalloc_matches_decode_on_two_calls_in_a_row():
    dev = _cuda()
    from grammar import runtime as rt
    for i, (B, H, Nq, N, D, dt, splits) in enumerate(CASES):
        print(f"[case] noalloc call {i}: B{B} H{H} Nq{Nq} N{N} D{D} {dt} splits {splits}", flush=True)
        q, k, v = (t.to(dev) for t in _inputs(B, H, Nq, N, D, dt, seed=i))
        need = int(rt.lib().gr_attn_decode_workspace(B, H, Nq, D, splits))
        assert 0 < need <= rt.DECODE_SCRATCH_BYTES
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
        want = torch.full_like(q, float("nan"))
        got = torch.full_like(q, float("nan"))
        assert _call(False, q, k, v, want, splits, ws) == 0, rt.last_error()
        assert _call(True, q, k, v, got, splits) == 0, rt.last_error()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"call {i}: noalloc differs from gr_attn_decode"
        ref = O.attention(q.float().cpu().numpy(), k.float().cpu().numpy(), v.float().cpu().numpy())
        mx, mn = O.errors(got.float().cpu().numpy(), ref)
        assert np.isfinite(mx) and mx <= O.MAX_ABS_TOL and mn <= O.MEAN_ABS_TOL, (i, mx, mn)


def test_noalloc_flash_body_split_and_repeat():
    """More than 4 queries take the flash body with key parts; the scratch
    array keeps the previous call's contents, which must not leak in."""
    dev = _cuda()
    q, k, v = (t.to(dev) for t in _inputs(1, 2, 64, 2048, 64, torch.float16, seed=7))
    print("[case] noalloc flash body B1 H2 Nq64 N2048 D64 splits 4", flush=True)
    from grammar import runtime as rt
    ws = torch.empty(int(rt.lib().gr_attn_decode_workspace(1, 2, 64, 64, 4)), dtype=torch.uint8, device=dev)
    want = torch.empty_like(q)
    a, b = torch.empty_like(q), torch.empty_like(q)
    assert _call(False, q, k, v, want, 4, ws) == 0
    assert _call(True, q, k, v, a, 4) == 0
    assert _call(True, q, k, v, b, 4) == 0
    torch.cuda.synchronize()
    assert torch.equal(a, want) and torch.equal(b, want)


def test_noalloc_refuses_a_split_beyond_the_scratch_array():
    dev = _cuda()
    from grammar import runtime as rt
    B, H, Nq, N, D, splits = 8, 64, 4, 2048, 128, 32
    assert int(rt.lib().gr_attn_decode_workspace(B, H, Nq, D, splits)) > rt.DECODE_SCRATCH_BYTES
    q = torch.zeros((B, H, Nq, D), dtype=torch.bfloat16, device=dev)
    kv = torch.zeros((B, H, N, D), dtype=torch.bfloat16, device=dev)
    o = torch.zeros_like(q)
    print("[case] noalloc oversize split refused", flush=True)
    rc = _call(True, q, kv, kv, o, splits)
    assert rc == rt.GR_E_ARG
    assert "maximum" in rt.last_error()
    torch.cuda.synchronize()
    assert not o.any()          # nothing ran


def test_python_binding_uses_the_noalloc_entry():
    dev = _cuda()
    from grammar.attention import bind_flash_attention_decode, bind_flash_attention_decode_noalloc
    q, k, v = (t.to(dev) for t in _inputs(2, 3, 1, 4096, 64, torch.float16, seed=3))
    launch, out = bind_flash_attention_decode_noalloc(q, k, v)
    launch()
    ref_launch, ref_out = bind_flash_attention_decode(q, k, v)
    ref_launch()
    torch.cuda.synchronize()
    assert torch.equal(out, ref_out)


def test_default_split_fits_the_scratch_array():
    """splits = 0 picks the split for the scratch array: at B1 H64 Nq128 N4096
    D128 the usual decode split (8 parts, 34 MB of partials) would not fit,
    so the binding lowers it; the result equals gr_attn_decode at the same
    split bit for bit, and the oracle on sampled heads."""
    dev = _cuda()
    from grammar import runtime as rt
    from grammar.attention import bind_flash_attention_decode_noalloc, decode_splits, decode_splits_noalloc
    B, H, Nq, N, D = 1, 64, 128, 4096, 128
    cu = rt.device_info(0)["cu_count"]
    s_noalloc = decode_splits_noalloc(B, H, Nq, N, D, cu)
    L = rt.lib()
    assert int(L.gr_attn_decode_workspace(B, H, Nq, D, s_noalloc)) <= rt.DECODE_SCRATCH_BYTES
    print(f"[case] noalloc default split B{B} H{H} Nq{Nq} N{N} D{D}: decode_splits {decode_splits(B, H, Nq, N, cu)}, "
          f"noalloc {s_noalloc}", flush=True)
    q, k, v = (t.to(dev) for t in _inputs(B, H, Nq, N, D, torch.bfloat16, seed=5))
    launch, got = bind_flash_attention_decode_noalloc(q, k, v)
    launch()
    want = torch.empty_like(q)
    need = int(L.gr_attn_decode_workspace(B, H, Nq, D, s_noalloc))
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
    assert _call(False, q, k, v, want, s_noalloc, ws) == 0, rt.last_error()
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    for h in (0, 37, 63):
        ref = O.attention(q[0, h].float().cpu().numpy(), k[0, h].float().cpu().numpy(), v[0, h].float().cpu().numpy())
        mx, mn = O.errors(got[0, h].float().cpu().numpy(), ref)
        assert np.isfinite(mx) and mx <= O.MAX_ABS_TOL and mn <= O.MEAN_ABS_TOL, (h, mx, mn)
