"""The C-ABI library loads on the CPU host and exports every function that
include/grammar_rt.h declares (no compute calls: there is no GPU here)."""
import ctypes
import os
import re

from conftest import REPO

HEADER = os.path.join(REPO, "include", "grammar_rt.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b(gr_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_header_declares_the_runtime_surface():
    names = declared_functions()
    for must in ("gr_compile", "gr_module_load", "gr_get_kernel", "gr_launch", "gr_plan_time",
                 "gr_attn_fwd", "gr_last_error"):
        assert must in names


def test_library_exports_every_declared_symbol():
    from grammar import runtime as rt
    L = rt.lib()
    missing = [n for n in declared_functions() if not hasattr(L, n)]
    assert not missing, f"declared but not exported: {missing}"
    assert set(rt.EXPORTED) == set(declared_functions())


def test_version_string_and_error_slot():
    from grammar import runtime as rt
    assert rt.version().startswith("gfx950 hiprtc")
    assert isinstance(rt.last_error(), str)


def test_hiprtc_compiles_on_the_host():
    # hiprtc needs no device: compile a tiny gfx950 kernel through the ABI.
    from grammar import runtime as rt
    code = rt.compile_source('#include "gr_common.h"\n'
                             'extern "C" __global__ void k(float* x) { x[threadIdx.x] = gr_exp2(1.0f); }\n')
    assert len(code) > 1000 and code[:4] == b"\x7fELF"


def test_compile_error_is_reported():
    from grammar import runtime as rt
    import pytest
    with pytest.raises(rt.CompileError) as ei:
        rt.compile_source('extern "C" __global__ void k(float* x) { this is not c++; }\n')
    assert "error" in str(ei.value).lower()


def test_null_arguments_are_rejected_without_a_device():
    from grammar import runtime as rt
    L = rt.lib()
    rc = L.gr_attn_fwd(None, None, None, None, 1, 1, 1, 128, 64, rt._ll3(0, 0, 0), rt._ll3(0, 0, 0),
                       rt._ll3(0, 0, 0), rt._ll3(0, 0, 0), 0, 0, ctypes.c_float(0.125), 0, 0, None)
    assert rc == rt.GR_E_ARG and "null" in rt.last_error()


def test_noalloc_default_split_fits_the_scratch_array():
    """The split gr_attn_decode_noalloc is given by default never needs more
    partials than the library's scratch array holds (host-side sizing only)."""
    from grammar import runtime as rt
    from grammar.attention import decode_splits, decode_splits_noalloc
    L = rt.lib()
    for B, H, Nq, N, D in ((1, 64, 128, 4096, 128), (1, 32, 64, 8192, 128), (2, 3, 1, 4096, 64),
                           (4, 16, 1, 8192, 128), (8, 64, 4, 2048, 128)):
        s = decode_splits_noalloc(B, H, Nq, N, D)
        assert 1 <= s <= decode_splits(B, H, Nq, N)
        assert s == 1 or int(L.gr_attn_decode_workspace(B, H, Nq, D, s)) <= rt.DECODE_SCRATCH_BYTES
    # the shape the usual split would overflow: 8 parts need 34 MB, so it is lowered
    assert decode_splits(1, 64, 128, 4096) == 8
    assert int(L.gr_attn_decode_workspace(1, 64, 128, 128, 8)) > rt.DECODE_SCRATCH_BYTES
    assert decode_splits_noalloc(1, 64, 128, 4096, 128) < 8
