"""ctypes binding of libgrammar_rt.so (include/grammar_rt.h).

This is the thin C-ABI layer between the Python grammar and the MI355X: hiprtc
compilation, code-object loading, launch plans and hipEvent timing, plus the
hand-written attention baseline. Tensors are PyTorch-ROCm tensors; only their
raw device pointers cross the boundary.

The library must have been built (build_native.py / __graft_entry__.build());
loading fails loudly otherwise -- there is no CPU fallback on this path.
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.dirname(_HERE)
LIB_PATH = os.path.join(PKG_ROOT, "lib", "libgrammar_rt.so")
CSRC_DIR = os.path.join(PKG_ROOT, "csrc")

GR_F32, GR_F16, GR_BF16 = 0, 1, 2
GR_TIME_BATCH, GR_TIME_MIN = 0, 1

GR_E_ARG, GR_E_COMPILE, GR_E_LOAD, GR_E_LAUNCH, GR_E_RUNTIME = -1, -2, -3, -4, -5


class GrError(RuntimeError):
    """A failure reported by libgrammar_rt (status code + message)."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[gr {code}] {msg}")
        self.code = code
        self.msg = msg


class CompileError(GrError):
    pass


_lib = None
_lock = threading.Lock()

_u32x3 = ctypes.c_uint32 * 3
_ll3 = ctypes.c_longlong * 3
_ll2 = ctypes.c_longlong * 2


def lib() -> ctypes.CDLL:
    """The loaded library (raises if it was never built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python __graft_entry__.py` "
                "or build_native.py before using the HIP path")
        # torch must bring its HIP runtime into the process first: when this
        # library is loaded first, /opt/rocm's libamdhip64 comes in ahead of
        # torch's bundled one and torch then reports "No HIP GPUs are available".
        import torch  # noqa: F401
        L = ctypes.CDLL(LIB_PATH)
        vp, sz, i32, u64p = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.POINTER(ctypes.c_uint64)
        L.gr_last_error.restype = ctypes.c_char_p
        L.gr_version.restype = ctypes.c_char_p
        L.gr_device_info.argtypes = [i32, ctypes.POINTER(ctypes.c_longlong)]
        L.gr_compile.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p), i32,
                                 ctypes.POINTER(vp), ctypes.POINTER(sz), ctypes.c_char_p, sz]
        L.gr_free_code.argtypes = [vp]
        L.gr_free_code.restype = None
        L.gr_module_load.argtypes = [vp, sz, ctypes.POINTER(vp)]
        L.gr_module_free.argtypes = [vp]
        L.gr_module_free.restype = None
        L.gr_get_kernel.argtypes = [vp, ctypes.c_char_p, ctypes.POINTER(vp)]
        L.gr_launch.argtypes = [vp, _u32x3, _u32x3, ctypes.c_uint32, vp, u64p, i32]
        L.gr_plan_create.argtypes = [i32, ctypes.POINTER(vp)]
        L.gr_plan_set_step.argtypes = [vp, i32, vp, _u32x3, _u32x3, ctypes.c_uint32, u64p, i32]
        L.gr_plan_run.argtypes = [vp, vp]
        L.gr_plan_free.argtypes = [vp]
        L.gr_plan_free.restype = None
        L.gr_plan_time.argtypes = [vp, vp, i32, i32, i32, ctypes.POINTER(ctypes.c_float)]
        L.gr_attn_fwd.argtypes = [vp, vp, vp, vp, i32, i32, i32, i32, i32, _ll3, _ll3, _ll3, _ll3,
                                  i32, i32, ctypes.c_float, i32, i32, vp]
        L.gr_selftest_mfma32.argtypes = [vp, vp, vp, vp]
        L.gr_gemm.argtypes = [vp, vp, vp, i32, i32, i32, i32, i32, _ll2, _ll2, _ll2, i32, i32,
                              ctypes.c_float, i32, i32, vp]
        L.gr_mlp_fwd.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, vp]
        L.gr_attn_fwd_train.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, _ll3, _ll3, _ll3, _ll3,
                                        i32, i32, ctypes.c_float, i32, i32, vp]
        L.gr_attn_bwd_workspace.argtypes = [i32, i32, i32, i32]
        L.gr_attn_bwd_workspace.restype = ctypes.c_size_t
        L.gr_attn_bwd.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, _ll3, i32,
                                  ctypes.c_float, vp, ctypes.c_size_t, vp]
        L.gr_attn_decode_workspace.argtypes = [i32, i32, i32, i32, i32]
        L.gr_attn_decode_workspace.restype = ctypes.c_size_t
        L.gr_attn_decode.argtypes = [vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, _ll3, _ll3, _ll3, _ll3,
                                     ctypes.c_float, i32, vp, ctypes.c_size_t, vp]
        L.gr_attn_decode_noalloc.argtypes = [vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, _ll3, _ll3, _ll3, _ll3,
                                             ctypes.c_float, i32, vp]
        _lib = L
        return L


# Every symbol the C header declares; tests check the library exports them all.
EXPORTED = (
    "gr_last_error", "gr_version", "gr_device_info", "gr_compile", "gr_free_code",
    "gr_module_load", "gr_module_free", "gr_get_kernel", "gr_launch", "gr_plan_create",
    "gr_plan_set_step", "gr_plan_run", "gr_plan_free", "gr_plan_time", "gr_attn_fwd",
    "gr_selftest_mfma32", "gr_gemm", "gr_mlp_fwd", "gr_attn_decode_workspace", "gr_attn_decode",
    "gr_attn_fwd_train", "gr_attn_bwd_workspace", "gr_attn_bwd", "gr_attn_decode_noalloc",
)

# Bytes of the per-device scratch array behind gr_attn_decode_noalloc (GR_DECODE_SCRATCH_BYTES).
DECODE_SCRATCH_BYTES = 16 << 20


def last_error() -> str:
    return lib().gr_last_error().decode(errors="replace")


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        msg = last_error()
        raise (CompileError if rc == GR_E_COMPILE else GrError)(rc, f"{what}: {msg}" if what else msg)


def version() -> str:
    return lib().gr_version().decode()


def device_info(device: int = 0) -> dict:
    out = (ctypes.c_longlong * 5)()
    check(lib().gr_device_info(device, out), "gr_device_info")
    return {"cu_count": out[0], "lds_per_block": out[1], "wave_size": out[2],
            "clock_khz": out[3], "l2_bytes": out[4]}


def compile_source(src: str, name: str = "gr_module.hip", options: list[str] | None = None) -> bytes:
    """hiprtc-compile `src` for gfx950; returns the code object bytes.
    Thread-safe and GIL-free while compiling, so callers may compile many
    candidates concurrently from a thread pool."""
    L = lib()
    opts = ["-I" + CSRC_DIR] + list(options or [])
    arr = (ctypes.c_char_p * len(opts))(*[o.encode() for o in opts])
    code = ctypes.c_void_p()
    size = ctypes.c_size_t()
    log = ctypes.create_string_buffer(16384)
    rc = L.gr_compile(src.encode(), name.encode(), arr, len(opts), ctypes.byref(code), ctypes.byref(size),
                      log, len(log))
    if rc != 0:
        raise CompileError(rc, log.value.decode(errors="replace") or last_error())
    try:
        return ctypes.string_at(code, size.value)
    finally:
        L.gr_free_code(code)


class Kernel(ctypes.c_void_p):
    """A kernel handle; it holds a reference to its Module, so the code object
    stays loaded as long as the handle (or a Plan using it) is alive."""


class Module:
    """A loaded code object; kernels are looked up by extern "C" name."""

    def __init__(self, code: bytes):
        self._code = code
        h = ctypes.c_void_p()
        check(lib().gr_module_load(code, len(code), ctypes.byref(h)), "gr_module_load")
        self.handle = h
        self._kernels: dict[str, ctypes.c_void_p] = {}

    def kernel(self, name: str) -> Kernel:
        k = self._kernels.get(name)
        if k is None:
            if not self.handle:
                raise GrError(GR_E_ARG, "Module.kernel: module is closed")
            k = Kernel()
            check(lib().gr_get_kernel(self.handle, name.encode(), ctypes.byref(k)), f"gr_get_kernel({name})")
            k.module = self
            self._kernels[name] = k
        return k

    def close(self) -> None:
        if self.handle:
            lib().gr_module_free(self.handle)
            self.handle = None
            self._kernels.clear()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _stream_ptr(stream) -> ctypes.c_void_p:
    if stream is None:
        import torch
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream))


class Plan:
    """Ordered launches with bound pointer arguments (one generated module)."""

    def __init__(self, steps: list[tuple]):
        """steps: [(kernel_handle, grid(3), block(3), lds_bytes, [u64 args])]."""
        h = ctypes.c_void_p()
        check(lib().gr_plan_create(len(steps), ctypes.byref(h)), "gr_plan_create")
        self.handle = h
        self._kernels = [st[0] for st in steps]   # keep the kernels' modules loaded
        for i, (k, grid, block, lds, args) in enumerate(steps):
            arr = (ctypes.c_uint64 * max(1, len(args)))(*args)
            check(lib().gr_plan_set_step(h, i, k, _u32x3(*grid), _u32x3(*block), int(lds), arr, len(args)),
                  f"gr_plan_set_step({i})")

    def run(self, stream=None) -> None:
        check(lib().gr_plan_run(self.handle, _stream_ptr(stream)), "gr_plan_run")

    def time(self, warmup: int, iters: int, mode: int = GR_TIME_BATCH, stream=None) -> float:
        ms = ctypes.c_float()
        check(lib().gr_plan_time(self.handle, _stream_ptr(stream), warmup, iters, mode, ctypes.byref(ms)),
              "gr_plan_time")
        return float(ms.value)

    def close(self) -> None:
        if self.handle:
            lib().gr_plan_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def dtype_code(torch_dtype) -> int:
    import torch
    if torch_dtype == torch.float16:
        return GR_F16
    if torch_dtype == torch.bfloat16:
        return GR_BF16
    if torch_dtype == torch.float32:
        return GR_F32
    raise ValueError(f"unsupported dtype {torch_dtype}")
