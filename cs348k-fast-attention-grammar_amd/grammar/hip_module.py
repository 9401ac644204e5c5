"""Load and run a rendered HIP module (the MI355X counterpart of importing a
generated cuTile module, grammar/optimization.py:306-318, and of the module
contract fn(*inputs) + KERNEL_META, bench.py:14-20).

    mod = load_module(emit_module(program))
    out = mod.fn(*inputs)                   # inputs in sorted-name order
    ms = mod.time(inputs, warmup, iters)    # hipEvents around the launch plan

Compilation goes through hiprtc (runtime.compile_source, or a CompilePool of
worker processes) with an in-process cache and an on-disk code-object cache.
The cache key covers everything the code object depends on: the rendered
source, the hiprtc version, the compile options and the bytes of every header
the source can include (csrc/*.h, pulled in through -I csrc), so an edited
header never reaches a kernel through a stale code object. Intermediates and
outputs are allocated once per bound input set
(the reference reallocates them with cp.zeros on every call,
kernel_ast.py:1271-1272); they start NaN-filled so an incomplete write shows.
"""
from __future__ import annotations

import hashlib
import os
import threading

from . import runtime as rt
from .hip_backend import parse_plan

_mem_cache: dict = {}
_lock = threading.Lock()


def cache_dir() -> str | None:
    d = os.environ.get("GR_CACHE_DIR", os.path.join(os.path.expanduser("~"), ".cache", "gr_hip"))
    if d.lower() in ("", "0", "off", "none"):
        return None
    return d


_toolchain = None


def toolchain_digest() -> str:
    """Digest of what a rendered module's code object depends on besides its
    own text: hiprtc's version, the fixed compile options (set in
    csrc/gr_rtc.cpp) and every header under csrc/. Computed once per process."""
    global _toolchain
    if _toolchain is None:
        h = hashlib.sha256()
        h.update(rt.version().encode())
        for name in sorted(os.listdir(rt.CSRC_DIR)):
            if name.endswith(".h") or name == "gr_rtc.cpp":
                h.update(b"\0" + name.encode() + b"\0")
                with open(os.path.join(rt.CSRC_DIR, name), "rb") as f:
                    h.update(f.read())
        _toolchain = h.hexdigest()
    return _toolchain


def source_key(src: str) -> str:
    h = hashlib.sha256()
    h.update(toolchain_digest().encode())
    h.update(b"\0")
    h.update(src.encode())
    return h.hexdigest()[:32]


def _cache_path(key: str) -> str | None:
    d = cache_dir()
    return os.path.join(d, key + ".co") if d else None


def lookup_cached(src: str) -> bytes | None:
    """The code object of `src` from the in-process or on-disk cache, or None."""
    key = source_key(src)
    with _lock:
        code = _mem_cache.get(key)
    if code is not None:
        return code
    path = _cache_path(key)
    if path and os.path.exists(path):
        with open(path, "rb") as f:
            code = f.read()
        with _lock:
            _mem_cache[key] = code
        return code
    return None


def store_cached(src: str, code: bytes) -> None:
    key = source_key(src)
    with _lock:
        _mem_cache[key] = code
    path = _cache_path(key)
    if path:
        try:
            os.makedirs(os.path.dirname(path), exist_ok=True)
            tmp = f"{path}.{os.getpid()}.{threading.get_ident()}.tmp"
            with open(tmp, "wb") as f:
                f.write(code)
            os.replace(tmp, path)
        except OSError:
            pass


def compile_cached(src: str, name: str = "gr_module.hip") -> tuple:
    """(code object bytes, cache hit?) for `src`, compiled in this process on a miss."""
    code = lookup_cached(src)
    if code is not None:
        return code, True
    code = rt.compile_source(src, name)
    store_cached(src, code)
    return code, False


_TORCH_DT = {"fp32": "float32", "fp16": "float16", "bf16": "bfloat16"}


# The checking build's findings buffer (csrc/gr_check.h): one count per kind,
# then the first finding at words 8-10.
CHECK_ARG = "__check__"
CHECK_WORDS = 16
CHECK_KINDS = ("lds_range", "global_range", "raw", "war", "waw")


class HipModule:
    def __init__(self, src: str, code: bytes | None = None):
        self.src = src
        self.plan = parse_plan(src)
        self.KERNEL_META = self.plan["meta"]
        self.inputs = list(self.plan["inputs"])
        self.code = code if code is not None else compile_cached(src)[0]
        self.module = rt.Module(self.code)
        self.kernels = [self.module.kernel(st["kernel"]) for st in self.plan["steps"]]
        self._bound = None

    @property
    def dtype(self):
        import torch
        return getattr(torch, _TORCH_DT[self.plan["dtype"]])

    def allocate(self, device="cuda") -> dict:
        """NaN-filled intermediates and outputs (and, for a checking build,
        the zeroed findings buffer "__check__")."""
        import torch
        out = {}
        for name in self.plan["intermediates"] + self.plan["outputs"]:
            out[name] = torch.full(tuple(self.plan["tensors"][name]), float("nan"), dtype=self.dtype, device=device)
        if self.plan.get("check"):
            out[CHECK_ARG] = torch.zeros(CHECK_WORDS, dtype=torch.int32, device=device)
        return out

    @staticmethod
    def check_report(tensors: dict) -> dict:
        """The findings of a checking build's run (csrc/gr_check.h): counts per
        kind and the first finding's kind, source line and index."""
        w = [int(x) & 0xFFFFFFFF for x in tensors[CHECK_ARG].cpu().tolist()]
        rep = {k: w[i] for i, k in enumerate(CHECK_KINDS)}
        rep["first"] = CHECK_KINDS[w[8] - 1] if w[8] else None
        rep["first_line"], rep["first_index"] = (w[9], w[10]) if w[8] else (None, None)
        return rep

    def bind(self, tensors: dict) -> rt.Plan:
        """A launch plan with every stage's tensor arguments bound."""
        import torch
        steps = []
        for st, k in zip(self.plan["steps"], self.kernels):
            args = []
            for a in st["args"]:
                t = tensors[a]
                if a == CHECK_ARG:
                    if t.dtype != torch.int32 or t.numel() < CHECK_WORDS or not t.is_contiguous():
                        raise ValueError(f"{CHECK_ARG}: need {CHECK_WORDS} contiguous int32")
                    args.append(t.data_ptr())
                    continue
                if tuple(t.shape) != tuple(self.plan["tensors"][a]) or t.dtype != self.dtype or not t.is_contiguous():
                    raise ValueError(f"tensor {a}: need contiguous {self.plan['tensors'][a]} {self.dtype}, "
                                     f"got {tuple(t.shape)} {t.dtype}")
                args.append(t.data_ptr())
            steps.append((k, st["grid"], st["block"], st["lds"], args))
        return rt.Plan(steps)

    def _check_inputs(self, inputs):
        if len(inputs) != len(self.inputs):
            raise ValueError(f"expected inputs {self.inputs}")
        for n, t in zip(self.inputs, inputs):
            if not t.is_cuda:
                raise ValueError(f"input {n} must be a GPU tensor (no CPU path)")

    def fn(self, *inputs):
        """Run the module on `inputs` (sorted-name order) and return the output
        (or a tuple of outputs)."""
        self._check_inputs(inputs)
        tensors = dict(zip(self.inputs, inputs))
        tensors.update(self.allocate(inputs[0].device))
        self.bind(tensors).run()
        outs = [tensors[o] for o in self.plan["outputs"]]
        return outs[0] if len(outs) == 1 else tuple(outs)

    __call__ = fn

    def time(self, inputs, warmup: int = 1, iters: int = 3, mode: int = rt.GR_TIME_MIN) -> float:
        """ms per run of the whole plan, hipEvents on the current stream:
        GR_TIME_MIN = min over per-run event pairs (the descent loss,
        grammar/optimization.py:284-300); GR_TIME_BATCH = mean over one pair
        around `iters` runs (bench.py:55-61)."""
        self._check_inputs(inputs)
        tensors = dict(zip(self.inputs, inputs))
        tensors.update(self.allocate(inputs[0].device))
        plan = self.bind(tensors)
        plan.run()
        return plan.time(max(0, warmup - 1), iters, mode)

    def run_with(self, inputs) -> dict:
        """Run once and return every tensor (inputs, intermediates, outputs)."""
        self._check_inputs(inputs)
        tensors = dict(zip(self.inputs, inputs))
        tensors.update(self.allocate(inputs[0].device))
        self.bind(tensors).run()
        return tensors


def load_module(src: str) -> HipModule:
    return HipModule(src)


def save_best(path: str, program, doc: str, best_loss_ms: float, iterations: int, stats: dict) -> dict:
    """Write a descent's best program as JSON: its structural key (rebuilt by
    kernel_ast.program_from_key), stage tiles and the lowering the HIP
    renderer picks for each stage (no compile). `stats` is Evaluator.stats()."""
    import json
    from .kernel_ast import emit_module, structural_key
    plan = parse_plan(emit_module(program))
    rec = {"_doc": doc, "best_loss_ms": best_loss_ms, "iterations": iterations,
           "evals_per_min": stats.get("evals_per_min"), "timed_variants": stats.get("timed_variants"),
           "stages": [[loop.out, list(loop.tile_shape)] for loop in program.body],
           "lowering": [[st["kernel"], st["lowering"], st.get("tiles")] for st in plan["steps"]],
           "key": json.loads(json.dumps(structural_key(program)))}
    with open(path, "w") as f:
        json.dump(rec, f)
        f.write("\n")
    return rec
