"""Stochastic Rewrite Descent (SRD) over the kernel grammar, with the measured
MI355X runtime of each rendered variant as the loss.

The reference's search (grammar/optimization.py) and its API:
  Stage 1: coordinate descent over tile sizes (stage1_sweep,
           parameter_vector, TileParam; :342-510);
  Stage 2: sample K applicable rewrites, tune each, commit the best
           non-worsening one (enumerate_rewrites, stage2_step; :528-793);
  autotune: the outer loop with best tracking, JSONL log, durable best
           sources and resume snapshots (:813-1035).
Rewrites come from the rule registry in rewrites.py; a menu entry records
its targets by pre-order position so it can be replayed on any copy of the
program it was enumerated on.

The Evaluator (:139-300) keeps the reference's scoring: structural-key memo;
an illegal fusion or unrenderable program is inf; over the tile budget or
compile-risky is MEM_PENALTY_BASE + excess (never compiled); a compile that
exceeds compile_timeout is MEM_PENALTY_BASE. A compiled variant runs on the
GPU on seeded inputs, is checked against the tiling-independent expected
output (torch_eval) -- a variant out of tolerance scores inf, so a wrong
kernel can never win -- and is timed with hipEvents (min over `iters`
per-call event pairs after `warmup`). Compilation goes through hiprtc; the
candidates of a coordinate are compiled concurrently before they are timed.
Evaluator.refine times the search's best few distinct programs again, side
by side with warm clocks and batched events, for the final choice.

Snapshots are JSON (programs as structural keys, the RNG state, the score
cache), written atomically; the reference pickles them (:879-891).
"""
from __future__ import annotations

import json
import math
import os
import random
import threading
import time
from concurrent.futures import Future
from dataclasses import dataclass, field

from . import rewrites as R
from .kernel_ast import (
    Program, ParallelLoop, ReductionLoop, Load, Store, Compute, emit_module, structural_key,
    peak_tile_bytes, kernel_peak_tile_bytes, kernel_compile_risk, program_flops, program_from_key,
    kernel_meta, _loads_feeding, _iter_loads,
)

MEM_PENALTY_BASE = 1e9
TILE_LADDER = (16, 32, 64, 128, 256)  # the full extent is added per axis; 256 for gfx950 (160 KiB LDS, 256-wide MFMA tiles)


@dataclass
class EvalConfig:
    warmup: int = 1
    iters: int = 3
    proxy: bool = False                 # dev-only fake score, no GPU
    seed: int = 0
    log: bool = False
    mem_budget: int = 128 * 1024        # largest single fp32 tile of a generic stage (gfx950 LDS is
                                        # 160 KiB per workgroup); flash-lowered stages are exempt
    compile_timeout: float = 60.0       # seconds for one hiprtc compile; 0 disables
    max_compile_risk: int = 0           # straight-line contraction extent gate; 0 disables. The
                                        # reference gates ptxas compile-time blow-up (default 256);
                                        # hiprtc compiles every stage form in well under a second
                                        # (loops are not unrolled), so it is off here
    repairable: bool = True             # memory check soft (penalty) vs hard precondition
    reduction_tile_default: int = 32    # tile of a fresh subtile_reduction loop
    check: bool = True                  # tolerance-check every compiled variant
    max_abs_tol: float | None = None    # default by dtype (fp32 1e-3, fp16/bf16 2e-2)
    mean_abs_tol: float | None = None   # default by dtype (fp32 1e-3, fp16/bf16 2e-3)
    compile_workers: int = 4            # concurrent hiprtc compiles (worker processes)
    repeat_check: bool = True           # run every checked variant twice; outputs must match bitwise
    checked_build: bool = False         # also run the checking build of every variant with a generic
                                        # stage (LDS/global bounds and LDS races, csrc/gr_check.h);
                                        # any finding scores inf


def _tolerances(cfg: EvalConfig, dtype: str):
    if dtype == "fp32":
        return cfg.max_abs_tol or 1e-3, cfg.mean_abs_tol or 1e-3
    return cfg.max_abs_tol or 2e-2, cfg.mean_abs_tol or 2e-3


class Evaluator:
    """Renders, compiles, checks and times programs; memoised by structural
    key so an identical program is never recompiled or re-timed."""

    def __init__(self, cfg: EvalConfig = EvalConfig(), reference=None, inputs=None, compiler=None):
        """reference: optional callable(inputs dict) -> expected output tensor;
        by default the expected output is the whole-tensor evaluation of the
        first program checked (all rewrites preserve it). inputs: optional
        name -> GPU tensor; by default seeded N(0,1) rounded to the dtype.
        compiler: a compile_pool.CompilePool (default: one of
        cfg.compile_workers worker processes with cfg.compile_timeout)."""
        self.cfg = cfg
        self._cache: dict = {}
        self._compiles = 0               # real hiprtc compiles
        self._code_hits = 0              # code objects found in the in-process / on-disk cache
        self._timeouts = 0
        self._nondeterministic = 0
        self._checked = 0                # variants whose checking build ran
        self._check_findings = 0         # ... and reported something (scored inf)
        self._runs = 0
        self._cache_hits = 0             # structural-key memo hits (no render, no compile)
        self.ctx = ""
        self.reference = reference
        self._inputs = inputs or {}
        self._expected = {}
        self._pool = compiler
        self._futures = {}
        self.timeline = []               # (wall time, key digest, loss, phase ms) per evaluated variant
        self.t_start = time.time()
        self._lock = threading.Lock()

    @property
    def _tag(self) -> str:
        return f"[{self.ctx}]" if self.ctx else "[eval]"

    # ---- public ------------------------------------------------------------
    def __call__(self, program: Program) -> float:
        key = structural_key(program)
        if key in self._cache:
            self._cache_hits += 1
            return self._cache[key]
        ms = self._measure(program, key)
        self._cache[key] = ms
        return ms

    def prefetch(self, programs) -> None:
        """Render and start compiling `programs` concurrently (no GPU work);
        the later __call__ picks up the code object."""
        if self.cfg.proxy:
            return
        for p in programs:
            key = structural_key(p)
            if key in self._cache or key in self._futures:
                continue
            try:
                src = emit_module(p)
            except Exception:
                continue
            if self._gated(p) is not None:
                continue
            self._futures[key] = self._submit(src)

    def _submit(self, src: str) -> Future:
        """A future of (code object, came from a cache?)."""
        from .hip_module import lookup_cached, store_cached
        code = lookup_cached(src)
        out: Future = Future()
        if code is not None:
            out.set_result((code, True))
            return out
        if self._pool is None:
            from .compile_pool import CompilePool
            self._pool = CompilePool(self.cfg.compile_workers, self.cfg.compile_timeout)
        inner = self._pool.submit(src)

        def done(f, out=out):
            e = f.exception()
            if e is not None:
                out.set_exception(e)
            else:
                store_cached(src, f.result())
                out.set_result((f.result(), False))
        inner.add_done_callback(done)
        return out

    def _require_device(self):
        """A missing GPU is an error of the run, not a loss of the variant."""
        if getattr(self, "_device_ok", False):
            return
        import torch
        from . import runtime as rt
        rt.lib()
        if not torch.cuda.is_available():
            raise RuntimeError("Evaluator: no HIP device visible to torch; timed evaluation needs a GPU "
                               "(use proxy=True on a CPU-only host)")
        self._device_ok = True

    def close(self) -> None:
        """End the compile worker processes (they also end at interpreter exit)."""
        if self._pool is not None:
            self._pool.close()
            self._pool = None

    def refine(self, k: int = 6, rounds: int = 3, iters: int = 200, ramp_ms: float = 50.0):
        """Time the k best distinct programs scored so far again, side by side,
        and return (fastest program, [records]).

        A loss is the minimum over a few per-call event pairs, taken while
        the GPU's clocks still ramp with the search's bursts of work. At
        microsecond scale, tilings within a few percent of each other swap
        places from run to run on those numbers. So the finalists (distinct
        rendered sources, all already checked against the reference) each
        get `rounds` interleaved rounds of `iters` back-to-back runs between
        one event pair, after `ramp_ms` of load on the first. The median
        round decides. Records: search loss and refined ms per finalist,
        fastest first."""
        if self.cfg.proxy:
            raise RuntimeError("Evaluator.refine: proxy scores have nothing to re-time")
        self._require_device()
        import statistics
        from .hip_backend import render_module
        from .hip_module import HipModule, compile_cached
        from .kernel_ast import program_from_key
        from . import runtime as rt
        ranked = sorted((loss, key) for key, loss in self._cache.items()
                        if math.isfinite(loss) and loss < MEM_PENALTY_BASE)
        cands, seen = [], set()
        for loss, key in ranked:
            prog = program_from_key(key)
            src = render_module(prog)
            # programs that render to the same kernels (comments aside) are one finalist
            body = "\n".join(l for l in src.splitlines() if not l.lstrip().startswith(("//", "/*GR_PLAN")))
            if body in seen:
                continue
            seen.add(body)
            cands.append((loss, prog, src))
            if len(cands) >= k:
                break
        if not cands:
            raise RuntimeError("Evaluator.refine: no feasible program scored")
        bound = []
        for loss, prog, src in cands:
            mod = HipModule(src, compile_cached(src)[0])
            _, ins = self._inputs_for(prog)
            tensors = dict(zip(mod.inputs, ins))
            tensors.update(mod.allocate(ins[0].device))
            bound.append((mod, mod.bind(tensors)))
        plan0 = bound[0][1]
        t0 = time.time()
        while (time.time() - t0) * 1e3 < ramp_ms:
            plan0.time(0, 50, rt.GR_TIME_BATCH)
        times = [[] for _ in bound]
        for _ in range(rounds):
            for i, (_, plan) in enumerate(bound):
                times[i].append(plan.time(1, iters, rt.GR_TIME_BATCH))
        recs = []
        for (loss, prog, _), (mod, _), ts in zip(cands, bound, times):
            recs.append({"program": prog, "search_ms": loss, "refined_ms": statistics.median(ts),
                         "stages": [[l.out, list(l.tile_shape)] for l in prog.body],
                         "tiles": [s.get("tiles") for s in mod.plan["steps"]]})
        recs.sort(key=lambda r: r["refined_ms"])
        return recs[0]["program"], recs

    def stats(self) -> dict:
        """Counters of the evaluations so far. evals_per_min counts variants
        that were compiled (or taken from the code-object cache), checked and
        timed; hiprtc_compiles and code_cache_hits split where their code
        objects came from; memo_hits are programs already scored."""
        el = max(1e-9, time.time() - self.t_start)
        return {"hiprtc_compiles": self._compiles,
                "code_cache_hits": self._code_hits, "compile_timeouts": self._timeouts,
                "nondeterministic": self._nondeterministic, "checked_builds": self._checked,
                "check_findings": self._check_findings, "timed_variants": self._runs,
                "memo_hits": self._cache_hits,
                "distinct_scored": len(self._cache), "wall_s": el, "evals_per_min": 60.0 * self._runs / el}

    # ---- scoring -------------------------------------------------------------
    def _tile_excess(self, program: Program) -> int:
        """Bytes by which the stages staged tile by tile in LDS exceed the
        per-stage tile budget (0 when within it, or when the gate is off)."""
        if not self.cfg.mem_budget:
            return 0
        from .hip_backend import flash_stage_indices
        try:
            per = kernel_peak_tile_bytes(program)
        except (AssertionError, ValueError, KeyError):
            return 0
        for i in flash_stage_indices(program):
            per[i] = 0
        return sum(max(0, k - self.cfg.mem_budget) for k in per)

    def _gated(self, program: Program):
        """Static penalty (memory / compile risk), or None if the program may be compiled."""
        cfg = self.cfg
        excess = self._tile_excess(program)
        if excess:
            return MEM_PENALTY_BASE + excess / 1024.0
        if cfg.max_compile_risk:
            per = kernel_compile_risk(program)
            if per and max(per) > cfg.max_compile_risk:
                return MEM_PENALTY_BASE + sum(max(0, r - cfg.max_compile_risk) for r in per)
        return None

    def _measure(self, program: Program, key) -> float:
        from .hip_backend import LdsOverflow, UnsupportedProgram
        t0 = time.perf_counter()
        try:
            src = emit_module(program)
        except AssertionError:
            if self.cfg.log:
                print(f"{self._tag} illegal fusion (incompatible tile widths) -> inf", flush=True)
            return math.inf
        except LdsOverflow as e:
            if self.cfg.log:
                print(f"{self._tag} {e} -> penalty", flush=True)
            # the LDS excess and the tile-budget excess of the other stages add
            # up, so a program's penalty falls whichever stage shrinks
            return MEM_PENALTY_BASE + (e.need + self._tile_excess(program)) / 1024.0
        except Exception as e:
            if self.cfg.log:
                print(f"{self._tag} emit failed ({type(e).__name__}: {e}) -> inf", flush=True)
            return math.inf
        t_emit = time.perf_counter() - t0
        if self.cfg.log:
            stages = ", ".join(f"{l.out}:{'x'.join(map(str, l.tile_shape))}" for l in program.body)
            print(f"{self._tag} emit {1e3 * t_emit:.0f}ms  {len(program.body)} stage(s): {stages}", flush=True)
        if self.cfg.proxy:
            return _proxy_score(program, src)
        g = self._gated(program)
        if g is not None:
            if self.cfg.log:
                print(f"{self._tag} static gate -> penalty {g:.0f} (not compiled)", flush=True)
            return g
        from .compile_pool import CompileTimeout
        t1 = time.perf_counter()
        try:
            code = self._compile(key, src)
        except CompileTimeout:
            self._timeouts += 1
            if self.cfg.log:
                print(f"{self._tag} COMPILE TIMEOUT (>{self.cfg.compile_timeout:.0f}s) -> penalty", flush=True)
            return MEM_PENALTY_BASE
        except Exception as e:
            if self.cfg.log:
                print(f"{self._tag} compile FAILED ({type(e).__name__}: {str(e)[:300]}) -> inf", flush=True)
            return math.inf
        t_comp = time.perf_counter() - t1
        self._require_device()
        try:
            return self._run_gpu(program, src, code, t_emit, t_comp)
        except Exception as e:
            if self.cfg.log:
                print(f"{self._tag} run FAILED ({type(e).__name__}: {str(e)[:300]}) -> inf", flush=True)
            return math.inf

    def _compile(self, key, src) -> bytes:
        fut = self._futures.pop(key, None) or self._submit(src)
        code, hit = fut.result()       # the pool bounds every compile by compile_timeout
        if hit:
            self._code_hits += 1
        else:
            self._compiles += 1
        return code

    def _inputs_for(self, program: Program):
        import torch
        from .workloads import torch_dtype
        meta = kernel_meta(program)
        out = []
        for name, shape in meta["inputs"]:
            k = (name, tuple(shape), program.dtype)
            t = self._inputs.get(name)
            if t is None or tuple(t.shape) != tuple(shape) or t.dtype != torch_dtype(program.dtype):
                t = self._inputs.get(k)
            if t is None:
                gen = torch.Generator("cpu").manual_seed(self.cfg.seed + sum(map(ord, name)))
                t = torch.randn(tuple(shape), generator=gen).to(torch_dtype(program.dtype)).to("cuda")
                self._inputs[k] = t
            out.append(t)
        return meta, out

    def expected(self, program: Program, meta, inputs):
        sig = (tuple((n, tuple(s)) for n, s in meta["inputs"]), meta["output"][0], program.dtype)
        e = self._expected.get(sig)
        if e is None:
            named = dict(zip([n for n, _ in meta["inputs"]], inputs))
            if self.reference is not None:
                e = self.reference(named).float()
            else:
                from .torch_eval import evaluate
                e = evaluate(program, named)[meta["output"][0]]
            self._expected[sig] = e
        return e

    def _run_gpu(self, program, src, code, t_emit, t_comp) -> float:
        import torch
        from .hip_module import HipModule
        from . import runtime as rt
        log = self.cfg.log
        mod = HipModule(src, code)
        meta, ins = self._inputs_for(program)
        t2 = time.perf_counter()
        out = mod.fn(*ins)
        torch.cuda.synchronize()
        if self.cfg.check:
            want = self.expected(program, meta, ins)
            got = out.float()
            mx_tol, mn_tol = _tolerances(self.cfg, program.dtype)
            d = (got - want).abs()
            ok = bool(torch.isfinite(got).all()) and float(d.max()) <= mx_tol and float(d.mean()) <= mn_tol
            if not ok:
                if log:
                    print(f"{self._tag} TOLERANCE FAIL max {float(d.max()):.3g} mean {float(d.mean()):.3g} -> inf",
                          flush=True)
                return math.inf
            if self.cfg.repeat_check:
                # a second run (fresh NaN-filled intermediates) must reproduce
                # the first bit for bit: a race between threads of a stage
                # (an LDS read before its write is visible) shows up here
                again = mod.fn(*ins)
                torch.cuda.synchronize()
                if not torch.equal(again, out):
                    self._nondeterministic += 1
                    if log:
                        print(f"{self._tag} NONDETERMINISTIC (two runs differ) -> inf", flush=True)
                    return math.inf
            if self.cfg.checked_build and "generic" in [s["lowering"] for s in mod.plan["steps"]]:
                rep = self._run_checked(program, ins)
                if rep is not None and any(rep[k] for k in ("lds_range", "global_range", "raw", "war", "waw")):
                    self._check_findings += 1
                    if log:
                        print(f"{self._tag} CHECKING BUILD: {rep} -> inf", flush=True)
                    return math.inf
        t_check = time.perf_counter() - t2
        t3 = time.perf_counter()
        best = mod.time(ins, warmup=self.cfg.warmup, iters=self.cfg.iters, mode=rt.GR_TIME_MIN)
        if best < 0.25:
            # microsecond-scale variants: a min over 3 runs is within the
            # run-to-run noise of competing tilings, so take a longer min
            reps = min(50, max(self.cfg.iters, int(2.0 / max(best, 1e-3))))
            best = min(best, mod.time(ins, warmup=1, iters=reps, mode=rt.GR_TIME_MIN))
        self._runs += 1
        t_time = time.perf_counter() - t3
        self.timeline.append({"t": time.time() - self.t_start, "loss": best,
                              "emit_ms": 1e3 * t_emit, "compile_ms": 1e3 * t_comp,
                              "check_ms": 1e3 * t_check, "time_ms": 1e3 * t_time,
                              "lowering": [s["lowering"] for s in mod.plan["steps"]]})
        if log:
            print(f"{self._tag}   compile {1e3 * t_comp:.0f}ms check {1e3 * t_check:.0f}ms "
                  f"{self.cfg.iters} timed reps -> min {best:.4g}ms", flush=True)
        return best


    def _run_checked(self, program: Program, ins) -> dict | None:
        """Run the checking build of `program` once on `ins` and return its
        findings; None when its shadow words do not fit in LDS at these
        tiles (the variant is then not checked this way)."""
        import torch
        from .hip_backend import UnsupportedProgram, render_module
        from .hip_module import HipModule
        try:
            src = render_module(program, check=True)
        except UnsupportedProgram:
            return None
        code = self._compile(("check",) + tuple(structural_key(program)), src)
        mod = HipModule(src, code)
        tensors = dict(zip(mod.inputs, ins))
        tensors.update(mod.allocate(ins[0].device))
        mod.bind(tensors).run()
        torch.cuda.synchronize()
        self._checked += 1
        return mod.check_report(tensors)


def _proxy_score(program: Program, src: str) -> float:
    """Cheap fake objective for exercising the loop without a GPU: bigger
    tiles worse, accumulating matmuls and sub-tile reads rewarded
    (reference _proxy_score, grammar/optimization.py:321-334)."""
    score = 0.0
    for loop in program.body:
        score += math.prod(loop.tile_shape)
        for rl in _loops_inside(loop):
            score += rl.tile * 4
    if "mma:" in src or "flash attention" in src:
        score *= 0.4
    if "GR_SUBTILE" in src:
        score *= 0.95
    return score


# ---------------------------------------------------------------------------
# Tile parameters (the reference's TileParam / parameter_vector, :342-453)
# ---------------------------------------------------------------------------
@dataclass
class TileParam:
    """One tunable tile size: `name` as the renderer emits it (TILE_<out>[d] or
    RTILE_<out>), the axis `extent`, the `current` size, the `setters` that
    write a size into every IR slot sharing the name, and the base rungs."""
    name: str
    extent: int
    current: int
    setters: list = field(default_factory=list)
    rungs_src: tuple = TILE_LADDER

    def ladder(self) -> list:
        """The base rungs that fit the axis, plus the whole extent."""
        return sorted({r for r in self.rungs_src if r <= self.extent} | {self.extent})

    def set(self, size: int) -> None:
        for put in self.setters:
            put(size)
        self.current = size


class ChoiceParam(TileParam):
    """A schedule knob of one stage (the renderer's choices for it, e.g. the
    flash kernel's query blocks per wave); its ladder is its choices."""

    def __init__(self, name: str, choices: tuple, current, setters: list):
        super().__init__(name, max(choices), current, setters, tuple(choices))

    def ladder(self) -> list:
        return list(self.rungs_src)


class _Knob:
    """Setter of a stage's schedule knob; the renderer's default is stored as
    an absent knob, so programs that never moved it keep their keys."""

    def __init__(self, stage: ParallelLoop, name: str, default):
        self.stage, self.name, self.default = stage, name, default

    def __call__(self, value) -> None:
        if value == self.default:
            self.stage.knobs.pop(self.name, None)
        else:
            self.stage.knobs[self.name] = value


class _OutputDim:
    """Setter of one dim of a stage's output tile."""

    def __init__(self, stage: ParallelLoop, dim: int):
        self.stage, self.dim = stage, dim

    def __call__(self, size: int) -> None:
        shape = list(self.stage.tile_shape)
        shape[self.dim] = size
        self.stage.tile_shape = tuple(shape)


class _LoopStep:
    """Setter of a ReductionLoop's step."""

    def __init__(self, loop: ReductionLoop):
        self.loop = loop

    def __call__(self, size: int) -> None:
        self.loop.tile = size


class _Clamped:
    """A setter that never exceeds its own axis (the coupled ablation)."""

    def __init__(self, put, limit: int):
        self.put, self.limit = put, limit

    def __call__(self, size: int) -> None:
        self.put(min(size, self.limit))


def _loops_inside(stage: ParallelLoop) -> list:
    return [s for s in R.statements(stage.body) if isinstance(s, ReductionLoop)]


def _loop_extent(program: Program, loop: ReductionLoop) -> int:
    """Global extent of the axis `loop` walks, from a Load indexed by it."""
    for ld in list(_loads_feeding(loop)) + list(_iter_loads(loop.body)):
        if loop.axis in ld.index:
            return program.tensors[ld.source][ld.index.index(loop.axis)]
    return loop.tile


def _knobs(program: Program):
    """(name, extent, current size, setter) of every tile slot: each output
    dim wider than 1, then each reduction loop (named after its stage)."""
    for stage in program.body:
        for d, (size, ext) in enumerate(zip(stage.tile_shape, program.tensors[stage.out])):
            if ext > 1:
                yield f"TILE_{stage.out}[{d}]", ext, size, _OutputDim(stage, d)
        for lp in _loops_inside(stage):
            yield f"RTILE_{stage.out}", _loop_extent(program, lp), lp.tile, _LoopStep(lp)


def _schedule_params(program: Program) -> list:
    """SCHED_<out>.<knob> for every schedule knob the renderer offers a stage."""
    from .hip_backend import schedule_knobs, KNOB_DEFAULTS
    out = []
    for stage in program.body:
        try:
            offered = schedule_knobs(stage, program)
        except Exception:
            continue
        for name, (choices, current) in sorted(offered.items()):
            out.append(ChoiceParam(f"SCHED_{stage.out}.{name}", tuple(choices), current,
                                   [_Knob(stage, name, KNOB_DEFAULTS.get(name))]))
    return out


def parameter_vector(program: Program, ladder: tuple | None = None, couple: bool = False,
                     schedule: bool = True) -> list:
    """The tunable tile sizes of `program`, one TileParam per emitted name
    (slots sharing a name move together), then the schedule knobs the
    renderer offers its stages (ChoiceParam; schedule=False leaves them
    out). couple=True folds the tile sizes into one TILE_GLOBAL knob, each
    slot clamped to its own extent, and offers nothing else -- the
    local-control ablation."""
    rungs = TILE_LADDER if ladder is None else ladder
    by_name: dict = {}
    for name, ext, size, put in _knobs(program):
        if name not in by_name:
            by_name[name] = TileParam(name, ext, size, [], rungs)
        by_name[name].setters.append(put)
    params = list(by_name.values())
    if couple and params:
        clamped = [_Clamped(put, p.extent) for p in params for put in p.setters]
        params = [TileParam("TILE_GLOBAL", max(p.extent for p in params), max(p.current for p in params),
                            clamped, rungs)]
    # the coupled vector is the single knob of the local-control ablation: no
    # per-stage schedule knobs beside it
    return params + (_schedule_params(program) if schedule and not couple else [])


def _owner(param_name: str) -> str:
    """The stage a parameter name belongs to."""
    head = param_name.split("[", 1)[0].split(".", 1)[0]
    for prefix in ("RTILE_", "TILE_", "SCHED_"):
        if head.startswith(prefix):
            return head[len(prefix):]
    return head


def _changed_stages(before: Program, after: Program) -> set:
    """Stages of `after` that are new, or differ from the same-named stage of
    `before` in anything but tile sizes."""
    def skeleton(stage):
        return tuple(x for x in structural_key(stage)
                     if not (isinstance(x, tuple) and all(isinstance(v, int) for v in x)))
    old = {s.out: skeleton(s) for s in before.body}
    return {s.out for s in after.body if old.get(s.out) != skeleton(s)}


def _copy(program: Program) -> Program:
    return R._duplicate(program)[0]


# ---------------------------------------------------------------------------
# Stage 1: one coordinate sweep over the tile sizes (reference :461-510)
# ---------------------------------------------------------------------------
def _sizes_to_try(p: TileParam, local: bool, exhaustive: bool) -> list:
    """Every other rung while the program is infeasible, for the stages a
    rewrite just changed, or when the current size is off the ladder; the
    neighbouring rungs once it is feasible."""
    rungs = p.ladder()
    if local and not exhaustive and p.current in rungs:
        at = rungs.index(p.current)
        rungs = rungs[max(0, at - 1):at + 2]
    return [r for r in rungs if r != p.current]


def _try_sizes(work: Program, ev: Evaluator, params: list, sizes: list, base: float):
    """Score `work` with each assignment in `sizes` (one size per param), the
    variants compiled together first; returns (best loss, its assignment) --
    the assignment None when nothing beats `base` (first best wins ties)."""
    keep = [p.current for p in params]
    variants = []
    for assign in sizes:
        for p, v in zip(params, assign):
            p.set(v)
        variants.append(_copy(work))
    for p, v in zip(params, keep):
        p.set(v)
    ev.prefetch(variants)
    winner, best = None, base
    for assign, prog in zip(sizes, variants):
        loss = ev(prog)
        if loss < best:
            winner, best = assign, loss
    return best, winner


def stage1_sweep(program: Program, ev: Evaluator, ladder: tuple | None = None, couple: bool = False,
                 neighbor: bool = False, full_ladder_for: set | None = None) -> tuple:
    """Tune a copy of `program` one tile parameter at a time: each parameter
    moves to the best of its candidate sizes (every rung while the program is
    over budget, adjacent rungs once it is feasible with neighbor=True, every
    rung always for the stages in `full_ladder_for`). Returns (program, loss).
    When changed stages leave the program infeasible, their parameters are
    also swept jointly."""
    work = _copy(program)
    params = parameter_vector(work, ladder=ladder, couple=couple)
    loss = ev(work)
    for p in params:
        local = neighbor and loss < MEM_PENALTY_BASE
        exhaustive = bool(full_ladder_for) and _owner(p.name) in full_ladder_for
        sizes = [(s,) for s in _sizes_to_try(p, local, exhaustive)]
        loss, pick = _try_sizes(work, ev, [p], sizes, loss)
        if pick is not None:
            p.set(pick[0])
    if full_ladder_for and loss >= MEM_PENALTY_BASE:
        loss = _joint_sweep(work, params, full_ladder_for, ev, loss)
    loss = _template_snaps(work, params, ev, loss)
    return work, loss


def _template_snaps(work: Program, params: list, ev: Evaluator, loss: float) -> float:
    """The tilings at which a stage lowers to a hand-written template (GEMM,
    flash), tried as joint moves of the stage's output tile dims: a
    one-coordinate sweep cannot reach them when the tilings in between lower
    to the generic kernel and score worse (a GEMM wants both its tile dims in
    its set at once). Scores are memoised, so a repeated sweep costs nothing."""
    from .hip_backend import template_tilings
    for stage in work.body:
        try:
            shapes = template_tilings(stage, work)
        except Exception:
            continue
        mine = {}
        for p in params:
            if p.name.startswith(f"TILE_{stage.out}[") and not isinstance(p, ChoiceParam):
                mine[int(p.name[len(f"TILE_{stage.out}["):-1])] = p
        dims = sorted(mine)
        if not dims or not shapes:
            continue
        here = tuple(mine[d].current for d in dims)
        combos = []
        for shape in shapes:
            c = tuple(shape[d] for d in dims)
            if c != here and c not in combos:
                combos.append(c)
        if combos:
            loss, pick = _try_sizes(work, ev, [mine[d] for d in dims], combos, loss)
            if pick is not None:
                for d, v in zip(dims, pick):
                    mine[d].set(v)
    return loss


JOINT_MAX = 256   # tile combinations per stage in a joint sweep


def _joint_sweep(work: Program, params: list, stages: set, ev: Evaluator, loss: float) -> float:
    """Every combination of the tile parameters of each changed stage, tried
    when the coordinate sweep left the program over the memory budget. A
    stage whose lowering needs two tiles to change together (the flash kernel
    wants both its row tile in its ladder and the full head dim) cannot be
    reached one coordinate at a time from tiles a penalty shrank."""
    import itertools
    for stage in sorted(stages):
        mine = [p for p in params if _owner(p.name) == stage]
        if len(mine) < 2:
            continue
        grids = [sorted(set(p.ladder()) | {p.current}) for p in mine]
        if math.prod(len(g) for g in grids) > JOINT_MAX:
            continue
        here = tuple(p.current for p in mine)
        combos = [c for c in itertools.product(*grids) if c != here]
        loss, pick = _try_sizes(work, ev, mine, combos, loss)
        if pick is not None:
            for p, v in zip(mine, pick):
                p.set(v)
    return loss


# ---------------------------------------------------------------------------
# Stage 2: rewrites (reference :517-793)
# ---------------------------------------------------------------------------
DEFAULT_RULES = ("hoist", "sink", "subtile_reduction", "unwrap_reduction", "merge", "merge_reductions",
                 "reorder", "sink_compute", "hoist_compute", "fuse_softmax", "split_softmax",
                 "fuse_softmax_chain")
REFERENCE_RULES = DEFAULT_RULES[:7]


@dataclass(frozen=True)
class _Move:
    """One application of a rule, with its node targets recorded as
    positions in the program's pre-order walk (the same in every copy of the
    program), so it can be replayed on a copy."""
    rule: str
    slots: tuple        # per target: ("node", pre-order position) or ("arg", value)
    kw: tuple

    def replay(self, program: Program):
        t = R.Tree(program)
        targets = []
        for kind, v in self.slots:
            node = t.at(v) if kind == "node" else v
            if node is None:
                return None
            targets.append(node)
        r = R.RULES[self.rule]
        kw = dict(self.kw)
        try:
            if not r.check_tree(t, *targets, **kw)[0]:
                return None
            return r.apply(program, *targets, **kw)
        except Exception:
            return None


class Rewrite:
    """A rewrite the descent may take: `label` for logs, `resolve(program)`
    applies it to `program` (or to any copy of it) and returns the new
    program, or None where it does not apply."""

    def __init__(self, label: str, move: _Move):
        self.label = label
        self.move = move

    def resolve(self, program: Program):
        return self.move.replay(program)

    def __repr__(self):
        return f"Rewrite({self.label})"


def _risk_excess(program: Program, threshold: int) -> int:
    """How far the stages' straight-line contraction extents exceed the gate
    (0 when the gate is off)."""
    return 0 if not threshold else sum(r - threshold for r in kernel_compile_risk(program) if r > threshold)


def _applicable(program: Program, rules, reduction_tile) -> list:
    t = R.Tree(program)
    menu = []
    for name in rules:
        r = R.RULES[name]
        for targets, kw in r.sites(t):
            if name == "subtile_reduction" and reduction_tile is not None:
                kw = {**kw, "tile": reduction_tile}
            if not r.check_tree(t, *targets, **kw)[0]:
                continue
            slots = tuple(("node", t.ordinal(x)) if t.has(x) else ("arg", x) for x in targets)
            menu.append(Rewrite(r.label(*targets, **{**r.defaults, **kw}), _Move(name, slots, tuple(sorted(kw.items())))))
    return menu


def enumerate_rewrites(program: Program, rules, max_risk: int = 0, reduction_tile: int | None = None,
                       mem_precondition: int = 0) -> list:
    """Every rewrite of the enabled `rules` that applies to `program`
    (reference :635-729). max_risk > 0 drops rewrites whose result is
    compile-risky without lowering the program's risk excess;
    mem_precondition > 0 (the repairability ablation) drops rewrites whose
    result exceeds that tile budget at the tiles it inherits."""
    menu = _applicable(program, rules, reduction_tile)
    if not (max_risk or mem_precondition):
        return menu
    base_excess = _risk_excess(program, max_risk)

    def admissible(rw) -> bool:
        out = rw.resolve(program)
        if out is None:
            return False
        try:
            if max_risk and 0 < _risk_excess(out, max_risk) >= base_excess:
                return False
            return not (mem_precondition and peak_tile_bytes(out) > mem_precondition)
        except (AssertionError, ValueError, KeyError):
            return False            # an illegal fusion: no tiling can render it
    return [rw for rw in menu if admissible(rw)]


def stage2_step(program: Program, ev: Evaluator, K: int, rules, rng: random.Random, ladder=None,
                couple: bool = False, depth: int = 1, it: int = 0) -> tuple:
    """Up to `depth` rewrites in a row: each time, tune a sample of K
    applicable rewrites (every applicable one while the program is still over
    budget) and commit the best whose loss does not exceed the current one.
    Returns (program, loss, [(label, improvement)])."""
    verbose = ev.cfg.log
    ev.ctx = f"iteration {it}: stage 2, current program"
    loss = stage1_sweep(program, ev, ladder, couple, neighbor=True)[1]
    taken = []
    for link in range(max(1, depth)):
        menu = enumerate_rewrites(program, rules, ev.cfg.max_compile_risk,
                                  reduction_tile=ev.cfg.reduction_tile_default,
                                  mem_precondition=0 if ev.cfg.repairable else ev.cfg.mem_budget)
        if not menu:
            break
        # over budget, a random K can keep missing the one fusion that reaches
        # a feasible program (most such candidates are rejected statically)
        trial = menu if loss >= MEM_PENALTY_BASE else rng.sample(menu, min(K, len(menu)))
        if verbose:
            print(f"===== it {it} | stage 2 link {link + 1}: {len(trial)} rewrite(s) vs loss {loss:.4g} =====",
                  flush=True)
        pick = None
        for rw in trial:
            moved = rw.resolve(program)
            if moved is None:
                continue
            ev.ctx = f"iteration {it}: stage 2, {rw.label}"
            tuned, got = stage1_sweep(moved, ev, ladder, couple, neighbor=True,
                                      full_ladder_for=_changed_stages(program, moved))
            if verbose:
                print(f"     {rw.label}: {got:.4g} ({'kept' if got <= loss else 'dropped'})", flush=True)
            if got <= loss and (pick is None or got < pick[0]):
                pick = (got, tuned, rw.label)
        if pick is None:
            break
        taken.append((pick[2], loss - pick[0]))
        loss, program = pick[0], pick[1]
    return program, loss, taken


# ---------------------------------------------------------------------------
# Run artefacts and resume (reference :808-907; JSON instead of pickle)
# ---------------------------------------------------------------------------
def loss_kind(loss: float) -> str:
    """feasible (a measured time), penalty (over a budget) or infeasible (inf)."""
    return "infeasible" if loss == math.inf else "penalty" if loss >= MEM_PENALTY_BASE else "feasible"


def _enc(x):
    return "inf" if x == math.inf else x


def _dec(x):
    return math.inf if x == "inf" else x


def _plain(v):
    """A JSON-able copy: scalars as they are, sequences as lists, the rest as text."""
    if v is None or isinstance(v, (bool, int, float, str)):
        return v
    return [_plain(i) for i in v] if isinstance(v, (tuple, list)) else str(v)


def _as_tuples(x):
    return tuple(_as_tuples(i) for i in x) if isinstance(x, list) else x


def program_to_json(p: Program) -> dict:
    return {"key": structural_key(p), "dtype": p.dtype}


def program_from_json(d: dict) -> Program:
    return program_from_key(d["key"], d.get("dtype"))


def _write_atomic(path: str, text: str) -> None:
    tmp = f"{path}.tmp"
    with open(tmp, "w") as f:
        f.write(text)
        f.flush()
        os.fsync(f.fileno())
    os.replace(tmp, path)


class RunLogger:
    """The files of one descent run under `run_dir`:
      config.json            search settings and the start program (key and source)
      log.jsonl              one record per iteration (the reference's fields, plus
                             wall time and the evaluator's counters)
      kernels/best_itN.hip   rendered source of each new feasible best (+ .json key)
      snapshot.json          everything a resume needs, replaced atomically
    A resumed run first cuts the log and the kernels back to the snapshot's
    iteration: a run killed between writing a record and its snapshot leaves
    records (or a torn last line) the resumed run will write again."""

    def __init__(self, run_dir: str, cfg, start_program: Program, resume_from: int | None = None):
        self.dir = run_dir
        self.kernels_dir = os.path.join(run_dir, "kernels")
        self.log_path = os.path.join(run_dir, "log.jsonl")
        self.snap_path = os.path.join(run_dir, "snapshot.json")
        os.makedirs(self.kernels_dir, exist_ok=True)
        if resume_from is not None:
            self.truncate(resume_from)
            return
        try:
            source = emit_module(start_program)
        except Exception:
            source = None
        doc = {"search": {k: _plain(v) for k, v in vars(cfg).items()},
               "start_stages": [[s.out, list(s.tile_shape)] for s in start_program.body],
               "start_program": program_to_json(start_program), "start_source": source}
        _write_atomic(os.path.join(run_dir, "config.json"), json.dumps(doc, indent=2))
        for stale in (self.log_path, self.snap_path):
            if os.path.exists(stale):
                os.remove(stale)

    def truncate(self, iteration: int) -> None:
        kept = []
        if os.path.exists(self.log_path):
            with open(self.log_path) as f:
                for line in f:
                    try:
                        rec = json.loads(line)
                    except ValueError:
                        break                      # a torn last record
                    if rec.get("iter", math.inf) > iteration:
                        break
                    kept.append(line if line.endswith("\n") else line + "\n")
        _write_atomic(self.log_path, "".join(kept))
        for name in os.listdir(self.kernels_dir):
            stem = name.split(".", 1)[0]
            if stem.startswith("best_it") and stem[7:].isdigit() and int(stem[7:]) > iteration:
                os.remove(os.path.join(self.kernels_dir, name))

    def log_iter(self, *, iteration, loss, best_loss, applied, program, best_key, ev: Evaluator | None = None):
        try:
            flops, exact = program_flops(program)
        except Exception:
            flops, exact = None, False
        try:
            footprint = peak_tile_bytes(program)
        except Exception:
            footprint = None
        rec = {"iter": iteration, "time": time.time(), "loss": _enc(loss), "loss_kind": loss_kind(loss),
               "best_loss": _enc(best_loss), "best_loss_kind": loss_kind(best_loss),
               "applied": [label for label, _ in applied],
               "stages": [[s.out, list(s.tile_shape)] for s in program.body], "n_stages": len(program.body),
               "flops": flops, "flops_exact": exact, "peak_tile_bytes": footprint, "best_key": best_key}
        if ev is not None:
            rec["eval"] = ev.stats()
        with open(self.log_path, "a") as f:
            f.write(json.dumps(rec) + "\n")
            f.flush()

    def save_best_source(self, iteration: int, best_program: Program) -> None:
        try:
            source = emit_module(best_program)
        except Exception:
            return
        stem = os.path.join(self.kernels_dir, f"best_it{iteration}")
        _write_atomic(stem + ".hip", source)
        _write_atomic(stem + ".json", json.dumps(program_to_json(best_program)))

    def snapshot(self, state: dict) -> None:
        _write_atomic(self.snap_path, json.dumps(state))


def load_snapshot(run_dir: str) -> dict:
    """The resume state a RunLogger wrote, with programs rebuilt from keys."""
    with open(os.path.join(run_dir, "snapshot.json")) as f:
        st = json.load(f)
    st["program"] = program_from_json(st["program"])
    st["best_prog"] = program_from_json(st["best_prog"])
    st["best_loss"] = _dec(st["best_loss"])
    version, internal, gauss = st["rng_state"]
    st["rng_state"] = (version, tuple(internal), gauss)
    st["eval_cache"] = {_as_tuples(k): _dec(v) for k, v in st.get("eval_cache", [])}
    return st


# ---------------------------------------------------------------------------
# The outer loop (reference :913-1035)
# ---------------------------------------------------------------------------
@dataclass
class SearchConfig:
    iters: int = 30
    N: int = 4                   # Stage 2 every N iterations
    K: int = 6                   # rewrites sampled per Stage-2 step
    depth: int = 1
    rules: tuple = DEFAULT_RULES
    seed: int = 0
    verbose: bool = True
    run_dir: str | None = None
    resume: bool = False
    tile_ladder: tuple | None = None
    couple_tiles: bool = False
    time_budget_s: float = 0.0   # stop after this much wall time (0 = none)


def _better(loss: float, best: float) -> bool:
    """Feasible < penalty < inf, and lower within a kind: plain `<`."""
    return loss < best


class _Descent:
    """State of one search: the program on the accepted path, the best one
    seen on it, the iteration reached and the RNG stream."""

    def __init__(self, ev: Evaluator, cfg: SearchConfig):
        self.ev, self.cfg = ev, cfg
        self.log = None
        self.iterations_done = 0

    def _tune(self, program):
        return stage1_sweep(program, self.ev, self.cfg.tile_ladder, self.cfg.couple_tiles, neighbor=True)

    def begin(self, program: Program) -> None:
        cfg = self.cfg
        if cfg.resume and cfg.run_dir:
            st = load_snapshot(cfg.run_dir)
            self.program, self.best, self.best_loss = st["program"], st["best_prog"], st["best_loss"]
            self.rng = random.Random()
            self.rng.setstate(st["rng_state"])
            self.ev._cache.update(st["eval_cache"])
            self.next_it = st["iteration"] + 1
            self.log = RunLogger(cfg.run_dir, cfg, self.program, resume_from=st["iteration"])
            if cfg.verbose:
                print(f"[resume] after iteration {st['iteration']}, best {self.best_loss:.4g}", flush=True)
            return
        self.log = RunLogger(cfg.run_dir, cfg, program) if cfg.run_dir else None
        self.rng = random.Random(cfg.seed)
        self.ev.ctx = "init | S1"
        self.program, loss = self._tune(program)
        self.best, self.best_loss = _copy(self.program), loss
        self.next_it = 1
        if cfg.verbose:
            print(f"[init] loss={loss:.4g}", flush=True)
        self._record(0, loss, [], improved=True)

    def _record(self, it: int, loss: float, applied: list, improved: bool) -> None:
        self.iterations_done = it
        if self.log is None:
            return
        if improved and loss_kind(self.best_loss) == "feasible":
            self.log.save_best_source(it, self.best)
        self.log.log_iter(iteration=it, loss=loss, best_loss=self.best_loss, applied=applied,
                          program=self.program, best_key=structural_key(self.best), ev=self.ev)
        self.log.snapshot({"program": program_to_json(self.program), "best_prog": program_to_json(self.best),
                           "best_loss": _enc(self.best_loss), "iteration": it, "rng_state": self.rng.getstate(),
                           "eval_cache": [[k, _enc(v)] for k, v in self.ev._cache.items()],
                           "config": {k: _plain(v) for k, v in vars(self.cfg).items()}})

    def step(self, it: int) -> None:
        cfg = self.cfg
        applied = []
        if it % cfg.N == 0:
            self.program, _, applied = stage2_step(self.program, self.ev, cfg.K, cfg.rules, self.rng,
                                                   cfg.tile_ladder, cfg.couple_tiles, cfg.depth, it)
            if cfg.verbose and applied:
                print(f"[it {it}] applied {[label for label, _ in applied]}", flush=True)
        self.ev.ctx = f"it {it} | S1"
        self.program, loss = self._tune(self.program)
        improved = _better(loss, self.best_loss)
        if improved:
            self.best, self.best_loss = _copy(self.program), loss
        if cfg.verbose:
            s = self.ev.stats()
            print(f"[it {it}] loss={loss:.4g}  best={self.best_loss:.4g}  stages={len(self.program.body)}  "
                  f"timed={s['timed_variants']} evals/min={s['evals_per_min']:.1f}", flush=True)
        self._record(it, loss, applied, improved)

    def run(self, program: Program) -> Program:
        t0 = time.time()
        self.begin(program)
        for it in range(self.next_it, self.cfg.iters + 1):
            if self.cfg.time_budget_s and time.time() - t0 > self.cfg.time_budget_s:
                if self.cfg.verbose:
                    print(f"[budget] stopped after iteration {it - 1} ({time.time() - t0:.0f}s)", flush=True)
                break
            self.step(it)
        if self.cfg.verbose:
            s = self.ev.stats()
            print(f"[done] best={self.best_loss:.4g} hiprtc compiles={s['hiprtc_compiles']} "
                  f"timed={s['timed_variants']} evals/min={s['evals_per_min']:.1f}", flush=True)
        return self.best


def autotune(program: Program, ev: Evaluator | None = None, cfg: SearchConfig = SearchConfig()) -> Program:
    """Stochastic Rewrite Descent: a Stage-1 sweep every iteration, preceded
    by a Stage-2 rewrite step every N-th; returns the best program on the
    accepted path. With cfg.run_dir the run is logged and snapshotted every
    iteration; with cfg.resume it continues from the snapshot. The iteration
    reached is left in the evaluator's `iterations` attribute."""
    ev = ev or Evaluator()
    d = _Descent(ev, cfg)
    best = d.run(program)
    ev.iterations = d.iterations_done
    return best
