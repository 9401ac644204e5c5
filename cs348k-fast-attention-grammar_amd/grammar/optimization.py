"""Stochastic Rewrite Descent (SRD) over the kernel grammar, with the measured
MI355X runtime of each rendered variant as the loss.

Same structure and API as the reference (grammar/optimization.py):
  Stage 1: discrete coordinate descent over tile sizes (stage1_sweep,
           parameter_vector, TileParam; :342-510);
  Stage 2: sample K applicable rewrites, neighbour-tune each, commit the best
           non-worsening one (enumerate_rewrites, stage2_step; :528-793);
  autotune: the outer loop with best tracking, JSONL log, durable best
           sources and resume snapshots (:813-1035).

The Evaluator (:139-300) keeps the reference's scoring: structural-key memo;
an illegal fusion or unrenderable program is inf; over the tile budget or
compile-risky is MEM_PENALTY_BASE + excess (never compiled); a compile that
exceeds compile_timeout is MEM_PENALTY_BASE. A compiled variant runs on the
GPU on seeded inputs, is checked against the tiling-independent expected
output (torch_eval) -- a variant out of tolerance scores inf, so a wrong
kernel can never win -- and is timed with hipEvents (min over `iters`
per-call event pairs after `warmup`). Compilation goes through hiprtc; the
candidates of a coordinate are compiled concurrently before they are timed.

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
from concurrent.futures import ThreadPoolExecutor, TimeoutError as FutTimeout
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
    compile_workers: int = 4            # concurrent hiprtc compiles for prefetch


class _CompileTimeout(Exception):
    pass


def _tolerances(cfg: EvalConfig, dtype: str):
    if dtype == "fp32":
        return cfg.max_abs_tol or 1e-3, cfg.mean_abs_tol or 1e-3
    return cfg.max_abs_tol or 2e-2, cfg.mean_abs_tol or 2e-3


class Evaluator:
    """Renders, compiles, checks and times programs; memoised by structural
    key so an identical program is never recompiled or re-timed."""

    def __init__(self, cfg: EvalConfig = EvalConfig(), reference=None, inputs=None):
        """reference: optional callable(inputs dict) -> expected output tensor;
        by default the expected output is the whole-tensor evaluation of the
        first program checked (all rewrites preserve it). inputs: optional
        name -> GPU tensor; by default seeded N(0,1) rounded to the dtype."""
        self.cfg = cfg
        self._cache: dict = {}
        self._compiles = 0
        self._runs = 0
        self._cache_hits = 0
        self.ctx = ""
        self.reference = reference
        self._inputs = inputs or {}
        self._expected = {}
        self._pool = None
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
        the later __call__ finds the code object in the compile cache."""
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
            if self._pool is None:
                self._pool = self._new_pool()
            from .hip_module import compile_cached
            self._futures[key] = self._pool.submit(compile_cached, src)

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

    def _new_pool(self):
        # load the runtime (and torch's HIP runtime before it) on this thread,
        # not inside a compile worker
        from . import runtime as rt
        rt.lib()
        return ThreadPoolExecutor(max_workers=max(1, self.cfg.compile_workers))

    def stats(self) -> dict:
        el = max(1e-9, time.time() - self.t_start)
        return {"compiled_variants": self._compiles, "timed_variants": self._runs,
                "cache_hits": self._cache_hits, "distinct_scored": len(self._cache),
                "wall_s": el, "evals_per_min": 60.0 * self._runs / el}

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
            tiles = " ".join(f"{l.out}{tuple(l.tile_shape)}" for l in program.body)
            print(f"{self._tag} emit {1e3 * t_emit:.0f}ms  {len(program.body)} stage(s): {tiles}", flush=True)
        if self.cfg.proxy:
            return _proxy_score(program, src)
        g = self._gated(program)
        if g is not None:
            if self.cfg.log:
                print(f"{self._tag} static gate -> penalty {g:.0f} (not compiled)", flush=True)
            return g
        self._require_device()
        try:
            return self._run_gpu(program, key, src, t_emit)
        except _CompileTimeout:
            if self.cfg.log:
                print(f"{self._tag} COMPILE TIMEOUT (>{self.cfg.compile_timeout:.0f}s) -> penalty", flush=True)
            return MEM_PENALTY_BASE
        except Exception as e:
            if self.cfg.log:
                print(f"{self._tag} run FAILED ({type(e).__name__}: {str(e)[:300]}) -> inf", flush=True)
            return math.inf

    def _compile(self, key, src):
        from .hip_module import compile_cached
        fut = self._futures.pop(key, None)
        if fut is None:
            if self._pool is None:
                self._pool = self._new_pool()
            fut = self._pool.submit(compile_cached, src)
        try:
            code, hit = fut.result(timeout=self.cfg.compile_timeout or None)
        except FutTimeout:
            raise _CompileTimeout()
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

    def _run_gpu(self, program, key, src, t_emit) -> float:
        import torch
        from .hip_module import HipModule
        from . import runtime as rt
        log = self.cfg.log
        t1 = time.perf_counter()
        code = self._compile(key, src)
        t_comp = time.perf_counter() - t1
        self._compiles += 1
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


def _proxy_score(program: Program, src: str) -> float:
    """Cheap fake objective for exercising the loop without a GPU: bigger
    tiles worse, accumulating matmuls and sub-tile reads rewarded
    (reference _proxy_score, grammar/optimization.py:321-334)."""
    score = 0.0
    for loop in program.body:
        score += math.prod(loop.tile_shape)
        for rl in _reduction_loops(loop):
            score += rl.tile * 4
    if "mma:" in src or "flash attention" in src:
        score *= 0.4
    if "GR_SUBTILE" in src:
        score *= 0.95
    return score


# ---------------------------------------------------------------------------
# Parameters (reference :342-453)
# ---------------------------------------------------------------------------
@dataclass
class TileParam:
    name: str
    extent: int
    current: int
    setters: list = field(default_factory=list)
    rungs_src: tuple = TILE_LADDER

    def ladder(self) -> list:
        return sorted({s for s in self.rungs_src if s <= self.extent} | {self.extent})

    def set(self, size: int) -> None:
        for s in self.setters:
            s(size)
        self.current = size


def _reduction_loops(loop: ParallelLoop):
    out = []

    def walk(body):
        for s in body:
            if isinstance(s, ReductionLoop):
                out.append(s)
                walk(s.body)
    walk(loop.body)
    return out


def _reduction_extent(program: Program, rl: ReductionLoop) -> int:
    for ld in list(_loads_feeding(rl)) + list(_iter_loads(rl.body)):
        if rl.axis in ld.index:
            return program.tensors[ld.source][ld.index.index(rl.axis)]
    return rl.tile


def parameter_vector(program: Program, ladder: tuple | None = None, couple: bool = False) -> list:
    """Tunable tile dims keyed by their emitted names: TILE_<out>[d] per output
    dim (extent > 1), RTILE_<out> per stage's reduction loops."""
    rungs = ladder if ladder is not None else TILE_LADDER
    params: dict = {}

    def add(name, ext, cur, setter):
        if name in params:
            params[name].setters.append(setter)
        else:
            params[name] = TileParam(name, ext, cur, [setter], rungs)

    for loop in program.body:
        g = program.tensors[loop.out]
        for d, (sz, ext) in enumerate(zip(loop.tile_shape, g)):
            if ext <= 1:
                continue

            def mk(L=loop, dd=d):
                def s(v):
                    t = list(L.tile_shape)
                    t[dd] = v
                    L.tile_shape = tuple(t)
                return s
            add(f"TILE_{loop.out}[{d}]", ext, sz, mk())
        for rl in _reduction_loops(loop):
            def mkr(RL=rl):
                def s(v):
                    RL.tile = v
                return s
            add(f"RTILE_{loop.out}", _reduction_extent(program, rl), rl.tile, mkr())
    plist = list(params.values())
    if couple and plist:
        setters = []
        for p in plist:
            for st in p.setters:
                def clamped(v, _st=st, _e=p.extent):
                    _st(min(v, _e))
                setters.append(clamped)
        return [TileParam("TILE_GLOBAL", max(p.extent for p in plist), max(p.current for p in plist),
                          setters, rungs)]
    return plist


def _param_stage(name: str) -> str:
    """The stage a parameter belongs to: TILE_<out>[d] or RTILE_<out>."""
    base = name.split("[", 1)[0]
    return base[len("RTILE_"):] if base.startswith("RTILE_") else base[len("TILE_"):]


def _changed_stages(before: Program, after: Program) -> set:
    """Names of the stages of `after` that are new or differ structurally
    (tiles aside) from the stage of the same name in `before`."""
    def shape_free(loop):
        k = structural_key(loop)
        return tuple(x for x in k if not (isinstance(x, tuple) and all(isinstance(v, int) for v in x)))
    old = {l.out: shape_free(l) for l in before.body}
    return {l.out for l in after.body if old.get(l.out) != shape_free(l)}


def stage1_sweep(program: Program, ev: Evaluator, ladder: tuple | None = None, couple: bool = False,
                 neighbor: bool = False, full_ladder_for: set | None = None) -> tuple:
    """One coordinate sweep over the tile parameters of a clone of `program`
    (reference :461-510): all rungs while infeasible, adjacent rungs once
    feasible -- except the parameters of the stages in `full_ladder_for` (the
    stages a rewrite just changed), which always try every rung. The
    candidates of each coordinate are compiled concurrently."""
    prog = R.clone_program(program)
    R._strip_clone_meta(prog)
    params = parameter_vector(prog, ladder=ladder, couple=couple)
    best = ev(prog)
    use_neighbor = neighbor and best < MEM_PENALTY_BASE
    for p in params:
        rungs = p.ladder()
        if full_ladder_for and _param_stage(p.name) in full_ladder_for:
            cands = rungs
        elif use_neighbor and p.current in rungs:
            i = rungs.index(p.current)
            cands = [rungs[j] for j in (i - 1, i + 1) if 0 <= j < len(rungs)]
        else:
            cands = rungs
        cands = [c for c in cands if c != p.current]
        cur = p.current
        snaps = []
        for size in cands:
            p.set(size)
            snap = R.clone_program(prog)
            R._strip_clone_meta(snap)
            snaps.append(snap)
        p.set(cur)
        ev.prefetch(snaps)
        best_size, best_loss = cur, best
        for size, snap in zip(cands, snaps):
            loss = ev(snap)
            if loss < best_loss:
                best_loss, best_size = loss, size
        p.set(best_size)
        best = best_loss
        if neighbor and not use_neighbor and best < MEM_PENALTY_BASE:
            use_neighbor = True
    if full_ladder_for and best >= MEM_PENALTY_BASE:
        best = _joint_sweep(prog, params, full_ladder_for, ev, best)
    return prog, best


JOINT_MAX = 256   # tile combinations per stage in a joint sweep


def _joint_sweep(prog: Program, params: list, stages: set, ev: Evaluator, best: float) -> float:
    """Every combination of the tile parameters of each changed stage, tried
    when the coordinate sweep left the program over the memory budget. A
    stage whose lowering needs two tiles to change together (the flash kernel
    wants both its row tile in its ladder and the full head dim) cannot be
    reached one coordinate at a time from tiles a penalty shrank."""
    import itertools
    for stage in sorted(stages):
        sp = [p for p in params if _param_stage(p.name) == stage]
        if len(sp) < 2:
            continue
        grids = [sorted(set(p.ladder()) | {p.current}) for p in sp]
        if math.prod(len(g) for g in grids) > JOINT_MAX:
            continue
        cur = [p.current for p in sp]
        combos, snaps = [], []
        for combo in itertools.product(*grids):
            if list(combo) == cur:
                continue
            for p, v in zip(sp, combo):
                p.set(v)
            snap = R.clone_program(prog)
            R._strip_clone_meta(snap)
            combos.append(combo)
            snaps.append(snap)
        for p, v in zip(sp, cur):
            p.set(v)
        ev.prefetch(snaps)
        pick = None
        for combo, snap in zip(combos, snaps):
            loss = ev(snap)
            if loss < best:
                best, pick = loss, combo
        if pick is not None:
            for p, v in zip(sp, pick):
                p.set(v)
    return best


# ---------------------------------------------------------------------------
# Stage 2: rewrites (reference :517-793)
# ---------------------------------------------------------------------------
DEFAULT_RULES = ("hoist", "sink", "subtile_reduction", "unwrap_reduction", "merge", "merge_reductions",
                 "reorder", "sink_compute", "hoist_compute", "fuse_softmax", "split_softmax",
                 "fuse_softmax_chain")
REFERENCE_RULES = DEFAULT_RULES[:7]


def _iter_stmts(body):
    for s in body:
        yield s
        if isinstance(s, ReductionLoop):
            yield from _iter_stmts(s.body)


def _path_of(program: Program, node):
    for si, loop in enumerate(program.body):
        if loop is node:
            return (si, ())
        hit = _walk_path(loop.body, node, ())
        if hit is not None:
            return (si, hit)
    return None


def _walk_path(body, node, prefix):
    for i, s in enumerate(body):
        if s is node:
            return prefix + (i,)
        if isinstance(s, ReductionLoop):
            hit = _walk_path(s.body, node, prefix + (i,))
            if hit is not None:
                return hit
    return None


def _at_path(program: Program, path):
    si, idxs = path
    if si >= len(program.body):
        return None
    node = program.body[si]
    body = node.body
    for j, i in enumerate(idxs):
        if i >= len(body):
            return None
        node = body[i]
        if j < len(idxs) - 1:
            if not isinstance(node, ReductionLoop):
                return None
            body = node.body
    return node


@dataclass
class Rewrite:
    label: str
    resolve: object


_KINDS = {
    "hoist": (R.can_hoist, R.hoist),
    "sink": (R.can_sink, R.sink),
    "unwrap": (R.can_unwrap_reduction, R.unwrap_reduction),
    "merge": (R.can_merge, R.merge),
    "merge_red": (R.can_merge_reductions, R.merge_reductions),
    "reorder": (R.can_reorder, R.reorder),
    "sink_compute": (R.can_sink_compute, R.sink_compute),
    "hoist_compute": (R.can_hoist_compute, R.hoist_compute),
    "fuse_softmax": (R.can_fuse_softmax, R.fuse_softmax),
    "split_softmax": (R.can_split_softmax, R.split_softmax),
    "fuse_softmax_chain": (R.can_fuse_softmax_chain, R.fuse_softmax_chain),
    "fuse_attention": (lambda p, c: R.can_fuse_softmax_chain(p, c, True),
                       lambda p, c: R.fuse_softmax_chain(p, c, True)),
}


def _mk(kind, label, program, *nodes, **kw):
    """A rewrite addressed by path, re-resolved against whatever tree it is
    applied to (reference :583-625)."""
    paths = [_path_of(program, n) for n in nodes]

    def resolve(prog, kind=kind, paths=paths, kw=kw):
        targets = [_at_path(prog, p) for p in paths]
        if any(t is None for t in targets):
            return None
        try:
            if kind == "subtile":
                c, = targets
                if not R.can_subtile_reduction(prog, c, kw["axis"])[0]:
                    return None
                rt = kw.get("reduction_tile")
                return R.subtile_reduction(prog, c, kw["axis"], tile=rt) if rt is not None \
                    else R.subtile_reduction(prog, c, kw["axis"])
            can, do = _KINDS[kind]
            return do(prog, *targets) if can(prog, *targets)[0] else None
        except Exception:
            return None
    return Rewrite(label, resolve)


def _risk_excess(program: Program, threshold: int) -> int:
    if not threshold:
        return 0
    return sum(max(0, r - threshold) for r in kernel_compile_risk(program))


def enumerate_rewrites(program: Program, rules, max_risk: int = 0, reduction_tile: int | None = None,
                       mem_precondition: int = 0) -> list:
    """Every applicable rewrite (reference :635-729), with compile risk (and,
    for the repairability ablation, memory) folded in as preconditions."""
    out = []
    all_stmts = [s for loop in program.body for s in _iter_stmts(loop.body)]
    if "hoist" in rules:
        for s in all_stmts:
            if isinstance(s, Load) and R.can_hoist(program, s)[0]:
                out.append(_mk("hoist", f"hoist({s.source})", program, s))
    if "sink" in rules:
        for loop in program.body:
            loops_in = [x for x in _iter_stmts(loop.body) if isinstance(x, ReductionLoop)]
            for s in _iter_stmts(loop.body):
                if isinstance(s, Load):
                    for k in loops_in:
                        if R.can_sink(program, s, k)[0]:
                            out.append(_mk("sink", f"sink({s.source})", program, s, k))
    if "subtile_reduction" in rules:
        for s in all_stmts:
            if isinstance(s, Compute):
                for ax in sorted(R._contraction_axes(s)):
                    if R.can_subtile_reduction(program, s, ax)[0]:
                        out.append(_mk("subtile", f"subtile({s.op},{ax})", program, s, axis=ax,
                                       reduction_tile=reduction_tile))
    if "unwrap_reduction" in rules:
        for s in all_stmts:
            if isinstance(s, ReductionLoop) and R.can_unwrap_reduction(program, s)[0]:
                out.append(_mk("unwrap", f"unwrap({s.axis})", program, s))
    if "merge" in rules:
        for a, b in zip(program.body, program.body[1:]):
            if R.can_merge(program, a, b)[0]:
                out.append(_mk("merge", f"merge({a.out},{b.out})", program, a, b))
    if "merge_reductions" in rules:
        for loop in program.body:
            for a, b in zip(loop.body, loop.body[1:]):
                if isinstance(a, ReductionLoop) and isinstance(b, ReductionLoop) and \
                        R.can_merge_reductions(program, a, b)[0]:
                    out.append(_mk("merge_red", f"merge_red({a.axis})", program, a, b))
    if "reorder" in rules:
        for a, b in zip(program.body, program.body[1:]):
            if R.can_reorder(program, a, b)[0]:
                out.append(_mk("reorder", f"reorder({a.out},{b.out})", program, a, b))
        for loop in program.body:
            for a, b in zip(loop.body, loop.body[1:]):
                if R.can_reorder(program, a, b)[0]:
                    out.append(_mk("reorder", "reorder(stmt)", program, a, b))
    if "sink_compute" in rules:
        for loop in program.body:
            loops_in = [x for x in _iter_stmts(loop.body) if isinstance(x, ReductionLoop)]
            for s in _iter_stmts(loop.body):
                if isinstance(s, Compute):
                    for k in loops_in:
                        if R.can_sink_compute(program, s, k)[0]:
                            out.append(_mk("sink_compute", f"sink_compute({s.op})", program, s, k))
    if "hoist_compute" in rules:
        for s in all_stmts:
            if isinstance(s, Compute) and R.can_hoist_compute(program, s)[0]:
                out.append(_mk("hoist_compute", f"hoist_compute({s.op})", program, s))
    if "fuse_softmax" in rules:
        for a, b in zip(program.body, program.body[1:]):
            if R.can_fuse_softmax(program, a, b)[0]:
                out.append(_mk("fuse_softmax", f"fuse_softmax({a.out},{b.out})", program, a, b))
    if "fuse_softmax_chain" in rules:
        for b in program.body[2:]:
            if R.can_fuse_softmax_chain(program, b)[0]:
                out.append(_mk("fuse_softmax_chain", f"fuse_softmax_chain({b.out})", program, b))
            if R.can_fuse_softmax_chain(program, b, True)[0]:
                out.append(_mk("fuse_attention", f"fuse_attention({b.out})", program, b))
    if "split_softmax" in rules:
        for s in all_stmts:
            if isinstance(s, Compute) and s.op == "softmax_matmul" and R.can_split_softmax(program, s)[0]:
                out.append(_mk("split_softmax", "split_softmax", program, s))
    if not (max_risk or mem_precondition):
        return out
    cur = _risk_excess(program, max_risk)
    live = []
    for rw in out:
        cand = rw.resolve(program)
        if cand is None:
            continue
        try:
            if max_risk:
                ce = _risk_excess(cand, max_risk)
                if not (ce == 0 or ce < cur):
                    continue
            if mem_precondition and peak_tile_bytes(cand) > mem_precondition:
                continue
        except (AssertionError, ValueError, KeyError):
            continue            # an illegal fusion: no tiling can render it
        live.append(rw)
    return live


def stage2_step(program: Program, ev: Evaluator, K: int, rules, rng: random.Random, ladder=None,
                couple: bool = False, depth: int = 1, it: int = 0) -> tuple:
    """Depth-bounded greedy rewrite chain (reference :732-793)."""
    log = ev.cfg.log
    prog, applied = program, []
    ev.ctx = f"it {it} | S2 base-tune"
    cur = stage1_sweep(prog, ev, ladder, couple, neighbor=True)[1]
    for d in range(max(1, depth)):
        menu = enumerate_rewrites(prog, rules, ev.cfg.max_compile_risk,
                                  reduction_tile=ev.cfg.reduction_tile_default,
                                  mem_precondition=(0 if ev.cfg.repairable else ev.cfg.mem_budget))
        if not menu:
            break
        # While the program is still over the memory budget (a penalty, not a
        # time) every applicable rewrite is ranked instead of K sampled ones:
        # such candidates are mostly rejected statically (no compile), and a
        # random K can keep missing the one fusion that reaches a feasible
        # program, leaving the walk among penalties that differ in bytes only.
        sample = list(menu) if cur >= MEM_PENALTY_BASE else rng.sample(menu, min(K, len(menu)))
        if log:
            print(f"===== it {it} | STAGE 2: ranking {len(sample)} rewrite(s), base loss {cur:.4g} =====", flush=True)
        best = None
        for rw in sample:
            cand = rw.resolve(prog)
            if cand is None:
                continue
            ev.ctx = f"it {it} | S2 try {rw.label}"
            tuned, loss = stage1_sweep(cand, ev, ladder, couple, neighbor=True,
                                       full_ladder_for=_changed_stages(prog, cand))
            if log:
                print(f"     {rw.label} -> {loss:.4g} ({'ACCEPT' if loss <= cur else 'reject'}, base {cur:.4g})",
                      flush=True)
            if loss <= cur and (best is None or loss < best[0]):
                best = (loss, tuned, rw.label, cur - loss)
        if best is None:
            break
        prog = best[1]
        applied.append((best[2], best[3]))
        cur = best[0]
    return prog, cur, applied


# ---------------------------------------------------------------------------
# Persistence (reference :808-907)
# ---------------------------------------------------------------------------
def loss_kind(loss: float) -> str:
    if loss == math.inf:
        return "infeasible"
    if loss >= MEM_PENALTY_BASE:
        return "penalty"
    return "feasible"


def _num(x):
    return "inf" if x == math.inf else x


def _unnum(x):
    return math.inf if x == "inf" else x


def _jsonable(v):
    if isinstance(v, (str, int, float, bool)) or v is None:
        return v
    if isinstance(v, (tuple, list)):
        return [_jsonable(i) for i in v]
    return str(v)


def program_to_json(p: Program) -> dict:
    return {"key": structural_key(p), "dtype": p.dtype}


def program_from_json(d: dict) -> Program:
    return program_from_key(d["key"], d.get("dtype"))


class RunLogger:
    """config.json, log.jsonl (one record per iteration, with wall time and
    evaluator counters), kernels/best_it{N}.hip (durable emitted source of
    every new feasible best) and an atomic JSON resume snapshot."""

    def __init__(self, run_dir: str, cfg, start_program: Program):
        self.dir = run_dir
        self.kernels_dir = os.path.join(run_dir, "kernels")
        os.makedirs(self.kernels_dir, exist_ok=True)
        self.log_path = os.path.join(run_dir, "log.jsonl")
        self.snap_path = os.path.join(run_dir, "snapshot.json")
        try:
            start_src = emit_module(start_program)
        except Exception:
            start_src = None
        with open(os.path.join(run_dir, "config.json"), "w") as f:
            json.dump({"search": {k: _jsonable(v) for k, v in vars(cfg).items()},
                       "start_stages": [[s.out, list(s.tile_shape)] for s in start_program.body],
                       "start_program": program_to_json(start_program),
                       "start_source": start_src}, f, indent=2)

    def log_iter(self, *, iteration, loss, best_loss, applied, program, best_key, ev: Evaluator | None = None):
        try:
            flops, exact = program_flops(program)
        except Exception:
            flops, exact = None, False
        try:
            ptb = peak_tile_bytes(program)
        except Exception:
            ptb = None
        rec = {"iter": iteration, "time": time.time(), "loss": _num(loss), "loss_kind": loss_kind(loss),
               "best_loss": _num(best_loss), "best_loss_kind": loss_kind(best_loss),
               "applied": [a for a, _ in applied], "stages": [[s.out, list(s.tile_shape)] for s in program.body],
               "n_stages": len(program.body), "flops": flops, "flops_exact": exact, "peak_tile_bytes": ptb,
               "best_key": best_key}
        if ev is not None:
            rec["eval"] = ev.stats()
        with open(self.log_path, "a") as f:
            f.write(json.dumps(rec) + "\n")

    def save_best_source(self, iteration: int, best_program: Program):
        try:
            src = emit_module(best_program)
        except Exception:
            return
        with open(os.path.join(self.kernels_dir, f"best_it{iteration}.hip"), "w") as f:
            f.write(src)
        with open(os.path.join(self.kernels_dir, f"best_it{iteration}.json"), "w") as f:
            json.dump(program_to_json(best_program), f)

    def snapshot(self, state: dict):
        tmp = self.snap_path + ".tmp"
        with open(tmp, "w") as f:
            json.dump(state, f)
        os.replace(tmp, self.snap_path)


def load_snapshot(run_dir: str) -> dict:
    with open(os.path.join(run_dir, "snapshot.json")) as f:
        st = json.load(f)
    st["program"] = program_from_json(st["program"])
    st["best_prog"] = program_from_json(st["best_prog"])
    st["best_loss"] = _unnum(st["best_loss"])
    v, internal, gauss = st["rng_state"]
    st["rng_state"] = (v, tuple(internal), gauss)
    cache = {}
    for k, val in st.get("eval_cache", []):
        cache[_tup(k)] = _unnum(val)
    st["eval_cache"] = cache
    return st


def _tup(x):
    return tuple(_tup(i) for i in x) if isinstance(x, list) else x


def _search_state(program, best_prog, best_loss, iteration, rng, ev, cfg) -> dict:
    return {"program": program_to_json(program), "best_prog": program_to_json(best_prog),
            "best_loss": _num(best_loss), "iteration": iteration, "rng_state": rng.getstate(),
            "eval_cache": [[k, _num(v)] for k, v in ev._cache.items()],
            "config": {k: _jsonable(v) for k, v in vars(cfg).items()}}


# ---------------------------------------------------------------------------
# Outer loop (reference :913-1035)
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
    return loss < best


def autotune(program: Program, ev: Evaluator | None = None, cfg: SearchConfig = SearchConfig()) -> Program:
    """Stochastic Rewrite Descent; returns the best program on the accepted path."""
    ev = ev or Evaluator()
    logger = RunLogger(cfg.run_dir, cfg, program) if cfg.run_dir else None
    t0 = time.time()
    if cfg.resume and cfg.run_dir:
        st = load_snapshot(cfg.run_dir)
        program, best_prog, best_loss = st["program"], st["best_prog"], st["best_loss"]
        start_it = st["iteration"] + 1
        rng = random.Random()
        rng.setstate(st["rng_state"])
        ev._cache.update(st["eval_cache"])
        if cfg.verbose:
            print(f"[resume] from iter {st['iteration']} best={best_loss:.4g}", flush=True)
    else:
        rng = random.Random(cfg.seed)
        ev.ctx = "init | S1"
        program, loss = stage1_sweep(program, ev, cfg.tile_ladder, cfg.couple_tiles, neighbor=True)
        best_prog, best_loss = R.clone_program(program), loss
        R._strip_clone_meta(best_prog)
        start_it = 1
        if cfg.verbose:
            print(f"[init] loss={loss:.4g}", flush=True)
        if logger:
            if loss_kind(loss) == "feasible":
                logger.save_best_source(0, best_prog)
            logger.log_iter(iteration=0, loss=loss, best_loss=best_loss, applied=[], program=program,
                            best_key=structural_key(best_prog), ev=ev)
            logger.snapshot(_search_state(program, best_prog, best_loss, 0, rng, ev, cfg))
    for it in range(start_it, cfg.iters + 1):
        if cfg.time_budget_s and time.time() - t0 > cfg.time_budget_s:
            if cfg.verbose:
                print(f"[budget] stopping at iteration {it - 1} after {time.time() - t0:.0f}s", flush=True)
            break
        applied = []
        if it % cfg.N == 0:
            program, _, applied = stage2_step(program, ev, cfg.K, cfg.rules, rng, cfg.tile_ladder,
                                              cfg.couple_tiles, cfg.depth, it)
            if cfg.verbose and applied:
                print(f"[it {it}] applied {[a for a, _ in applied]}", flush=True)
        ev.ctx = f"it {it} | S1"
        program, loss = stage1_sweep(program, ev, cfg.tile_ladder, cfg.couple_tiles, neighbor=True)
        improved = _better(loss, best_loss)
        if improved:
            best_loss, best_prog = loss, R.clone_program(program)
            R._strip_clone_meta(best_prog)
        if cfg.verbose:
            s = ev.stats()
            print(f"[it {it}] loss={loss:.4g}  best={best_loss:.4g}  stages={len(program.body)}  "
                  f"timed={s['timed_variants']} evals/min={s['evals_per_min']:.1f}", flush=True)
        if logger:
            if improved and loss_kind(best_loss) == "feasible":
                logger.save_best_source(it, best_prog)
            logger.log_iter(iteration=it, loss=loss, best_loss=best_loss, applied=applied, program=program,
                            best_key=structural_key(best_prog), ev=ev)
            logger.snapshot(_search_state(program, best_prog, best_loss, it, rng, ev, cfg))
    if cfg.verbose:
        s = ev.stats()
        print(f"[done] best={best_loss:.4g} compiles={ev._compiles} runs={ev._runs} "
              f"evals/min={s['evals_per_min']:.1f}", flush=True)
    return best_prog
