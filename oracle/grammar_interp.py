"""Numpy tile interpreter for grammar programs -- test infrastructure only.

Executes a Program the way the reference's CPU mock of cuda.tile executes an
emitted module (test_renderer.py:60-123): every grid block runs serially, a
load is a slice copy, a store is a slice write, a reduction partial
accumulates into a fp32 accumulator (mma = acc + a @ b, kernel_ast.py:207-223),
and every buffer the program allocates is NaN-filled so an incomplete write
surfaces in the output. Values materialised outside a ReductionLoop are read
inside it as per-iteration sub-tiles (the reference's ct.extract bridge,
kernel_ast.py:755-780).

Tile shapes come from the grammar's own inference (grammar.kernel_ast), whose
results are pinned separately against the reference's logged numbers. The
online-softmax accumulator of a `softmax_matmul` partial is the textbook
recurrence (Milakov & Gimelshein 2018): m' = max(m, rowmax s), o' = o
e^(m-m') + e^(s-m') v, l' = l e^(m-m') + rowsum e^(s-m'), result o / l.
"""
from __future__ import annotations

import math
from itertools import product

import numpy as np

from grammar.kernel_ast import (
    Program, Load, Store, Compute, ReductionLoop, ROW_REDUCE_OPS, _infer_program, _resolve_index,
    _value_axes, _program_io, validate,
)


class _Tile:
    """A materialised tile: data plus its global offset on each axis."""
    __slots__ = ("a", "axes", "off")

    def __init__(self, a, axes, off):
        self.a, self.axes, self.off = a, list(axes), list(off)


def _ew(op, xs, const):
    if op == "add":
        return xs[0] + xs[1]
    if op == "sub":
        return xs[0] - xs[1]
    if op == "mul":
        return xs[0] * xs[1]
    if op == "div":
        return xs[0] / xs[1]
    if op == "relu":
        return np.maximum(xs[0], 0.0)
    if op == "exp":
        return np.exp(xs[0])
    if op == "sqrt":
        return np.sqrt(xs[0])
    if op == "mulc":
        return xs[0] * np.float32(const)
    if op == "addc":
        return xs[0] + np.float32(const)
    if op == "silu":
        return xs[0] / (1.0 + np.exp(-xs[0]))
    raise ValueError(f"interpreter: unknown op {op!r}")


def _softmax_rows(s):
    m = s.max(axis=-1, keepdims=True)
    m = np.where(np.isneginf(m), 0.0, m)
    e = np.exp(s - m)
    return e / e.sum(axis=-1, keepdims=True)


class _OnlineSoftmax:
    def __init__(self):
        self.m = self.l = self.o = None

    def update(self, s, v):
        mt = s.max(axis=-1, keepdims=True)
        if self.m is None:
            self.m = np.full_like(mt, -np.inf)
            self.l = np.zeros_like(mt)
            self.o = np.zeros(s.shape[:-1] + (v.shape[-1],), dtype=np.float32)
        mn = np.maximum(self.m, mt)
        ms = np.where(np.isneginf(mn), 0.0, mn)
        alpha = np.exp(self.m - ms)
        p = np.exp(s - ms)
        self.l = self.l * alpha + p.sum(axis=-1, keepdims=True)
        self.o = self.o * alpha + p @ v
        self.m = mn

    def value(self):
        return self.o / self.l


def run_program(program: Program, inputs: dict, storage_round=None) -> dict:
    """Run `program` on numpy `inputs` (name -> array). Returns every tensor.
    `storage_round(x)` (optional) rounds values written to / read from global
    memory, e.g. to fp16, to model a reduced-precision storage type."""
    validate(program)
    shapes = _infer_program(program)
    ins, inter, outs = _program_io(program)
    T = {}
    for n in ins:
        T[n] = np.asarray(inputs[n], dtype=np.float32)
    for n in inter + outs:
        T[n] = np.full(program.tensors[n], np.nan, dtype=np.float32)
    rnd = storage_round or (lambda x: x)

    for loop in program.body:
        g_out = program.tensors[loop.out]
        grid = [-(-g_out[d] // loop.tile_shape[d]) for d in range(len(g_out))]
        for coords in product(*[range(n) for n in grid]):
            scope = {v: c for v, c in zip(loop.index_vars, coords)}
            tile_of = dict(zip(loop.index_vars, loop.tile_shape))
            _run_block(loop.body, program, shapes, T, scope, tile_of, {}, [], rnd)
    return T


def _run_block(stmts, program, shapes, T, scope, tile_of, vals, loops, rnd, acc_for=None):
    """Execute `stmts`. vals: id -> (_Tile, depth materialised at). loops: the
    enclosing ReductionLoops, outermost first."""
    depth = len(loops)

    def read(v):
        t, d0 = vals[id(v)]
        a, off = t.a, list(t.off)
        for lp in loops[d0:]:                  # loops entered since materialisation
            if lp.axis in t.axes:
                p = t.axes.index(lp.axis)
                k = scope[lp.axis]
                if a.shape[p] > lp.tile:       # extract this iteration's sub-tile
                    sl = [slice(None)] * a.ndim
                    sl[p] = slice(k * lp.tile, (k + 1) * lp.tile)
                    a = a[tuple(sl)]
                    off[p] += k * lp.tile
        return a, off, t.axes

    for s in stmts:
        if isinstance(s, Load):
            shp = shapes[id(s)]
            g = program.tensors[s.source]
            idx = _resolve_index(s.index, shp, g, set(scope), f"load {s.source}")
            sl, off = [], []
            for name, t, gd in zip(idx, shp, g):
                c = 0 if name == "0" else scope[name]
                sl.append(slice(c * t, c * t + t))
                off.append(c * t)
            a = rnd(T[s.source][tuple(sl)]).astype(np.float32)
            if a.shape != tuple(min(t, gd - o) for t, gd, o in zip(shp, g, off)):
                raise AssertionError("load out of range")
            vals[id(s)] = (_Tile(a, s.index, off), depth)
        elif isinstance(s, Compute):
            args = [read(i) for i in s.inputs]
            if acc_for is not None and id(s) in acc_for:
                acc = acc_for[id(s)]
                acc.update(s, args)
                vals[id(s)] = (acc.tile(), depth)
                continue
            vals[id(s)] = (_Tile(*_compute(s, args)), depth)
        elif isinstance(s, ReductionLoop):
            accs = {id(p): _Acc(p) for p in s.partials}
            ext = _loop_extent(s, program)
            scope2 = dict(scope)
            for k in range(-(-ext // s.tile)):
                scope2[s.axis] = k
                _run_block(s.body, program, shapes, T, scope2, tile_of, vals, loops + [s], rnd, acc_for=accs)
            for p in s.partials:
                vals[id(p)] = (accs[id(p)].final(), depth)
            vals[id(s)] = vals[id(s.partials[0])]
        elif isinstance(s, Store):
            a, off, axes = read(s.src)
            shp = shapes[id(s.src)]
            g = program.tensors[s.dest]
            idx = _resolve_index(s.index, shp, g, set(scope), f"store {s.dest}")
            sl = []
            for d, (name, gd) in enumerate(zip(idx, g)):
                n = a.shape[d]
                c = 0 if name == "0" else scope[name]
                st = c * shp[d] if name != "0" else 0
                sl.append(slice(st, st + n))
            T[s.dest][tuple(sl)] = rnd(a)


def _loop_extent(rl, program):
    from grammar.kernel_ast import _loads_feeding, _iter_loads
    for ld in list(_loads_feeding(rl)) + list(_iter_loads(rl.body)):
        if rl.axis in ld.index:
            return program.tensors[ld.source][ld.index.index(rl.axis)]
    raise ValueError(f"reduction axis {rl.axis!r} not found in any load")


def _compute(c, args):
    arrs = [a for a, _, _ in args]
    if c.op in ("matmul", "softmax_matmul"):
        (a, oa, xa), (b, ob, xb) = args
        out_axes = _value_axes(c)
        off = oa[:-1] + [ob[-1]]
        if c.op == "softmax_matmul":
            return _softmax_rows(a) @ b, out_axes, off
        return a @ b, out_axes, off
    if c.op in ROW_REDUCE_OPS:
        a, off, axes = args[0]
        p = axes.index(c.axis)
        r = a.max(axis=p, keepdims=True) if c.op == "rowmax" else a.sum(axis=p, keepdims=True)
        off = list(off)
        off[p] = 0
        return r, axes, off
    if c.op == "causal":
        a, off, axes = args[0]
        p = axes.index(c.axis)
        q = p - 1
        qi = off[q] + np.arange(a.shape[q])
        kj = off[p] + np.arange(a.shape[p])
        mask = kj[None, :] > qi[:, None]
        shp = [1] * a.ndim
        shp[q], shp[p] = a.shape[q], a.shape[p]
        return np.where(mask.reshape(shp), -np.inf, a).astype(np.float32), axes, off
    # elementwise with broadcasting: the broadest operand sets axes/offsets
    bi = max(range(len(args)), key=lambda i: len(args[i][2]) * 10**6 + arrs[i].size)
    return _ew(c.op, arrs, c.const).astype(np.float32), args[bi][2], args[bi][1]


class _Acc:
    """Accumulator of one ReductionLoop partial."""

    def __init__(self, p):
        self.p = p
        self.a = None
        self.sm = _OnlineSoftmax() if p.op == "softmax_matmul" else None
        self.axes = self.off = None

    def update(self, c, args):
        if c.op == "softmax_matmul":
            (s, os_, _), (v, ov, _) = args
            self.sm.update(s, v)
            self.axes, self.off = _value_axes(c), os_[:-1] + [ov[-1]]
            return
        r, axes, off = _compute(c, args)
        self.axes, self.off = axes, off
        if self.a is None:
            init = -np.inf if c.op == "rowmax" else 0.0
            self.a = np.full(r.shape, init, dtype=np.float32)
        self.a = np.maximum(self.a, r) if c.op == "rowmax" else self.a + r

    def tile(self):
        if self.sm is not None:
            return _Tile(self.sm.value(), self.axes, self.off)
        return _Tile(self.a, self.axes, self.off)

    final = tile
