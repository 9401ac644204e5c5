"""Whole-tensor fp32 evaluation of a program's meaning, used only as the
checker of the descent: the Evaluator compares every rendered variant's
output against it (the reference checks only the final best,
run_attention_search.py:169-181).

Tiling does not enter: each stage is evaluated over whole tensors with named
axes (a ReductionLoop is its partial over the full range), so every
semantics-preserving rewrite of a program has the same expected output and
it is computed once per search. Runs on the inputs' device in fp32 (float32
matmuls on contiguous operands only)."""
from __future__ import annotations

from .kernel_ast import Program, Load, Store, Compute, ReductionLoop, ROW_REDUCE_OPS, _value_axes


class _NT:
    """A named-axis tensor."""

    def __init__(self, t, axes):
        self.t, self.axes = t, list(axes)


def evaluate(program: Program, inputs: dict) -> dict:
    """inputs: name -> torch tensor (any dtype); returns name -> fp32 tensor
    for every tensor the program writes."""
    env = {k: v.float() for k, v in inputs.items()}
    for loop in program.body:
        vals = {}
        _eval_body(loop.body, program, env, vals)
    return env


def _eval_body(stmts, program, env, vals):
    import torch
    for s in stmts:
        if isinstance(s, Load):
            vals[id(s)] = _NT(env[s.source], s.index)
        elif isinstance(s, Compute):
            vals[id(s)] = _compute(s, [vals[id(i)] for i in s.inputs])
        elif isinstance(s, ReductionLoop):
            _eval_body(s.body, program, env, vals)
            vals[id(s)] = vals[id(s.partial)]
        elif isinstance(s, Store):
            v = vals[id(s.src)]
            shape = tuple(program.tensors[s.dest])
            t = v.t
            if tuple(t.shape) != shape:
                t = t.expand(shape) if t.dim() == len(shape) else t.reshape(shape)
            env[s.dest] = t.contiguous()


def _align(a: _NT, axes):
    """a's tensor permuted/unsqueezed to `axes` (missing axes -> size 1)."""
    import torch
    t = a.t
    if a.axes == list(axes):
        return t
    perm = [a.axes.index(x) for x in axes if x in a.axes]
    t = t.permute(*perm) if perm != list(range(len(perm))) else t
    shape = []
    it = iter(t.shape)
    for x in axes:
        shape.append(next(it) if x in a.axes else 1)
    return t.reshape(shape)


def _compute(c: Compute, ins):
    import torch
    op = c.op
    if op in ("matmul", "softmax_matmul"):
        a, b = ins
        out_axes = _value_axes(c)
        k = a.axes[-1]
        A = a.t
        if op == "softmax_matmul":
            A = torch.softmax(A, dim=-1)
        r = torch.matmul(A.contiguous(), b.t.contiguous())
        return _NT(r, out_axes)
    if op in ROW_REDUCE_OPS:
        a = ins[0]
        p = a.axes.index(c.axis)
        r = a.t.amax(dim=p, keepdim=True) if op == "rowmax" else a.t.sum(dim=p, keepdim=True)
        return _NT(r, a.axes)
    if op == "causal":
        a = ins[0]
        p = a.axes.index(c.axis)
        n_q, n_k = a.t.shape[p - 1], a.t.shape[p]
        mask = torch.ones(n_q, n_k, dtype=torch.bool, device=a.t.device).triu(1)
        shape = [1] * a.t.dim()
        shape[p - 1], shape[p] = n_q, n_k
        return _NT(a.t.masked_fill(mask.reshape(shape), float("-inf")), a.axes)
    wide = max(ins, key=lambda x: (len(x.axes), x.t.numel()))
    axes = wide.axes
    xs = [_align(x, axes) for x in ins]
    if op == "add":
        r = xs[0] + xs[1]
    elif op == "sub":
        r = xs[0] - xs[1]
    elif op == "mul":
        r = xs[0] * xs[1]
    elif op == "div":
        r = xs[0] / xs[1]
    elif op == "relu":
        r = torch.relu(xs[0])
    elif op == "exp":
        r = torch.exp(xs[0])
    elif op == "sqrt":
        r = torch.sqrt(xs[0])
    elif op == "mulc":
        r = xs[0] * float(c.const)
    elif op == "addc":
        r = xs[0] + float(c.const)
    elif op == "silu":
        r = torch.nn.functional.silu(xs[0])
    else:
        raise ValueError(f"torch_eval: unknown op {op!r}")
    return _NT(r, axes)
