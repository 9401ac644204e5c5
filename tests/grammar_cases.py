"""Program builders shared by the grammar tests: the reference's renderer test
cases (test_renderer.py:298-509) restated, plus batched/fp16 attention, causal
and SiLU-MLP programs for the extensions. Each builder returns a fresh
Program; REFS maps a case to its closed-form numpy reference."""
import math

import numpy as np

from grammar.kernel_ast import Program, ParallelLoop, Load, Store, Compute, ReductionLoop


def p_elementwise_add():
    a, b = Load("a", ["n", "m"]), Load("b", ["n", "m"])
    s = Compute("add", [a, b])
    return Program({"a": (256, 256), "b": (256, 256), "o": (256, 256)},
                   [ParallelLoop("o", (64, 64), ("n", "m"), [a, b, s, Store("o", s, ["n", "m"])])])


def _unary(op):
    def build():
        a = Load("a", ["n", "m"])
        r = Compute(op, [a])
        return Program({"a": (256, 256), "o": (256, 256)},
                       [ParallelLoop("o", (64, 64), ("n", "m"), [a, r, Store("o", r, ["n", "m"])])])
    return build


p_relu = _unary("relu")
p_exp = _unary("exp")
p_silu = _unary("silu")


def p_mul():
    a, b = Load("a", ["n", "m"]), Load("b", ["n", "m"])
    s = Compute("mul", [a, b])
    return Program({"a": (256, 256), "b": (256, 256), "o": (256, 256)},
                   [ParallelLoop("o", (64, 64), ("n", "m"), [a, b, s, Store("o", s, ["n", "m"])])])


def p_relu_of_sum():
    a, b = Load("a", ["n", "m"]), Load("b", ["n", "m"])
    s = Compute("add", [a, b])
    r = Compute("relu", [s])
    return Program({"a": (256, 256), "b": (256, 256), "o": (256, 256)},
                   [ParallelLoop("o", (64, 64), ("n", "m"), [a, b, s, r, Store("o", r, ["n", "m"])])])


def p_matmul_full_k():
    x, y = Load("x", ["n", "k"]), Load("y", ["k", "m"])
    mm = Compute("matmul", [x, y])
    return Program({"x": (256, 128), "y": (128, 256), "c": (256, 256)},
                   [ParallelLoop("c", (64, 64), ("n", "m"), [x, y, mm, Store("c", mm, ["n", "m"])])])


def p_matmul_reduction():
    x, y = Load("x", ["n", "k"]), Load("y", ["k", "m"])
    mm = Compute("matmul", [x, y])
    red = ReductionLoop("k", 32, [x, y, mm], mm)
    return Program({"x": (256, 128), "y": (128, 256), "c": (256, 256)},
                   [ParallelLoop("c", (64, 64), ("n", "m"), [red, Store("c", red, ["n", "m"])])])


def p_extract_matmul():
    x, y = Load("x", ["n", "k"]), Load("y", ["k", "m"])
    mm = Compute("matmul", [x, y])
    red = ReductionLoop("k", 32, [mm], mm)
    return Program({"x": (256, 128), "y": (128, 256), "c": (256, 256)},
                   [ParallelLoop("c", (64, 64), ("n", "m"), [x, y, red, Store("c", red, ["n", "m"])])])


def p_softmax():
    S = Load("S", ["n", "m"])
    mx = Compute("rowmax", [S], axis="m")
    sub = Compute("sub", [S, mx])
    e = Compute("exp", [sub])
    sm = Compute("rowsum", [e], axis="m")
    P = Compute("div", [e, sm])
    return Program({"S": (256, 256), "P": (256, 256)},
                   [ParallelLoop("P", (64, 256), ("n", "m"), [S, mx, sub, e, sm, P, Store("P", P, ["n", "m"])])])


def p_attention():
    N, d = 128, 64
    Q, KT = Load("Q", ["i", "dd"]), Load("KT", ["dd", "j"])
    s = Compute("matmul", [Q, KT])
    st1 = ParallelLoop("S", (64, N), ("i", "j"), [Q, KT, s, Store("S", s, ["i", "j"])])
    S2 = Load("S", ["i", "j"])
    mx = Compute("rowmax", [S2], axis="j")
    sb = Compute("sub", [S2, mx])
    e = Compute("exp", [sb])
    sm = Compute("rowsum", [e], axis="j")
    P = Compute("div", [e, sm])
    st2 = ParallelLoop("P", (64, N), ("i", "j"), [S2, mx, sb, e, sm, P, Store("P", P, ["i", "j"])])
    P3, V = Load("P", ["i", "j"]), Load("V", ["j", "dd"])
    o = Compute("matmul", [P3, V])
    st3 = ParallelLoop("O", (64, d), ("i", "dd"), [P3, V, o, Store("O", o, ["i", "dd"])])
    return Program({"Q": (N, d), "KT": (d, N), "V": (N, d), "S": (N, N), "P": (N, N), "O": (N, d)},
                   [st1, st2, st3])


def p_attention_atomic():
    N, d = 128, 64
    Q, KT = Load("Q", ["i", "dd"]), Load("KT", ["dd", "j"])
    S = Compute("matmul", [Q, KT])
    s_S = ParallelLoop("S", (64, N), ("i", "j"), [Q, KT, S, Store("S", S, ["i", "j"])])
    SsL = Load("S", ["i", "j"])
    mx = Compute("rowmax", [SsL], axis="j")
    s_mx = ParallelLoop("mx", (64, N), ("i", "j"), [SsL, mx, Store("mx", mx, ["i", "j"])])
    S2, mxL = Load("S", ["i", "j"]), Load("mx", ["i", "j"])
    sb = Compute("sub", [S2, mxL])
    s_sb = ParallelLoop("sb", (64, N), ("i", "j"), [S2, mxL, sb, Store("sb", sb, ["i", "j"])])
    sbL = Load("sb", ["i", "j"])
    e = Compute("exp", [sbL])
    s_e = ParallelLoop("e", (64, N), ("i", "j"), [sbL, e, Store("e", e, ["i", "j"])])
    eL = Load("e", ["i", "j"])
    sm = Compute("rowsum", [eL], axis="j")
    s_sm = ParallelLoop("sm", (64, N), ("i", "j"), [eL, sm, Store("sm", sm, ["i", "j"])])
    e2, smL = Load("e", ["i", "j"]), Load("sm", ["i", "j"])
    P = Compute("div", [e2, smL])
    s_P = ParallelLoop("P", (64, N), ("i", "j"), [e2, smL, P, Store("P", P, ["i", "j"])])
    P3, V = Load("P", ["i", "j"]), Load("V", ["j", "dd"])
    o = Compute("matmul", [P3, V])
    s_O = ParallelLoop("O", (64, d), ("i", "dd"), [P3, V, o, Store("O", o, ["i", "dd"])])
    return Program({"Q": (N, d), "KT": (d, N), "V": (N, d), "S": (N, N), "mx": (N, 1), "sb": (N, N),
                    "e": (N, N), "sm": (N, 1), "P": (N, N), "O": (N, d)},
                   [s_S, s_mx, s_sb, s_e, s_sm, s_P, s_O])


def p_fused_matmul_add():
    x, y = Load("x", ["n", "k"]), Load("y", ["k", "m"])
    mm = Compute("matmul", [x, y])
    red = ReductionLoop("k", 32, [x, y, mm], mm)
    s1 = ParallelLoop("a", (64, 64), ("n", "m"), [red, Store("a", red, ["n", "m"])])
    a2, b2 = Load("a", ["n", "m"]), Load("b", ["n", "m"])
    add = Compute("add", [a2, b2])
    s2 = ParallelLoop("o", (32, 32), ("n", "m"), [a2, b2, add, Store("o", add, ["n", "m"])])
    return Program({"x": (256, 128), "y": (128, 256), "b": (256, 256), "a": (256, 256), "o": (256, 256)}, [s1, s2])


def p_tname_collision():
    a, b = Load("a", ["n", "m"]), Load("b", ["n", "m"])
    add = Compute("add", [a, b])
    s1 = ParallelLoop("t1", (64, 64), ("n", "m"), [a, b, add, Store("t1", add, ["n", "m"])])
    t1, c = Load("t1", ["n", "m"]), Load("c", ["n", "m"])
    mul = Compute("mul", [t1, c])
    s2 = ParallelLoop("t2", (64, 64), ("n", "m"), [t1, c, mul, Store("t2", mul, ["n", "m"])])
    return Program({"a": (256, 256), "b": (256, 256), "c": (256, 256), "t1": (256, 256), "t2": (256, 256)}, [s1, s2])


def _layernorm(tile_f):
    D, eps = 128, 1e-5
    rL = Load("r", ["b", "f"])
    s1 = Compute("rowsum", [rL], axis="f")
    r2a, r2b = Load("r", ["b", "f"]), Load("r", ["b", "f"])
    rr = Compute("mul", [r2a, r2b])
    s2 = Compute("rowsum", [rr], axis="f")
    mean = Compute("mulc", [s1], const=1.0 / D)
    meansq = Compute("mulc", [s2], const=1.0 / D)
    mean2 = Compute("mul", [mean, mean])
    var = Compute("sub", [meansq, mean2])
    vareps = Compute("addc", [var], const=eps)
    std = Compute("sqrt", [vareps])
    r3 = Load("r", ["b", "f"])
    centered = Compute("sub", [r3, mean])
    out = Compute("div", [centered, std])
    return Program({"r": (64, D), "o": (64, D)},
                   [ParallelLoop("o", (64, tile_f), ("b", "f"),
                                 [rL, s1, r2a, r2b, rr, s2, mean, meansq, mean2, var, vareps, std,
                                  r3, centered, out, Store("o", out, ["b", "f"])])])


def p_layernorm():
    return _layernorm(128)


def p_layernorm_ftiled():
    return _layernorm(64)


def p_batched_4d_relu():
    x = Load("x", ["b0", "b1", "n", "m"])
    r = Compute("relu", [x])
    return Program({"x": (2, 4, 128, 128), "y": (2, 4, 128, 128)},
                   [ParallelLoop("y", (1, 1, 64, 64), ("b0", "b1", "n", "m"), [x, r, Store("y", r, ["b0", "b1", "n", "m"])])])


def p_inner_escape():
    x, y = Load("x", ["n", "k"]), Load("y", ["k", "m"])
    mm = Compute("matmul", [x, y])
    r = Compute("relu", [mm])
    red = ReductionLoop("k", 32, [x, y, mm, r], mm)
    return Program({"x": (256, 128), "y": (128, 256), "c": (256, 256)},
                   [ParallelLoop("c", (64, 64), ("n", "m"), [red, Store("c", r, ["n", "m"])])])


# ---- extensions ----------------------------------------------------------
def p_flash_attention(B=2, H=2, N=128, d=64, bm=64, bn=32, causal=False, scale=None, dtype="fp32"):
    """Batched attention as ONE stage: a ReductionLoop over keys whose partial
    is the online softmax of (Q KT) * scale [causal] against V."""
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    Q = Load("Q", ["b", "h", "i", "dd"])
    KT = Load("KT", ["b", "h", "dd", "j"])
    V = Load("V", ["b", "h", "j", "dd"])
    S = Compute("matmul", [Q, KT])
    Ss = Compute("mulc", [S], const=scale)
    body = [KT, V, S, Ss]
    x = Ss
    if causal:
        x = Compute("causal", [Ss], axis="j")
        body.append(x)
    sm = Compute("softmax_matmul", [x, V], axis="j")
    body.append(sm)
    red = ReductionLoop("j", bn, body, sm)
    st = ParallelLoop("O", (1, 1, bm, d), ("b", "h", "i", "dd"), [Q, red, Store("O", red, ["b", "h", "i", "dd"])])
    return Program({"Q": (B, H, N, d), "KT": (B, H, d, N), "V": (B, H, N, d), "O": (B, H, N, d)}, [st], dtype)


def p_mlp_silu(M=128, Dm=64, Hd=96, tm=64, tn=32, tk=32):
    X, W1 = Load("X", ["m", "k"]), Load("W1", ["k", "h"])
    h = Compute("matmul", [X, W1])
    r1 = ReductionLoop("k", tk, [X, W1, h], h)
    a = Compute("silu", [r1])
    s1 = ParallelLoop("A", (tm, tn), ("m", "h"), [r1, a, Store("A", a, ["m", "h"])])
    AL, W2 = Load("A", ["m", "h"]), Load("W2", ["h", "n"])
    y = Compute("matmul", [AL, W2])
    r2 = ReductionLoop("h", tk, [AL, W2, y], y)
    s2 = ParallelLoop("Y", (tm, tn), ("m", "n"), [r2, Store("Y", r2, ["m", "n"])])
    return Program({"X": (M, Dm), "W1": (Dm, Hd), "A": (M, Hd), "W2": (Hd, Dm), "Y": (M, Dm)}, [s1, s2])


def _np_softmax(s):
    e = np.exp(s - s.max(axis=-1, keepdims=True))
    return e / e.sum(axis=-1, keepdims=True)


def _ref_layernorm(i):
    r = i["r"].astype(np.float64)
    mean = r.mean(-1, keepdims=True)
    var = (r * r).mean(-1, keepdims=True) - mean * mean
    return (r - mean) / np.sqrt(var + 1e-5)


def _ref_flash(i, causal=False, d=64):
    q, kt, v = (i[n].astype(np.float64) for n in ("Q", "KT", "V"))
    s = (q @ kt) / math.sqrt(q.shape[-1])
    if causal:
        n = s.shape[-1]
        s = np.where(np.triu(np.ones((n, n), bool), 1), -np.inf, s)
    return _np_softmax(s) @ v


def _silu(x):
    return x / (1.0 + np.exp(-x))


REFS = {
    "elementwise_add": (p_elementwise_add, lambda i: i["a"] + i["b"]),
    "relu": (p_relu, lambda i: np.maximum(i["a"], 0)),
    "mul": (p_mul, lambda i: i["a"] * i["b"]),
    "exp": (p_exp, lambda i: np.exp(i["a"])),
    "relu_of_sum": (p_relu_of_sum, lambda i: np.maximum(i["a"] + i["b"], 0)),
    "matmul_full_k": (p_matmul_full_k, lambda i: i["x"] @ i["y"]),
    "matmul_reduction": (p_matmul_reduction, lambda i: i["x"] @ i["y"]),
    "extract_matmul": (p_extract_matmul, lambda i: i["x"] @ i["y"]),
    "softmax": (p_softmax, lambda i: _np_softmax(i["S"])),
    "attention": (p_attention, lambda i: _np_softmax(i["Q"] @ i["KT"]) @ i["V"]),
    "attention_atomic": (p_attention_atomic, lambda i: _np_softmax(i["Q"] @ i["KT"]) @ i["V"]),
    "fused_matmul_add": (p_fused_matmul_add, lambda i: i["x"] @ i["y"] + i["b"]),
    "batched_4d_relu": (p_batched_4d_relu, lambda i: np.maximum(i["x"], 0)),
    "tname_collision": (p_tname_collision, lambda i: (i["a"] + i["b"]) * i["c"]),
    "layernorm": (p_layernorm, _ref_layernorm),
    "layernorm_ftiled": (p_layernorm_ftiled, _ref_layernorm),
    # extensions
    "silu": (p_silu, lambda i: _silu(i["a"].astype(np.float64))),
    "flash_attention": (p_flash_attention, _ref_flash),
    "flash_attention_causal": (lambda: p_flash_attention(causal=True), lambda i: _ref_flash(i, causal=True)),
    "mlp_silu": (p_mlp_silu, lambda i: _silu(i["X"].astype(np.float64) @ i["W1"]) @ i["W2"]),
}

# The reference's 16 numeric cases (test_renderer.py:526-543).
REFERENCE_CASES = ["elementwise_add", "relu", "mul", "exp", "relu_of_sum", "matmul_full_k",
                   "matmul_reduction", "extract_matmul", "softmax", "attention", "attention_atomic",
                   "fused_matmul_add", "batched_4d_relu", "tname_collision", "layernorm", "layernorm_ftiled"]


def inputs_for(program, seed=0):
    """default_rng(seed).standard_normal per input, fp32 (test_renderer.py:263-265)."""
    from grammar.kernel_ast import kernel_meta
    rng = np.random.default_rng(seed)
    return {n: rng.standard_normal(tuple(s)).astype(np.float32) for n, s in kernel_meta(program)["inputs"]}
