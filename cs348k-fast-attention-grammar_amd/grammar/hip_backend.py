"""HIP (gfx950) renderer for grammar programs.

render_module(program) -> one HIP C++ translation unit: an extern "C" kernel
per ParallelLoop stage, plus a trailing /*GR_PLAN ...*/ comment holding the
launch plan (kernel, grid, block, LDS bytes, tensor arguments) and
KERNEL_META. The source alone is a durable, re-runnable artefact (the
reference keeps emitted cuTile modules the same way, grammar/optimization.py:
869-876).

Lowering, per stage (first match wins):
  * flash: one ReductionLoop over the key axis whose single partial is
    softmax_matmul(x, V) with x = [causal](mulc(matmul(Q, KT), scale)) computed
    inside the loop -> the hand-written CDNA4 body in gr_flash_fwd.h,
    instantiated with the stage's query tile, the loop's key tile, the
    program's scale/mask and storage type (fp16/bf16).
  * generic: every other stage. Each tile lives in LDS as fp32 (row-major in
    its materialised shape); statements run in program order across the 256
    threads of the workgroup with a barrier after each; values produced
    outside a ReductionLoop are read as per-iteration sub-tile views (the
    reference's ct.extract); ReductionLoop partials accumulate in fp32
    (matmul: sum of products, rowmax/rowsum, online softmax). Loads convert
    from and stores convert to the storage type.
Unsupported structures raise UnsupportedProgram (the Evaluator scores them as
infeasible), never a silent fallback.
"""
from __future__ import annotations

import json
import math
import re

from .kernel_ast import (
    Program, ParallelLoop, Load, Store, Compute, ReductionLoop, ROW_REDUCE_OPS, ELEMENTWISE_OPS,
    _infer_program, _resolve_index, _value_axes, _program_io, _loop_tensors, validate, kernel_meta,
    _loads_feeding, _iter_loads, _axis_global_extent, _contraction_axis,
)

NT = 256                      # threads per workgroup of generic kernels
LDS_LIMIT = 160 * 1024        # gfx950 LDS per workgroup
CTYPE = {"fp32": "float", "fp16": "_Float16", "bf16": "__bf16"}
LOG2E = 1.4426950408889634


class UnsupportedProgram(Exception):
    """The program uses a structure this renderer cannot lower."""


class LdsOverflow(UnsupportedProgram):
    """Stages need more LDS than one gfx950 workgroup has. `need` is the sum
    over all overflowing stages of their excess bytes (each over-budget stage
    contributes, so shrinking any one of them lowers it)."""

    def __init__(self, stage, need):
        super().__init__(f"stage(s) {stage}: {need} bytes of LDS beyond {LDS_LIMIT} per workgroup")
        self.need = need


def _cname(name: str) -> str:
    """C identifier for a tensor: prefixed so no tensor name can collide with
    the generated code's locals (e, k, i0, ...)."""
    return "t_" + re.sub(r"[^A-Za-z0-9_]", "_", name)


def _prod(xs):
    return math.prod(xs) if xs else 1


def _cdiv(a, b):
    return -(-a // b)


def _flt(x: float) -> str:
    r = repr(float(x))
    if "inf" in r or "nan" in r:
        raise UnsupportedProgram(f"non-finite constant {x}")
    return r + "f"


# ---------------------------------------------------------------------------
# Flash lowering
# ---------------------------------------------------------------------------
FLASH_BM = {32: (1, 1), 64: (2, 1), 128: (4, 1), 256: (8, 1)}   # block_m -> default (waves, query blocks/wave)

# Schedule knobs of a flash-lowered stage (ParallelLoop.knobs), with their
# choices: "qb" 32-query blocks per wave (the workgroup then has
# block_m / (32 qb) waves; 2 halves the LDS fragment reads per MFMA at twice
# the registers, head dim 64 only) and "pipe" the software-pipelined
# schedule that issues the next key tile's score MFMAs during this tile's
# softmax; "w2" the two-waves-per-SIMD body with the hand-ordered main loop
# (256 x 64 tiles, N a multiple of 256: gr_flash_w2.h for fp16, head dim 64,
# non-causal, scale log2(e) <= 1; gr_flash_w2h.h for fp16 or bf16, head dim
# 128, causal or not), on by default where it applies.
FLASH_KNOBS = {"qb": (1, 2), "pipe": (0, 1), "w2": (0, 1)}
FLASH_KNOB_DEFAULTS = {"qb": 1, "pipe": 0, "w2": 1}     # what an absent knob means
KNOB_DEFAULTS = {**FLASH_KNOB_DEFAULTS, "ksplit": 1, "waves": 4}


FLASH_DEFAULT_BN = {64: 128, 128: 64}    # key tile when the stage does not tile the key axis

# fp32 flash stages (gr_flash_f32.h): each wave owns 32 queries and a chunk of
# BN keys, and the stage's partials live in module-scope device arrays, capped
# at this many bytes; the chunk defaults to N / 16 keys (at least 32)
FLASH32_WS_LIMIT = 32 << 20


def _flash_scores(x, scope_ids):
    """Walk the score operand of a softmax_matmul down to its Q K^T product.
    Accepts [causal] and [mulc] (either order, at most one each) over a
    matmul(Load Q, Load KT) that is bare or the sole partial of a
    ReductionLoop over the head dim. Returns (causal, scale, qload, ktload,
    nodes) or None; every node must be in `scope_ids`."""
    causal, scale, nodes = False, 1.0, []
    seen_mulc = False
    while isinstance(x, Compute) and x.op in ("causal", "mulc"):
        if id(x) not in scope_ids:
            return None
        if x.op == "causal":
            if causal:
                return None
            causal = True
            cax = x.axis
        else:
            if seen_mulc:
                return None
            seen_mulc, scale = True, float(x.const)
        nodes.append(x)
        x = x.inputs[0]
    if id(x) not in scope_ids:
        return None
    dloop = None
    if isinstance(x, ReductionLoop):
        dloop = x
        if len(dloop.partials) != 1 or not all(isinstance(s, (Load, Compute)) for s in dloop.body):
            return None
        nodes.append(dloop)
        nodes.extend(dloop.body)
        x = dloop.partial
    if not (isinstance(x, Compute) and x.op == "matmul"):
        return None
    if dloop is not None and (dloop.axis != _contraction_axis(x) or
                              any(isinstance(s, Compute) and s is not x for s in dloop.body)):
        return None
    qload, ktload = x.inputs
    if not (isinstance(qload, Load) and isinstance(ktload, Load)):
        return None
    nodes += [x, qload, ktload]
    return causal, scale, qload, ktload, nodes


def _match_flash(loop: ParallelLoop, program: Program):
    """Return the flash parameters if `loop` is one attention stage, else None:
    O = softmax_matmul(x, V) over the key axis j -- bare (full key range) or
    the sole partial of a ReductionLoop over j -- with x the scaled and
    optionally causally masked Q K^T of `_flash_scores`, and nothing else."""
    if program.dtype not in ("fp16", "bf16", "fp32"):
        return None
    stores = [s for s in loop.body if isinstance(s, Store)]
    if len(stores) != 1 or stores[0].dest != loop.out:
        return None
    st = stores[0]
    src = st.src
    rl = None
    if isinstance(src, ReductionLoop):
        rl = src
        if len(rl.partials) != 1:
            return None
        smm = rl.partial
        if not (isinstance(smm, Compute) and smm.op == "softmax_matmul" and smm.axis == rl.axis):
            return None
    elif isinstance(src, Compute) and src.op == "softmax_matmul":
        smm = src
    else:
        return None
    x, vload = smm.inputs
    if not isinstance(vload, Load):
        return None

    def walk(body):
        for s in body:
            yield s
            if isinstance(s, ReductionLoop):
                yield from walk(s.body)
    every = list(walk(loop.body))
    found = _flash_scores(x, {id(s) for s in every})
    if found is None:
        return None
    causal, scale, qload, ktload, nodes = found
    allowed = {id(st), id(smm), id(vload)} | {id(n) for n in nodes}
    if rl is not None:
        allowed.add(id(rl))
    if any(id(s) not in allowed for s in every):
        return None
    jax = smm.axis
    T = program.tensors
    qs, kts, vs, os_ = T[qload.source], T[ktload.source], T[vload.source], T[loop.out]
    nb = len(qs) - 2
    if nb < 0 or len(kts) != len(qs) or len(vs) != len(qs) or len(os_) != len(qs):
        return None
    iv = list(loop.index_vars)
    if len(iv) != len(qs):
        return None
    bax, iax, dax = iv[:nb], iv[nb], iv[nb + 1]
    if any(n.op == "causal" and n.axis != jax for n in nodes if isinstance(n, Compute)):
        return None
    dred = _contraction_axis(nodes[-3]) if isinstance(nodes[-3], Compute) else None
    if dred is None or qload.index != bax + [iax, dred] or ktload.index != bax + [dred, jax] or \
            vload.index != bax + [jax, dax] or st.index != bax + [iax, dax]:
        return None
    N, D = qs[-2], qs[-1]
    if tuple(kts[-2:]) != (D, N) or tuple(vs[-2:]) != (N, D) or tuple(os_) != tuple(qs) or \
            tuple(kts[:nb]) != tuple(qs[:nb]) or tuple(vs[:nb]) != tuple(qs[:nb]):
        return None
    tile = loop.tile_shape
    if any(t != 1 for t in tile[:nb]):
        return None
    if D not in (64, 128):
        return None
    if program.dtype == "fp32":
        return _match_flash32(loop, rl, tile, nb, N, D, causal, scale, qload, ktload, vload, _prod(qs[:nb]))
    BM = tile[nb]
    BN = rl.tile if rl is not None else FLASH_DEFAULT_BN[D]
    if tile[nb + 1] < D:
        return None
    if BM not in FLASH_BM or BN not in (32, 64, 128):
        return None
    if D == 128 and BN > 64:
        return None
    if N % BM or N % BN:
        return None
    nw, qb = FLASH_BM[BM]
    knobs = getattr(loop, "knobs", {}) or {}
    want_qb = int(knobs.get("qb", qb))
    if want_qb in FLASH_KNOBS["qb"] and BM % (32 * want_qb) == 0 and not (D == 128 and want_qb > 1):
        qb, nw = want_qb, BM // (32 * want_qb)        # a choice the tile cannot take keeps the default
    pipe = 1 if int(knobs.get("pipe", 0)) else 0
    if D == 128 and qb > 1:
        return None
    w2_ok = BM == 256 and BN == 64 and N % 256 == 0 and (
        (program.dtype == "fp16" and D == 64 and not causal and scale * LOG2E <= 1.0) or
        (program.dtype in ("fp16", "bf16") and D == 128))
    w2 = w2_ok and bool(int(knobs.get("w2", FLASH_KNOB_DEFAULTS["w2"])))
    if w2:
        qb, nw, pipe = 1, 8, 0
    return {"q": qload.source, "kt": ktload.source, "v": vload.source, "o": loop.out,
            "lead": _prod(qs[:nb]), "N": N, "D": D, "BM": BM, "BN": BN, "NW": nw, "QB": qb,
            "pipe": pipe, "causal": causal, "scale": scale, "w2_ok": w2_ok, "W2": w2}


def _match_flash32(loop, rl, tile, nb, N, D, causal, scale, qload, ktload, vload, lead):
    """fp32 flash stage parameters (gr_flash_f32.h): non-causal. A workgroup
    owns 32 queries and NW = block_m / 32 chunks of block_n keys (the key
    reduction tile, else 32), one per wave; PARTS = N / (NW block_n)
    workgroups per query block leave partials in module-scope device arrays
    (capped at FLASH32_WS_LIMIT bytes) that the last of them merges."""
    if causal or tile[nb + 1] < D:
        return None
    BM = tile[nb]
    BN = rl.tile if rl is not None else 32
    if BM not in FLASH_BM or BN % 32:
        return None
    nw = BM // 32
    if (D // nw) % 16 or N % 32 or N % (nw * BN):
        return None
    parts = N // (nw * BN)
    if parts > 1 and parts * lead * N * (D + 2) * 4 > FLASH32_WS_LIMIT:
        return None
    return {"q": qload.source, "kt": ktload.source, "v": vload.source, "o": loop.out, "lead": lead,
            "N": N, "D": D, "BM": BM, "BN": BN, "NW": nw, "QB": 1, "pipe": 0, "causal": False,
            "scale": scale, "f32": True, "parts": parts}


def template_tilings(loop: ParallelLoop, program: Program) -> list:
    """Output tile shapes at which `loop` lowers to a hand-written template
    (the flash or the GEMM kernel), whatever its current tiling: the
    candidates the descent tries as one joint move of the stage's tile dims.
    Empty for stages no template takes, or pinned to the generic lowering."""
    if (getattr(loop, "knobs", None) or {}).get("lowering") == "generic":
        return []
    out_shape = program.tensors[loop.out]
    nb = len(out_shape) - 2
    if nb < 0:
        return []
    lead = (1,) * nb
    cols = GEMM_F32_TILES if program.dtype == "fp32" else tuple(sorted(GEMM_WAVES_N))
    gemm_rows = GEMM_F32_TILES if program.dtype == "fp32" else tuple(sorted(GEMM_WAVES_M))
    cands = [lead + (bm, out_shape[-1]) for bm in sorted(FLASH_BM)] + \
        [lead + (bm, bn) for bm in gemm_rows for bn in cols]
    keep = loop.tile_shape
    found = []
    try:
        for shape in cands:
            if any(t > e for t, e in zip(shape, out_shape)) or shape in found:
                continue
            loop.tile_shape = shape
            if _match_flash(loop, program) is not None or _match_gemm(loop, program) is not None:
                found.append(shape)
    finally:
        loop.tile_shape = keep
    return found


def schedule_knobs(loop: ParallelLoop, program: Program) -> dict:
    """The schedule knobs the renderer honours for this stage, each with its
    choices and current value: {name: (choices, current)}: the flash kernel's
    query blocks per wave and pipelined schedule, the fp32 GEMM's split K,
    the 16-bit 256 x 256 GEMM's waves, the flash body with two waves per SIMD
    (which, when on, is the only flash knob offered: the other two do not
    apply to it); empty for other stages."""
    f = _match_flash(loop, program)
    if f is None:
        gm = _match_gemm(loop, program)
        if gm is not None and gm.get("f32"):
            return {"ksplit": (GEMM_KSPLIT, gm["ksplit"])}
        if gm is not None and gm.get("w4_ok"):
            return {"waves": (GEMM_TILE_WAVES, gm["waves"])}
        return {}
    if f.get("f32"):
        return {}
    if f.get("W2"):
        return {"w2": (FLASH_KNOBS["w2"], 1)}
    out = {"pipe": (FLASH_KNOBS["pipe"], f["pipe"])}
    if f["D"] == 64:
        out["qb"] = (FLASH_KNOBS["qb"], f["QB"])
    if f.get("w2_ok"):
        out["w2"] = (FLASH_KNOBS["w2"], 0)
    return out


def _render_flash32(loop, program, f) -> tuple:
    """The fp32 flash stage: one kernel, or with PARTS > 1 workgroups per
    query block a second one that merges their partials (two plan steps)."""
    kname = f"{_cname(loop.out)}_kernel"
    args = _loop_tensors(loop)
    params = ", ".join(f"{'const ' if a != loop.out else ''}float* __restrict__ {_cname(a)}" for a in args)
    N, D, lead, parts, nw = f["N"], f["D"], f["lead"], f["parts"], f["NW"]
    ws = _cname(loop.out)
    setup = f"""  gr_attn_args a;
  a.q = {_cname(f['q'])}; a.k = {_cname(f['kt'])}; a.v = {_cname(f['v'])}; a.o = {_cname(f['o'])};
  a.q_sb = {N * D}LL; a.q_sh = 0; a.q_sn = {D};
  a.k_sb = {N * D}LL; a.k_sh = 0; a.k_sn = {N};
  a.v_sb = {N * D}LL; a.v_sh = 0; a.v_sn = {D};
  a.o_sb = {N * D}LL; a.o_sh = 0; a.o_sn = {D};
  a.B = {lead}; a.H = 1; a.N = {N}; a.Nq = {N};
  a.scale_log2 = {_flt(f['scale'] * LOG2E)};"""
    if parts > 1:
        arrays = (f"// partials of the {parts} workgroups of each query block, merged by {kname[:-7]}_merge_kernel;\n"
                  f"// they are this module's, so two launches of it must not overlap\n"
                  f"__device__ float gr_ws_{ws}[{parts * lead * N * D}];\n"
                  f"__device__ float gr_ml_{ws}[{parts * lead * N * 2}];\n")
        ptrs = f"gr_ws_{ws}, gr_ml_{ws}"
    else:
        arrays, ptrs = "", "nullptr, nullptr"
    code = f"""
// stage {loop.out}: fp32 flash attention on the fp32 matrix cores (32 queries x {nw} chunk(s) of {f['BN']} keys
// per workgroup, one chunk per wave, merged in LDS; {parts} workgroup(s) per query block)
{arrays}extern "C" __global__ __launch_bounds__({nw * 64})
void {kname}({params}) {{
  extern __shared__ __attribute__((aligned(16))) char gr_flash_smem[];
{setup}
  gr_flash32_fwd_body<{D}, {f['BN']}, {nw}, true, {parts}>(a, gr_flash_smem, {ptrs});
}}
"""
    grid = lead * (N // 32) * parts
    lds = (nw * 32 * (D + 4) + nw * 32 * 2) * 4          # gr_flash32_lds<D, NW>::BYTES
    steps = [{"kernel": kname, "grid": [grid, 1, 1], "block": [nw * 64, 1, 1], "lds": lds,
              "args": args, "lowering": "flash",
              "tiles": {"block_m": f["BM"], "block_n": f["BN"], "waves": nw, "parts": parts}}]
    if parts > 1:
        mname = f"{kname[:-7]}_merge_kernel"
        code += f"""extern "C" __global__ __launch_bounds__(256)
void {mname}({params}) {{
{setup}
  gr_flash32_merge_body<{D}, {parts}>(a, gr_ws_{ws}, gr_ml_{ws});
}}
"""
        steps.append({"kernel": mname, "grid": [_cdiv(lead * N * (D // 8), 256), 1, 1], "block": [256, 1, 1],
                      "lds": 0, "args": args, "lowering": "flash", "merge": True})
    return code, steps


def _render_flash(loop, program, f) -> tuple:
    if f.get("f32"):
        return _render_flash32(loop, program, f)
    T = CTYPE[program.dtype]
    kname = f"{_cname(loop.out)}_kernel"
    args = _loop_tensors(loop)
    params = ", ".join(f"{'const ' if a != loop.out else ''}{T}* __restrict__ {_cname(a)}" for a in args)
    N, D = f["N"], f["D"]
    if f.get("W2"):
        return _render_flash_w2(loop, program, f, kname, args, params)
    pipe = "true" if f.get("pipe") else "false"
    nt = f["NW"] * 64
    # K^T / V tiles straight into LDS when each thread moves whole 16-byte chunks
    direct = "true" if (D * f["BN"] // 8) % nt == 0 else "false"
    code = f"""
// stage {loop.out}: flash attention (online softmax over key tiles of {f['BN']}, {f['BM']} queries/workgroup,
// {f['NW']} waves of {f['QB']} x 32 queries{', software-pipelined' if f.get('pipe') else ''})
extern "C" __global__ __launch_bounds__({nt})
__attribute__((amdgpu_waves_per_eu(gr_flash_wpe<{D}, {f['BN']}, {f['NW']}, {f['QB']}, true, {pipe}>::value)))
void {kname}({params}) {{
  extern __shared__ __attribute__((aligned(16))) char gr_flash_smem[];
  gr_attn_args a;
  a.q = {_cname(f['q'])}; a.k = {_cname(f['kt'])}; a.v = {_cname(f['v'])}; a.o = {_cname(f['o'])};
  a.q_sb = {N * D}LL; a.q_sh = 0; a.q_sn = {D};
  a.k_sb = {N * D}LL; a.k_sh = 0; a.k_sn = {N};
  a.v_sb = {N * D}LL; a.v_sh = 0; a.v_sn = {D};
  a.o_sb = {N * D}LL; a.o_sh = 0; a.o_sn = {D};
  a.B = {f['lead']}; a.H = 1; a.N = {N}; a.Nq = {N};
  a.kchunk = {N}; a.part_o = nullptr; a.part_ml = nullptr;
  a.scale_log2 = {_flt(f['scale'] * LOG2E)};
  gr_flash_fwd_body<{T}, {D}, {f['BN']}, {f['NW']}, {f['QB']}, {'true' if f['causal'] else 'false'}, true, {pipe}, true, {direct}>(a, gr_flash_smem);
}}
"""
    grid = f["lead"] * (N // f["BM"])
    lds = 2 * (f["BN"] * D * 2 + D * f["BN"] * 2)
    return code, {"kernel": kname, "grid": [grid, 1, 1], "block": [nt, 1, 1], "lds": lds,
                  "args": args, "lowering": "flash",
                  "tiles": {"block_m": f["BM"], "block_n": f["BN"], "waves": f["NW"], "qb": f["QB"],
                            "pipe": f.get("pipe", 0), "causal": bool(f["causal"])}}


def _render_flash_w2(loop, program, f, kname, args, params) -> tuple:
    """A flash stage on a two-waves-per-SIMD body: 256 queries per workgroup as
    8 waves of 32, 64-key tiles; at head dim 64 gr_flash_w2_body (two 8-slot
    LDS rings with per-wave Q / O areas), at 128 gr_flash_w2h_body (two 5-slot
    rings, Q and O staged through them); 160 KiB of LDS either way."""
    N, D = f["N"], f["D"]
    if D == 128:
        body = f"gr_flash_w2h_body<{CTYPE[program.dtype]}, {'true' if f['causal'] else 'false'}>(a, gr_flash_smem);"
        lds = FLASH_W2H_LDS
    else:
        body = "gr_flash_w2_body<true>(a, gr_flash_smem);"
        lds = FLASH_W2_LDS
    code = f"""
// stage {loop.out}: flash attention, two waves per SIMD with a hand-ordered main loop
// (256 queries/workgroup as 8 waves of 32, 64-key tiles)
extern "C" __global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2)))
void {kname}({params}) {{
  extern __shared__ __attribute__((aligned(16))) char gr_flash_smem[];
  gr_attn_args a;
  a.q = {_cname(f['q'])}; a.k = {_cname(f['kt'])}; a.v = {_cname(f['v'])}; a.o = {_cname(f['o'])};
  a.q_sb = {N * D}LL; a.q_sh = 0; a.q_sn = {D};
  a.k_sb = {N * D}LL; a.k_sh = 0; a.k_sn = {N};
  a.v_sb = {N * D}LL; a.v_sh = 0; a.v_sn = {D};
  a.o_sb = {N * D}LL; a.o_sh = 0; a.o_sn = {D};
  a.B = {f['lead']}; a.H = 1; a.N = {N}; a.Nq = {N};
  a.kchunk = {N}; a.part_o = nullptr; a.part_ml = nullptr;
  a.scale_log2 = {_flt(f['scale'] * LOG2E)};
  {body}
}}
"""
    grid = f["lead"] * (N // 256)
    return code, {"kernel": kname, "grid": [grid, 1, 1], "block": [512, 1, 1], "lds": lds,
                  "args": args, "lowering": "flash",
                  "tiles": {"block_m": 256, "block_n": 64, "waves": 8, "qb": 1, "pipe": 0,
                            "causal": bool(f["causal"]), "w2": 1}}


# GR_FLASH_W2_LDS: K and V rings of 8 tiles of 8 KiB, 4 KiB of Q / O per wave
FLASH_W2_LDS = 2 * 8 * 64 * 64 * 2 + 8 * 32 * 64 * 2
# GR_FLASH_W2H_LDS: K^T and V rings of 5 tiles of 16 KiB
FLASH_W2H_LDS = 2 * 5 * 64 * 128 * 2


# ---------------------------------------------------------------------------
# GEMM lowering
# ---------------------------------------------------------------------------
GEMM_ACTS = {"relu": 1, "silu": 2}
GEMM_RES = 4          # epilogue flag: + a residual tensor (GR_EPI_RES)
# fp32 GEMM stages may split K over workgroups (schedule knob "ksplit"): the
# partial products go to a module-scope workspace (capped at this many bytes)
# and a second launch sums them and applies the epilogue
GEMM_KSPLIT = (1, 2, 4, 8)
GEMM_WS_LIMIT = 32 << 20
GEMM_WAVES_M = {32: 1, 64: 1, 128: 2, 256: 2}
GEMM_WAVES_N = {32: 1, 64: 1, 128: 2, 256: 2}
# 16-bit 256 x 256 tiles with 32- or 64-deep k tiles (schedule knob "waves"):
# 4 = one wave per SIMD, 128 x 128 each, the hand-ordered main loop of
# gr_gemm_w4_body (the default); 8 = two waves per SIMD, 128 x 64 each
# (gr_gemm_body)
GEMM_TILE_WAVES = (4, 8)


GEMM_CUS = 256                # compute units of the gfx950 parts this backend targets (MI355X, MI350X)


def _gemm_w4_lds(bk, bnt=256):
    """LDS bytes of the one-wave 256 x BNT body (gr_gemm_w4_lds): two
    64-deep or four 32-deep operand stages, or the staged output tile."""
    stages = 2 if bk == 64 else 4
    return max(stages * (256 + bnt) * bk * 2, 256 * bnt * 2)


def _gemm_w4_split(M, N, batch, cus=GEMM_CUS):
    """The column split of a one-wave 256 x 256 GEMM launch whose last round
    of workgroups would leave more than half of the CUs idle (the library's
    launch_gemm_w4 rule): (col0, main tiles, 256 x 128 tail tiles) with the
    columns from col0 on in the tail launch, or None."""
    mt, nt = _cdiv(M, 256), _cdiv(N, 256)
    nblk = mt * nt
    if batch != 1 or nblk <= cus:
        return None
    rounds = _cdiv(nblk, cus)
    last = nblk - (rounds - 1) * cus
    nt_main = (rounds - 1) * cus // mt
    col0 = nt_main * 256
    rest = mt * _cdiv(N - col0, 128)
    if 2 * last <= cus and 0 < nt_main < nt and rest <= cus:
        return col0, mt * nt_main, rest
    return None


def _gemm_lds(bm, bn, bk):
    """LDS bytes of the GEMM kernel: two operand stages, or the staged output
    tile (gr_gemm_cfg::LDS)."""
    return max(2 * (bm + bn) * bk * 2, bm * bn * 2)


GEMM_F32_TILES = (32, 64, 128)


def _gemm_f32_lds(bm, bn, bk, kmajor):
    """LDS bytes of gr_gemm_f32_cfg: two stages of padded fp32 tiles."""
    a = bm * (bk + 4)
    b = bn * (bk + 4) if kmajor else bk * (bn + 8)
    return 2 * 4 * (a + b)


def _gemm_waves(bm, bn):
    wgm, wgn = GEMM_WAVES_M[bm], GEMM_WAVES_N[bn]
    if bm == 256 and bn == 256:
        wgn = 4
    return wgm, wgn


def _match_gemm(loop: ParallelLoop, program: Program):
    """Return the GEMM parameters if `loop` computes act(alpha * A @ B) from two
    loaded operands (the matmul over its contraction axis, at full extent or
    in one ReductionLoop, then mulc* and at most one relu/silu), else None.
    fp16/bf16 stages take gr_gemm.h, fp32 stages gr_gemm_f32.h (fp32 matrix
    cores; tiles of 32, 64 or 128 dividing M and N)."""
    if program.dtype not in ("fp16", "bf16", "fp32"):
        return None
    stores = [s for s in loop.body if isinstance(s, Store)]
    if len(stores) != 1 or stores[0].dest != loop.out:
        return None
    st = stores[0]
    x, alpha, act = st.src, 1.0, 0
    # outermost, optionally: + R, a tensor loaded at the output's own indices
    # (a residual add, fused as the GR_EPI_RES epilogue)
    res = resadd = None
    if isinstance(x, Compute) and x.op == "add" and len(x.inputs) == 2:
        for r_, other in ((x.inputs[1], x.inputs[0]), (x.inputs[0], x.inputs[1])):
            if isinstance(r_, Load) and r_.index == st.index and r_.source != loop.out and \
                    tuple(program.tensors[r_.source]) == tuple(program.tensors[loop.out]):
                res, resadd, x = r_, x, other
                break
    chain = []
    while isinstance(x, Compute) and x.op in ("mulc", "relu", "silu"):
        chain.append(x)
        x = x.inputs[0]
    for c in reversed(chain):            # innermost first: mulc* then one activation
        if c.op == "mulc":
            if act:
                return None
            alpha *= float(c.const)
        else:
            if act:
                return None
            act = GEMM_ACTS[c.op]
    rl = None
    if isinstance(x, ReductionLoop):
        rl = x
        if len(rl.partials) != 1 or any(isinstance(s, ReductionLoop) for s in rl.body):
            return None
        mm = rl.partial
        if not (isinstance(mm, Compute) and mm.op == "matmul"):
            return None
    elif isinstance(x, Compute) and x.op == "matmul":
        mm = x
    else:
        return None
    aload, bload = mm.inputs
    if not (isinstance(aload, Load) and isinstance(bload, Load)):
        return None
    allowed = {id(st), id(mm), id(aload), id(bload)} | {id(c) for c in chain}
    if res is not None:
        allowed |= {id(res), id(resadd)}
        act |= GEMM_RES
    if rl is not None:
        allowed.add(id(rl))
        if rl.axis != _contraction_axis(mm):
            return None
    body = list(loop.body) + (list(rl.body) if rl is not None else [])
    if any(id(s) not in allowed for s in body):
        return None
    T = program.tensors
    out = T[loop.out]
    nb = len(out) - 2
    iv = list(loop.index_vars)
    if nb < 0 or len(iv) != len(out):
        return None
    bax, iax, jax = iv[:nb], iv[nb], iv[nb + 1]
    kax = _contraction_axis(mm)
    if st.index != bax + [iax, jax]:
        return None
    ash, bsh = T[aload.source], T[bload.source]
    # A: [lead?, M, K]; B: [lead?, K, N] or K-major [lead?, N, K]; lead == bax or absent
    def lead_ok(ld, shape):
        lead = ld.index[:-2]
        if lead == bax:
            return tuple(shape[:-2]) == tuple(out[:nb]), True
        return (len(lead) == 0 or all(shape[d] == 1 for d in range(len(lead)))), False
    if aload.index[-2:] != [iax, kax]:
        return None
    if bload.index[-2:] == [kax, jax]:
        kmajor = False
    elif bload.index[-2:] == [jax, kax]:
        kmajor = True
    else:
        return None
    a_ok, a_batched = lead_ok(aload, ash)
    b_ok, b_batched = lead_ok(bload, bsh)
    if not (a_ok and b_ok) or not a_batched and nb > 0 and _prod(out[:nb]) > 1:
        return None
    M, K = ash[-2], ash[-1]
    N = bsh[-2] if kmajor else bsh[-1]
    if (bsh[-1] if kmajor else bsh[-2]) != K or tuple(out[-2:]) != (M, N):
        return None
    tile = loop.tile_shape
    if any(t != 1 for t in tile[:nb]):
        return None
    BM, BN = tile[nb], tile[nb + 1]
    batch = _prod(out[:nb])
    if program.dtype == "fp32":
        if BM not in GEMM_F32_TILES or BN not in GEMM_F32_TILES or M % BM or N % BN or K % 8:
            return None
        BK = rl.tile if rl is not None and rl.tile in (8, 16, 32) and K % rl.tile == 0 else \
            (32 if K % 32 == 0 else 16 if K % 16 == 0 else 8)
        # split K over workgroups (schedule knob "ksplit"): a choice the shape
        # cannot take (K / ksplit not a multiple of BK, or a workspace past the
        # cap) keeps one part
        ks = int((getattr(loop, "knobs", None) or {}).get("ksplit", 1))
        if ks not in GEMM_KSPLIT or K % (ks * BK) or ks * batch * M * N * 4 > GEMM_WS_LIMIT:
            ks = 1
        return {"a": aload.source, "b": bload.source, "c": loop.out, "M": M, "N": N, "K": K, "batch": batch,
                "a_sb": M * K if a_batched else 0, "b_sb": K * N if b_batched else 0, "c_sb": M * N,
                "kmajor": kmajor, "act": act, "alpha": alpha, "BM": BM, "BN": BN, "BK": BK,
                "WGM": 2 if BM >= 64 else 1, "WGN": 2 if BN >= 64 else 1, "f32": True,
                "res": res.source if res is not None else None, "ksplit": ks}
    if BM not in GEMM_WAVES_M or BN not in GEMM_WAVES_N:   # ragged M, N: edge tiles store their valid part
        return None
    BK = rl.tile if rl is not None else 64
    while BK > 16 and 2 * (BM + BN) * BK * 2 > LDS_LIMIT:
        BK //= 2
    if BK not in (16, 32, 64, 128) or K % BK:
        BK = 32 if K % 32 == 0 else (16 if K % 16 == 0 else 0)
    if not BK or _gemm_lds(BM, BN, BK) > LDS_LIMIT:
        return None
    if M * K % 8 or K * N % 8 or K % 8 or N % 8:
        return None
    wgm, wgn = _gemm_waves(BM, BN)
    w4_ok = BM == 256 and BN == 256 and BK in (32, 64)
    waves = int((getattr(loop, "knobs", None) or {}).get("waves", KNOB_DEFAULTS["waves"]))
    if waves not in GEMM_TILE_WAVES:
        waves = KNOB_DEFAULTS["waves"]
    return {"a": aload.source, "b": bload.source, "c": loop.out, "M": M, "N": N, "K": K, "batch": batch,
            "a_sb": M * K if a_batched else 0, "b_sb": K * N if b_batched else 0, "c_sb": M * N,
            "kmajor": kmajor, "act": act, "alpha": alpha, "BM": BM, "BN": BN, "BK": BK, "WGM": wgm, "WGN": wgn,
            "res": res.source if res is not None else None,
            "w4_ok": w4_ok, "waves": waves, "W4": w4_ok and waves == 4}


def _render_gemm_f32_split(loop, program, f, args, params, km) -> tuple:
    """An fp32 GEMM stage with K split over `ksplit` workgroups: the partial
    products go to a module-scope workspace, and a second launch sums them
    and applies alpha, the activation and the residual (two plan steps).
    With f["fuse_reduce"] (no activation; every consumer a row-lowered stage
    that sums the partials as it loads them) there is no second launch: each
    part applies alpha and the first part adds the residual."""
    ks, M, N, K, batch = f["ksplit"], f["M"], f["N"], f["K"], f["batch"]
    kname = f"{_cname(loop.out)}_kernel"
    rname = f"{_cname(loop.out)}_reduce_kernel"
    ws = f"gr_ws_{_cname(loop.out)}"
    nt = f["WGM"] * f["WGN"] * 64
    res_line = (f"\n  a.r = {_cname(f['res'])}; a.r_sb = {f['c_sb']}LL; a.r_sm = {N};" if f.get("res") else "")
    common = f"""  gr_gemm_args a;
  a.a = {_cname(f['a'])}; a.b = {_cname(f['b'])}; a.c = {_cname(f['c'])};
  a.a_sb = {f['a_sb']}LL; a.a_sm = {K};
  a.b_sb = {f['b_sb']}LL; a.b_s = {K if f['kmajor'] else N};
  a.c_sb = {f['c_sb']}LL; a.c_sm = {N};
  a.M = {M}; a.N = {N}; a.K = {K};
  a.alpha = {_flt(f['alpha'])};{res_line}"""
    if f.get("fuse_reduce"):
        code = f"""
// stage {loop.out}: fp32 MFMA GEMM {M}x{N}x{K} (x{batch}), tile {f['BM']}x{f['BN']}x{f['BK']}, K split over
// {ks} workgroups whose partial products (alpha applied, the residual added by the first) stay in this
// module's workspace: the stages reading {loop.out} sum them as they load it, so two runs of the module
// must not overlap
__device__ float {ws}[{ks * batch * M * N}];
extern "C" __global__ __launch_bounds__({nt})
void {kname}({params}) {{
  extern __shared__ __attribute__((aligned(16))) char gr_gemm_smem[];
{common}
  a.c = {ws}; a.c_sb = {M * N}LL;
  if (blockIdx.z != 0) a.r = nullptr;
  a.ksplit = {ks}; a.c_sz = {batch * M * N}LL;
  gr_gemm_f32_body<{f['BM']}, {f['BN']}, {f['BK']}, {f['WGM']}, {f['WGN']}, {km}, {f['act']}>(a, gr_gemm_smem);
}}
"""
        grid = (M // f["BM"]) * (N // f["BN"])
        return code, [{"kernel": kname, "grid": [grid, batch, ks], "block": [nt, 1, 1],
                       "lds": _gemm_f32_lds(f["BM"], f["BN"], f["BK"], f["kmajor"]), "args": args,
                       "lowering": "gemm", "tiles": {"block_m": f["BM"], "block_n": f["BN"], "block_k": f["BK"],
                                                     "ksplit": ks, "sum_in_consumer": True}}]
    code = f"""
// stage {loop.out}: fp32 MFMA GEMM {M}x{N}x{K} (x{batch}), tile {f['BM']}x{f['BN']}x{f['BK']}, K split over
// {ks} workgroups; their partial products live in this module's workspace between the two launches,
// so two runs of the module must not overlap
__device__ float {ws}[{ks * batch * M * N}];
extern "C" __global__ __launch_bounds__({nt})
void {kname}({params}) {{
  extern __shared__ __attribute__((aligned(16))) char gr_gemm_smem[];
{common}
  a.c = {ws}; a.c_sb = {M * N}LL; a.alpha = 1.0f; a.r = nullptr;
  a.ksplit = {ks}; a.c_sz = {batch * M * N}LL;
  gr_gemm_f32_body<{f['BM']}, {f['BN']}, {f['BK']}, {f['WGM']}, {f['WGN']}, {km}, 0>(a, gr_gemm_smem);
}}
extern "C" __global__ __launch_bounds__(256)
void {rname}({params}) {{
{common}
  gr_gemm_f32_reduce_body<{f['act']}>(a, {ws}, {ks}, {batch * M * N}LL, {batch});
}}
"""
    grid = (M // f["BM"]) * (N // f["BN"])
    steps = [{"kernel": kname, "grid": [grid, batch, ks], "block": [nt, 1, 1],
              "lds": _gemm_f32_lds(f["BM"], f["BN"], f["BK"], f["kmajor"]), "args": args, "lowering": "gemm",
              "tiles": {"block_m": f["BM"], "block_n": f["BN"], "block_k": f["BK"], "ksplit": ks}},
             {"kernel": rname, "grid": [_cdiv(batch * M * N // 4, 256), 1, 1], "block": [256, 1, 1], "lds": 0,
              "args": args, "lowering": "gemm", "merge": True}]
    return code, steps


def _render_gemm(loop, program, f) -> tuple:
    T = CTYPE[program.dtype]
    kname = f"{_cname(loop.out)}_kernel"
    args = _loop_tensors(loop)
    params = ", ".join(f"{'const ' if a != loop.out else ''}{T}* __restrict__ {_cname(a)}" for a in args)
    km = "true" if f["kmajor"] else "false"
    res_line = (f"\n  a.r = {_cname(f['res'])}; a.r_sb = {f['c_sb']}LL; a.r_sm = {f['N']};"
                if f.get("res") else "")
    if f.get("f32") and f.get("ksplit", 1) > 1:
        return _render_gemm_f32_split(loop, program, f, args, params, km)
    if f.get("f32"):
        nt = f["WGM"] * f["WGN"] * 64
        code = f"""
// stage {loop.out}: fp32 MFMA GEMM {f['M']}x{f['N']}x{f['K']} (x{f['batch']}), tile {f['BM']}x{f['BN']}x{f['BK']}
extern "C" __global__ __launch_bounds__({nt})
void {kname}({params}) {{
  extern __shared__ __attribute__((aligned(16))) char gr_gemm_smem[];
  gr_gemm_args a;
  a.a = {_cname(f['a'])}; a.b = {_cname(f['b'])}; a.c = {_cname(f['c'])};
  a.a_sb = {f['a_sb']}LL; a.a_sm = {f['K']};
  a.b_sb = {f['b_sb']}LL; a.b_s = {f['K'] if f['kmajor'] else f['N']};
  a.c_sb = {f['c_sb']}LL; a.c_sm = {f['N']};
  a.M = {f['M']}; a.N = {f['N']}; a.K = {f['K']};
  a.alpha = {_flt(f['alpha'])};{res_line}
  gr_gemm_f32_body<{f['BM']}, {f['BN']}, {f['BK']}, {f['WGM']}, {f['WGN']}, {km}, {f['act']}>(a, gr_gemm_smem);
}}
"""
        grid = (f["M"] // f["BM"]) * (f["N"] // f["BN"])
        return code, {"kernel": kname, "grid": [grid, f["batch"], 1], "block": [nt, 1, 1],
                      "lds": _gemm_f32_lds(f["BM"], f["BN"], f["BK"], f["kmajor"]), "args": args,
                      "lowering": "gemm", "tiles": {"block_m": f["BM"], "block_n": f["BN"], "block_k": f["BK"]}}
    if f.get("W4"):
        def w4_kernel(name, col0, ncols, bnt, what):
            # columns col0 .. col0 + ncols of C (B, C and R offset by col0)
            boff = f"{col0} * {f['K']}LL" if f["kmajor"] else f"{col0}LL"
            rl = (f"\n  a.r = {_cname(f['res'])} + {col0}LL; a.r_sb = {f['c_sb']}LL; a.r_sm = {f['N']};"
                  if f.get("res") else "")
            return f"""
// stage {loop.out}: MFMA GEMM {f['M']}x{f['N']}x{f['K']} (x{f['batch']}), {what},
// four waves of 128 x {bnt // 2} (one per SIMD, hand-ordered main loop)
extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1)))
void {name}({params}) {{
  extern __shared__ __attribute__((aligned(16))) char gr_gemm_smem[];
  gr_gemm_args a;
  a.a = {_cname(f['a'])}; a.b = {_cname(f['b'])} + {boff}; a.c = {_cname(f['c'])} + {col0}LL;
  a.a_sb = {f['a_sb']}LL; a.a_sm = {f['K']};
  a.b_sb = {f['b_sb']}LL; a.b_s = {f['K'] if f['kmajor'] else f['N']};
  a.c_sb = {f['c_sb']}LL; a.c_sm = {f['N']};
  a.M = {f['M']}; a.N = {ncols}; a.K = {f['K']};
  a.alpha = {_flt(f['alpha'])};{rl}
  gr_gemm_w4_body<{T}, {km}, {f['act']}, {f['BK']}, {bnt}>(a, gr_gemm_smem);
}}
"""
        tiles = {"block_m": 256, "block_n": 256, "block_k": f["BK"], "waves": 4}
        split = _gemm_w4_split(f["M"], f["N"], f["batch"])
        if split is None:
            code = w4_kernel(kname, 0, f["N"], 256, f"tile 256x256x{f['BK']}")
            grid = _cdiv(f["M"], 256) * _cdiv(f["N"], 256)
            return code, {"kernel": kname, "grid": [grid, f["batch"], 1], "block": [256, 1, 1],
                          "lds": _gemm_w4_lds(f["BK"]), "args": args, "lowering": "gemm", "tiles": tiles}
        # a last round of at most half the CUs: the columns past the whole
        # rounds go to a second launch of the body on 256 x 128 tiles
        col0, nmain, ntail = split
        tname = f"{_cname(loop.out)}_tail_kernel"
        code = (w4_kernel(kname, 0, col0, 256, f"columns 0-{col0 - 1}, tile 256x256x{f['BK']}")
                + w4_kernel(tname, col0, f["N"] - col0, 128,
                            f"columns {col0}-{f['N'] - 1}, tile 256x128x{f['BK']}"))
        return code, [{"kernel": kname, "grid": [nmain, 1, 1], "block": [256, 1, 1],
                       "lds": _gemm_w4_lds(f["BK"]), "args": args, "lowering": "gemm", "tiles": tiles},
                      {"kernel": tname, "grid": [ntail, 1, 1], "block": [256, 1, 1],
                       "lds": _gemm_w4_lds(f["BK"], 128), "args": args, "lowering": "gemm", "tail": True,
                       "tiles": {**tiles, "block_n": 128, "col0": col0}}]
    tpl = f"{T}, {f['BM']}, {f['BN']}, {f['BK']}, {f['WGM']}, {f['WGN']}, {km}, {f['act']}"
    nt = f["WGM"] * f["WGN"] * 64
    code = f"""
// stage {loop.out}: MFMA GEMM {f['M']}x{f['N']}x{f['K']} (x{f['batch']}), tile {f['BM']}x{f['BN']}x{f['BK']}
extern "C" __global__ __launch_bounds__({nt})
__attribute__((amdgpu_waves_per_eu(gr_gemm_wpe<{f['BM']}, {f['BN']}, {f['BK']}, {f['WGM']}, {f['WGN']}, {km}>::value)))
void {kname}({params}) {{
  extern __shared__ __attribute__((aligned(16))) char gr_gemm_smem[];
  gr_gemm_args a;
  a.a = {_cname(f['a'])}; a.b = {_cname(f['b'])}; a.c = {_cname(f['c'])};
  a.a_sb = {f['a_sb']}LL; a.a_sm = {f['K']};
  a.b_sb = {f['b_sb']}LL; a.b_s = {f['K'] if f['kmajor'] else f['N']};
  a.c_sb = {f['c_sb']}LL; a.c_sm = {f['N']};
  a.M = {f['M']}; a.N = {f['N']}; a.K = {f['K']};
  a.alpha = {_flt(f['alpha'])};{res_line}
  gr_gemm_body<{tpl}>(a, gr_gemm_smem);
}}
"""
    grid = -(-f["M"] // f["BM"]) * -(-f["N"] // f["BN"])
    lds = _gemm_lds(f["BM"], f["BN"], f["BK"])
    return code, {"kernel": kname, "grid": [grid, f["batch"], 1], "block": [nt, 1, 1], "lds": lds,
                  "args": args, "lowering": "gemm",
                  "tiles": {"block_m": f["BM"], "block_n": f["BN"], "block_k": f["BK"]}}


# ---------------------------------------------------------------------------
# Row lowering: pointwise stages and stages whose reductions run over the last
# axis (row max / row sum, softmax pieces, LayerNorm). HBM-bound: one wave per
# row, vectorised loads and stores, reductions by wave shuffles, nothing
# staged in LDS.
# ---------------------------------------------------------------------------
ROW_WAVES = 4                 # waves (rows) per workgroup


def _match_rows(loop: ParallelLoop, program: Program):
    """Parameters of the row lowering if every value of `loop` is either an
    element of a row (index = the loop's axes) or a per-row scalar (a row
    reduction over the last axis, or a load of a [..., 1] tensor), else None."""
    T = program.tensors
    iv = list(loop.index_vars)
    if len(iv) < 1:
        return None
    stores = [s for s in loop.body if isinstance(s, Store)]
    if len(stores) != 1 or stores[0].dest != loop.out or stores[0].index != iv:
        return None
    st = stores[0]
    out = tuple(T[loop.out])
    nodes, reds = [], {}

    def walk(body):
        for x in body:
            if isinstance(x, ReductionLoop):
                if x.axis != iv[-1] or any(not (isinstance(c, Compute) and c.op in ROW_REDUCE_OPS and
                                                c.axis == iv[-1]) for c in x.partials):
                    return False
                for c in x.partials:
                    reds[id(c)] = c
                if walk(x.body) is False:
                    return False
            elif isinstance(x, (Load, Compute)):
                nodes.append(x)
            elif not isinstance(x, Store):
                return False
        return True
    if walk(loop.body) is False:
        return None
    C = None
    for x in nodes:
        if isinstance(x, Load):
            if x.index != iv:
                return None
            sh = tuple(T[x.source])
            if len(sh) != len(out) or any(a != b and a != 1 for a, b in zip(sh[:-1], out[:-1])):
                return None
            if sh[-1] != 1:
                if C is not None and sh[-1] != C:
                    return None
                C = sh[-1]
        elif x.op in ROW_REDUCE_OPS:
            if x.axis != iv[-1]:
                return None
        elif x.op not in ELEMENTWISE_OPS:
            return None
        elif x.op == "causal" and (x.axis != iv[-1] or len(iv) < 2):
            return None
    if out[-1] != 1:
        if C is not None and out[-1] != C:
            return None
        C = out[-1]
    if C is None:
        return None
    kind = {}

    def k(v):
        """'e' (per element) or 's' (per row)."""
        if id(v) in kind:
            return kind[id(v)]
        if isinstance(v, ReductionLoop):
            r = "s"
        elif isinstance(v, Load):
            r = "e" if T[v.source][-1] != 1 else "s"
        elif v.op in ROW_REDUCE_OPS:
            if k(v.inputs[0]) != "e":
                raise UnsupportedProgram("row reduction of a per-row value")
            r = "s"
        elif v.op == "causal":
            r = "e"
        else:
            r = "e" if any(k(i) == "e" for i in v.inputs) else "s"
        kind[id(v)] = r
        return r
    try:
        ko = k(st.src)
    except (UnsupportedProgram, AttributeError):
        return None
    if (ko == "e") != (out[-1] != 1):
        return None
    rows = _prod(out[:-1])
    vec = 8 if C % 8 == 0 and C >= 512 else (4 if C % 4 == 0 and C >= 256 else 1)
    return {"C": C, "rows": rows, "vec": vec, "out": out, "store": st}


class _RowGen:
    def __init__(self, loop, program, f, fused=None):
        """fused: tensor -> (workspace, parts, part stride) for tensors a
        split-K GEMM stage left as partial products, summed here on load."""
        self.loop, self.p, self.f = loop, program, f
        self.fused = fused or {}
        self.T = CTYPE[program.dtype]
        self.lines = []
        self.n = 0
        self.scal = {}          # id(value) -> C name of a computed per-row scalar
        self.groups = {}        # id(partial) -> all partials of its multi-partial ReductionLoop

        def walk(body):
            for x in body:
                if isinstance(x, ReductionLoop):
                    if len(x.partials) > 1:
                        for c in x.partials:
                            self.groups[id(c)] = list(x.partials)
                    walk(x.body)
        walk(loop.body)

    def fresh(self, p):
        self.n += 1
        return f"{p}{self.n}"

    def row_load(self, nm, src):
        """Statement loading VEC row elements of `src` at column c0 into `nm`."""
        vec, off = self.f["vec"], self.row_off(src)
        if src in self.fused:
            ws, parts, stride = self.fused[src]
            return f"float {nm}[{vec}]; gr_row_load_parts<{vec}>({nm}, {ws} + {off} + c0, {stride}LL, {parts});"
        return f"float {nm}[{vec}]; gr_row_load<{vec}>({nm}, t_{src} + {off} + c0);"

    def scalar_load(self, src):
        """Expression of a per-row scalar of `src` (a [.., 1] tensor)."""
        off = self.row_off(src)
        if src in self.fused:
            ws, parts, stride = self.fused[src]
            return "(" + " + ".join(f"{ws}[{off} + {s * stride}LL]" for s in range(parts)) + ")"
        return f"(float)t_{src}[{off}]"

    def kind(self, v):
        if isinstance(v, ReductionLoop):
            return "s"
        if isinstance(v, Load):
            return "e" if self.p.tensors[v.source][-1] != 1 else "s"
        if v.op in ROW_REDUCE_OPS:
            return "s"
        if v.op == "causal":
            return "e"
        return "e" if any(self.kind(i) == "e" for i in v.inputs) else "s"

    def red_of(self, v):
        """(compute, op) if v is a row reduction value."""
        if isinstance(v, ReductionLoop):
            return v.partial
        if isinstance(v, Compute) and v.op in ROW_REDUCE_OPS:
            return v
        return None

    def row_off(self, name):
        """C expression: element offset of this row's start in tensor `name`
        (broadcast dims contribute nothing)."""
        sh = self.p.tensors[name]
        out = self.f["out"]
        st = _row_major(sh)
        terms = []
        rem = "row"
        # decompose the row index over out[:-1] (row-major)
        ost = _row_major(out[:-1]) if len(out) > 1 else ()
        for d in range(len(out) - 1):
            if out[d] == 1 or sh[d] == 1:
                continue
            coord = f"((row / {ost[d]}LL) % {out[d]}LL)" if d > 0 else f"(row / {ost[d]}LL)"
            terms.append(f"{coord} * {st[d]}LL")
        return " + ".join(terms) if terms else "0LL"

    def scalar(self, v, emit):
        """Emit code computing per-row scalar v (all lanes hold it)."""
        if id(v) in self.scal:
            return self.scal[id(v)]
        r = self.red_of(v)
        if r is not None:
            group = self.groups.get(id(r))
            if group is not None:
                # sibling partials of one ReductionLoop: one pass over the row
                names = self.reduction(group, emit)
                for c, nm in zip(group, names):
                    self.scal[id(c)] = nm
                return self.scal[id(r)]
            name = self.reduction([r], emit)[0]
        elif isinstance(v, Load):
            name = self.fresh("s")
            emit(f"const float {name} = {self.scalar_load(v.source)};")
        else:
            args = [self.scalar(i, emit) for i in v.inputs]
            name = self.fresh("s")
            emit(f"const float {name} = {_ew_expr(v.op, args, v.const)};")
        self.scal[id(v)] = name
        return name

    def element_code(self, v, loads, pre, memo):
        """C expression for element value v at column (c0 + k); loads collects
        the element loads needed; scalars are emitted into `pre`."""
        if id(v) in memo:
            return memo[id(v)]
        if self.kind(v) == "s":
            e = self.scalar(v, pre)
        elif isinstance(v, Load):
            loads.setdefault(v.source, self.fresh("x"))
            e = f"{loads[v.source]}[k]"
        elif v.op == "causal":
            a = self.element_code(v.inputs[0], loads, pre, memo)
            R = self.f["out"][-2] if len(self.f["out"]) >= 2 else 1
            e = f"((c0 + k) > (int)(row % {R}LL) ? -GR_INF : {a})"
        else:
            args = [self.element_code(i, loads, pre, memo) for i in v.inputs]
            e = f"({_ew_expr(v.op, args, v.const)})"
        memo[id(v)] = e
        return e

    def reduction(self, cs, emit):
        """Row reductions `cs` computed in one pass over the row; returns the
        names of their per-row results."""
        vec, C = self.f["vec"], self.f["C"]
        loads, memo, pre = {}, {}, []
        exprs = [self.element_code(c.inputs[0], loads, pre.append, memo) for c in cs]
        for x in pre:
            emit(x)
        accs = [self.fresh("r") for _ in cs]
        for c, acc in zip(cs, accs):
            emit(f"float {acc} = {'-GR_INF' if c.op == 'rowmax' else '0.f'};")
        emit(f"for (int c0 = lane * {vec}; c0 < {C}; c0 += {64 * vec}) {{")
        for src, nm in loads.items():
            emit(f"  {self.row_load(nm, src)}")
        emit(f"#pragma unroll")
        emit(f"  for (int k = 0; k < {vec}; ++k) {{")
        for c, acc, e in zip(cs, accs, exprs):
            emit(f"    {acc} = fmaxf({acc}, {e});" if c.op == "rowmax" else f"    {acc} += {e};")
        emit("  }")
        emit("}")
        for c, acc in zip(cs, accs):
            emit(f"{acc} = {'gr_wave_max' if c.op == 'rowmax' else 'gr_wave_sum'}({acc});")
        return accs

    def render(self):
        f = self.f
        loop = self.loop
        kname = f"{_cname(loop.out)}_kernel"
        args = _loop_tensors(loop)
        params = ", ".join(f"{'const ' if a != loop.out else ''}{self.T}* __restrict__ {_cname(a)}" for a in args)
        body = []
        emit = body.append
        st = f["store"]
        vec, C = f["vec"], f["C"]
        if f["out"][-1] == 1:
            val = self.scalar(st.src, emit)
            emit(f"if (lane == 0) t_{loop.out}[{self.row_off(loop.out)}] = ({self.T}){val};")
        else:
            loads, memo, pre = {}, {}, []
            expr = self.element_code(st.src, loads, pre.append, memo)
            for x in pre:
                emit(x)
            emit(f"for (int c0 = lane * {vec}; c0 < {C}; c0 += {64 * vec}) {{")
            for src, nm in loads.items():
                emit(f"  {self.row_load(nm, src)}")
            emit(f"  float y[{vec}];")
            emit(f"#pragma unroll")
            emit(f"  for (int k = 0; k < {vec}; ++k) y[k] = {expr};")
            emit(f"  gr_row_store<{vec}>(t_{loop.out} + {self.row_off(loop.out)} + c0, y);")
            emit("}")
        ind = "\n  ".join(body)
        code = f"""
// stage {loop.out}: row lowering ({f['rows']} rows x {C}, one wave per row, {vec}-wide accesses)
extern "C" __global__ __launch_bounds__({64 * ROW_WAVES})
void {kname}({params}) {{
  const int lane = threadIdx.x & 63;
  const long long row = (long long)blockIdx.x * {ROW_WAVES} + (threadIdx.x >> 6);
  if (row >= {f['rows']}LL) return;
  {ind}
}}
"""
        grid = _cdiv(f["rows"], ROW_WAVES)
        return code, {"kernel": kname, "grid": [grid, 1, 1], "block": [64 * ROW_WAVES, 1, 1], "lds": 0,
                      "args": args, "lowering": "rows", "tiles": {"vec": vec}}


# ---------------------------------------------------------------------------
# Generic lowering
# ---------------------------------------------------------------------------
class _View:
    """A tile as seen from the current scope: LDS base (floats), shape, the
    strides of the buffer it lives in, a dynamic offset expression, axes."""

    def __init__(self, base, shape, strides, dyn, axes, origin):
        self.base, self.shape, self.strides, self.dyn, self.axes = base, tuple(shape), tuple(strides), dyn, list(axes)
        self.origin = list(origin)     # C expression: global index of element 0, per axis

    def addr(self, idx_exprs) -> str:
        parts = [str(self.base)]
        if self.dyn:
            parts.append(f"({self.dyn})")
        for d, (e, s) in enumerate(zip(idx_exprs, self.strides)):
            if self.shape[d] > 1 and s:
                parts.append(f"({e})*{s}" if s != 1 else f"({e})")
        return " + ".join(parts)


def _row_major(shape):
    st, acc = [], 1
    for n in reversed(shape):
        st.append(acc)
        acc *= n
    return tuple(reversed(st))


class _StageGen:
    def __init__(self, loop: ParallelLoop, program: Program, shapes: dict, check: bool = False):
        self.loop, self.p, self.shapes = loop, program, shapes
        self.check = check
        self.T = CTYPE[program.dtype]
        self.lines = []
        self.ind = 1
        self.bufs = {}                 # LDS buffer name -> {size (floats), def, last}
        self.pos = 0                   # statement position (buffer lifetimes)
        self.nfl = 0                   # LDS floats after allocation
        self.vals = {}                 # id -> (base, shape, axes, depth, origin)
        self.loops = []                # enclosing ReductionLoops
        self.scope = {}                # index name -> C expression of its tile coordinate
        self.n = 0

    # -- helpers -----------------------------------------------------------
    def emit(self, s):
        self.lines.append("  " * self.ind + s)

    def fresh(self, p="v"):
        self.n += 1
        return f"{p}{self.n}"

    def alloc(self, shape) -> str:
        """A symbolic LDS buffer; offsets are assigned from lifetimes at the end."""
        name = f"B{len(self.bufs)}"
        self.bufs[name] = {"size": (max(1, _prod(shape)) + 3) & ~3, "def": self.pos, "last": self.pos}
        return name

    def touch(self, name):
        b = self.bufs[name]
        b["last"] = max(b["last"], self.pos)

    def step(self):
        self.pos += 1

    def assign_lds(self) -> list:
        """First-fit placement of buffers whose [def, last] intervals overlap."""
        placed, offs = [], {}
        for name in sorted(self.bufs, key=lambda n: (self.bufs[n]["def"], n)):
            b = self.bufs[name]
            conf = sorted((o, sz) for (o, sz, d, l) in placed if not (l < b["def"] or d > b["last"]))
            off = 0
            for o, sz in conf:
                if off + b["size"] <= o:
                    break
                off = max(off, o + sz)
            placed.append((off, b["size"], b["def"], b["last"]))
            offs[name] = off
        self.nfl = max((o + sz for o, sz, _, _ in placed), default=0)
        return [f"  constexpr int {n} = {offs[n]};" for n in sorted(offs, key=lambda x: int(x[1:]))]

    def sync_stmt(self) -> str:
        return "GR_SYNC();" if self.check else "__syncthreads();"

    def sync(self):
        self.emit(self.sync_stmt())

    # LDS and global accesses: plain in the product build; in the checking
    # build (gr_check.h) every LDS index is bounds- and race-checked and every
    # global index bounds-checked
    def lr(self, x) -> str:
        return f"GR_LR({x})" if self.check else f"gr_lds[{x}]"

    def lw(self, x) -> str:
        return f"GR_LW({x})" if self.check else f"gr_lds[{x}]"

    def gidx(self, i, n) -> str:
        return f"GR_GI({i}, {n}LL)" if self.check else i

    def define(self, node, base, shape, axes, origin):
        if len(origin) != len(axes):
            raise UnsupportedProgram("internal: origin/axes rank mismatch")
        self.vals[id(node)] = (base, tuple(shape), list(axes), len(self.loops), list(origin))

    def view(self, node) -> _View:
        if id(node) not in self.vals:
            raise UnsupportedProgram(f"value {type(node).__name__} used before it is produced")
        base, shape, axes, d0, origin = self.vals[id(node)]
        self.touch(base)
        strides = _row_major(shape)
        shape, origin = list(shape), list(origin)
        dyn = []
        for lp in self.loops[d0:]:
            if lp.axis in axes:
                p = axes.index(lp.axis)
                if shape[p] > lp.tile:
                    if shape[p] % lp.tile:
                        raise UnsupportedProgram("sub-tile does not divide the materialised tile")
                    dyn.append(f"GR_SUBTILE({self.loopvar(lp)}*{lp.tile * strides[p]})")
                    shape[p] = lp.tile
                    origin[p] = f"({origin[p]}) + {self.loopvar(lp)}*{lp.tile}"
        return _View(base, shape, strides, " + ".join(dyn), axes, origin)

    def loopvar(self, lp):
        return f"kk_{_cname(lp.axis)}_{id(lp) % 100000}"

    def elem_loop(self, shape, body_fn):
        """for (e in tile) with per-dim index names i0..; body_fn(idx_exprs, e)."""
        E = _prod(shape)
        self.emit(f"for (int e = threadIdx.x; e < {E}; e += {NT}) {{")
        self.ind += 1
        idx = []
        rem = "e"
        st = _row_major(shape)
        for d, n in enumerate(shape):
            if n == 1:
                idx.append("0")
                continue
            v = f"i{d}"
            if st[d] == 1:
                self.emit(f"const int {v} = {rem} % {n};" if d > 0 else f"const int {v} = {rem};")
            else:
                self.emit(f"const int {v} = ({rem} / {st[d]}){f' % {n}' if d > 0 else ''};")
            idx.append(v)
        body_fn(idx)
        self.ind -= 1
        self.emit("}")

    # -- statements ----------------------------------------------------------
    def gen_body(self, stmts, partial_acc=None):
        for s in stmts:
            self.step()
            if isinstance(s, Load):
                self.gen_load(s)
            elif isinstance(s, Compute):
                if partial_acc is not None and id(s) in partial_acc:
                    self.gen_partial(s, partial_acc[id(s)])
                else:
                    self.gen_compute(s)
            elif isinstance(s, ReductionLoop):
                self.gen_reduction(s)
            elif isinstance(s, Store):
                self.gen_store(s)
            else:
                raise UnsupportedProgram(f"statement {type(s).__name__}")

    def _coords(self, index, tile, g, what):
        names = _resolve_index(index, tile, g, set(self.scope), what)
        return [("0" if n == "0" else self.scope[n]) for n in names]

    def gen_load(self, s: Load):
        shp = self.shapes[id(s)]
        g = self.p.tensors[s.source]
        for t, gd in zip(shp, g):
            if (t < gd and gd % t) or (t > gd and gd != 1):
                raise UnsupportedProgram(f"load {s.source}: tile {t} does not tile extent {gd}")
        coords = self._coords(s.index, shp, g, f"load {s.source}")
        base = self.alloc(shp)
        gst = _row_major(g)
        src = _cname(s.source)

        def body(idx):
            terms = []
            for d, (c, t) in enumerate(zip(coords, shp)):
                if g[d] == 1:
                    continue
                ix = idx[d] if shp[d] > 1 else "0"
                e = f"({c})*{t} + {ix}" if c != "0" else ix
                terms.append(f"(long long)({e})*{gst[d]}" if gst[d] != 1 else f"(long long)({e})")
            gi = " + ".join(terms) if terms else "0"
            self.emit(f"{self.lw(f'{base} + e')} = (float){src}[{self.gidx(gi, _prod(g))}];")
        self.elem_loop(shp, body)
        self.sync()
        origin = [("0" if (c == "0" or g[d] == 1) else f"({c})*{shp[d]}") for d, c in enumerate(coords)]
        self.define(s, base, shp, s.index, origin)

    def gen_store(self, s: Store):
        v = self.view(s.src)
        g = self.p.tensors[s.dest]
        tile = self.shapes[id(s.src)]
        coords = self._coords(s.index, tile, g, f"store {s.dest}")
        gst = _row_major(g)
        dst = _cname(s.dest)
        if len(v.shape) != len(g):
            raise UnsupportedProgram("store rank mismatch")

        def body(idx):
            terms, conds = [], []
            for d, c in enumerate(coords):
                if g[d] == 1:
                    continue
                ix = idx[d] if v.shape[d] > 1 else "0"
                e = f"({c})*{tile[d]} + {ix}" if c != "0" else ix
                terms.append(f"(long long)({e})*{gst[d]}" if gst[d] != 1 else f"(long long)({e})")
                if (c != "0" and tile[d] * _cdiv(g[d], tile[d]) != g[d]) or (c == "0" and v.shape[d] > g[d]):
                    conds.append(f"({e}) < {g[d]}")
            gi = " + ".join(terms) if terms else "0"
            stmt = f"{dst}[{self.gidx(gi, _prod(g))}] = ({self.T}){self.lr(v.addr(idx))};"
            self.emit(f"if ({' && '.join(conds)}) {stmt}" if conds else stmt)
        self.elem_loop(v.shape, body)
        self.sync()

    def _bcast_shape(self, views):
        rank = len(views[0].shape)
        if any(len(v.shape) != rank for v in views):
            raise UnsupportedProgram("elementwise operands of different rank")
        out = []
        for d in range(rank):
            ns = {v.shape[d] for v in views if v.shape[d] != 1}
            if len(ns) > 1:
                raise UnsupportedProgram(f"elementwise shape mismatch on dim {d}: {[v.shape for v in views]}")
            out.append(ns.pop() if ns else 1)
        return out

    def gen_compute(self, c: Compute):
        op = c.op
        if op in ELEMENTWISE_OPS:
            ins = [self.view(i) for i in c.inputs]
            out_shape = self._bcast_shape(ins)
            wide = max(ins, key=lambda v: (len(v.axes), _prod(v.shape)))
            axes = wide.axes
            base = self.alloc(out_shape)

            def body(idx):
                a = [self.lr(v.addr(idx)) for v in ins]
                if op == "causal":
                    p = axes.index(c.axis)
                    q = p - 1
                    if q < 0:
                        raise UnsupportedProgram("causal needs a query axis before the key axis")
                    expr = (f"((({wide.origin[p]}) + {idx[p]}) > (({wide.origin[q]}) + {idx[q]})) "
                            f"? -GR_INF : {a[0]}")
                else:
                    expr = _ew_expr(op, a, c.const)
                self.emit(f"{self.lw(f'{base} + e')} = {expr};")
            self.elem_loop(out_shape, body)
            self.sync()
            self.define(c, base, out_shape, axes, wide.origin)
        elif op in ROW_REDUCE_OPS:
            v = self.view(c.inputs[0])
            p = v.axes.index(c.axis)
            out_shape = list(v.shape)
            L = out_shape[p]
            out_shape[p] = 1
            base = self.alloc(out_shape)
            self.emit_rowreduce(v, p, L, out_shape, base, op, None)
            self.sync()
            org = list(v.origin)
            org[p] = "0"
            self.define(c, base, out_shape, v.axes, org)
        elif op in ("matmul", "softmax_matmul"):
            a, b = self.view(c.inputs[0]), self.view(c.inputs[1])
            out_shape = self._mm_shape(a, b)
            base = self.alloc(out_shape)
            if op == "matmul":
                self.emit_matmul(a, b, out_shape, base, accumulate=False)
            else:
                self.emit_softmax_matmul_full(a, b, out_shape, base)
            self.sync()
            self.define(c, base, out_shape, _value_axes(c), a.origin[:-1] + [b.origin[-1]])
        else:
            raise UnsupportedProgram(f"op {op!r}")

    def _mm_shape(self, a, b):
        if len(a.shape) != len(b.shape) or len(a.shape) < 2:
            raise UnsupportedProgram("matmul operand ranks")
        if a.shape[-1] != b.shape[-2]:
            raise UnsupportedProgram(f"matmul contraction mismatch {a.shape} x {b.shape}")
        batch = []
        for x, y in zip(a.shape[:-2], b.shape[:-2]):
            if x != y and 1 not in (x, y):
                raise UnsupportedProgram("matmul batch mismatch")
            batch.append(max(x, y))
        return batch + [a.shape[-2], b.shape[-1]]

    def emit_matmul(self, a, b, out_shape, base, accumulate):
        K = a.shape[-1]
        r = len(out_shape)
        self.emit(f"// {'mma: acc += A @ B' if accumulate else 'matmul: C = A @ B'} (K = {K})")

        def body(idx):
            ai = idx[:r - 2] + [idx[r - 2], "k"]
            bi = idx[:r - 2] + ["k", idx[r - 1]]
            self.emit("float s = 0.f;")
            self.emit(f"for (int k = 0; k < {K}; ++k) s = fmaf({self.lr(a.addr(ai))}, {self.lr(b.addr(bi))}, s);")
            self.emit(f"{self.lw(f'{base} + e')} {'+' if accumulate else ''}= s;")
        self.elem_loop(out_shape, body)

    def emit_rowreduce(self, v, p, L, out_shape, base, op, acc_mode):
        init = "-GR_INF" if op == "rowmax" else "0.f"
        comb = "fmaxf(r, x)" if op == "rowmax" else "r + x"

        def body(idx):
            ii = list(idx)
            ii[p] = "k"
            self.emit(f"float r = {init};")
            self.emit(f"for (int k = 0; k < {L}; ++k) {{ const float x = {self.lr(v.addr(ii))}; r = {comb}; }}")
            if acc_mode is None:
                self.emit(f"{self.lw(f'{base} + e')} = r;")
            elif op == "rowmax":
                self.emit(f"{self.lw(f'{base} + e')} = fmaxf({self.lr(f'{base} + e')}, r);")
            else:
                self.emit(f"{self.lw(f'{base} + e')} += r;")
        self.elem_loop(out_shape, body)

    def emit_softmax_matmul_full(self, a, b, out_shape, base):
        """softmax over the last axis of a, then @ b, in one pass per output."""
        K = a.shape[-1]
        r = len(out_shape)

        def body(idx):
            ai = idx[:r - 2] + [idx[r - 2], "k"]
            bi = idx[:r - 2] + ["k", idx[r - 1]]
            self.emit("float m = -GR_INF;")
            self.emit(f"for (int k = 0; k < {K}; ++k) m = fmaxf(m, {self.lr(a.addr(ai))});")
            self.emit("if (m == -GR_INF) m = 0.f;")
            self.emit("float l = 0.f, s = 0.f;")
            self.emit(f"for (int k = 0; k < {K}; ++k) {{ const float p = __expf({self.lr(a.addr(ai))} - m); "
                      f"l += p; s = fmaf(p, {self.lr(b.addr(bi))}, s); }}")
            self.emit(f"{self.lw(f'{base} + e')} = s / l;")
        self.elem_loop(out_shape, body)

    # -- reduction loops -----------------------------------------------------
    def gen_reduction(self, rl: ReductionLoop):
        ext = None
        for ld in list(_loads_feeding(rl)) + list(_iter_loads(rl.body)):
            if rl.axis in ld.index:
                ext = self.p.tensors[ld.source][ld.index.index(rl.axis)]
                break
        if ext is None:
            raise UnsupportedProgram(f"reduction axis {rl.axis!r} not found in any load")
        if ext % rl.tile:
            raise UnsupportedProgram(f"reduction tile {rl.tile} does not divide {ext}")
        accs = {}
        for p in rl.partials:
            if not isinstance(p, Compute) or p.op not in ("matmul", "rowmax", "rowsum", "softmax_matmul"):
                raise UnsupportedProgram("unsupported reduction partial")
            accs[id(p)] = {"op": p.op, "node": p, "base": None}
        lv = self.loopvar(rl)
        # accumulators are allocated lazily at the first partial update (their
        # shape is known then); allocation/initialisation is hoisted before the loop
        init_mark = len(self.lines)
        loop_start = self.pos
        self.emit(f"for (int {lv} = 0; {lv} < {ext // rl.tile}; ++{lv}) {{")
        self.ind += 1
        self.loops.append(rl)
        saved = self.scope.get(rl.axis)
        self.scope[rl.axis] = lv
        self.gen_body(rl.body, partial_acc=accs)
        self.loops.pop()
        if saved is None:
            self.scope.pop(rl.axis, None)
        else:
            self.scope[rl.axis] = saved
        self.ind -= 1
        self.emit("}")
        self.step()
        loop_end = self.pos
        # values read inside the loop but made before it stay live for the
        # whole loop (the next iteration reads them again); accumulators are
        # live from their initialisation before the loop
        for b in self.bufs.values():
            if b["def"] < loop_start <= b["last"]:
                b["last"] = max(b["last"], loop_end)
        for p in rl.partials:
            a = accs[id(p)]
            for key in ("base", "m", "l", "alpha"):
                if a.get(key) is not None:
                    bb = self.bufs[a[key]]
                    bb["def"] = min(bb["def"], loop_start)
                    bb["last"] = max(bb["last"], loop_end)
        # initialisation code, inserted before the loop
        init = []
        for p in rl.partials:
            a = accs[id(p)]
            if a["base"] is None:
                raise UnsupportedProgram("reduction partial never evaluated")
            E = _prod(a["shape"])
            pad = "  " * self.ind
            if a["op"] == "softmax_matmul":
                R = _prod(a["shape"][:-1])
                init.append(f"{pad}for (int e = threadIdx.x; e < {E}; e += {NT}) {self.lw(a['base'] + ' + e')} = 0.f;")
                init.append(f"{pad}for (int e = threadIdx.x; e < {R}; e += {NT}) {{ {self.lw(a['m'] + ' + e')} = -GR_INF; "
                            f"{self.lw(a['l'] + ' + e')} = 0.f; }}")
            else:
                v = "-GR_INF" if a["op"] == "rowmax" else "0.f"
                init.append(f"{pad}for (int e = threadIdx.x; e < {E}; e += {NT}) {self.lw(a['base'] + ' + e')} = {v};")
        init.append("  " * self.ind + self.sync_stmt())
        self.lines[init_mark:init_mark] = init
        # finalise (online softmax -> o / l) and publish the values
        for p in rl.partials:
            a = accs[id(p)]
            if a["op"] == "softmax_matmul":
                E = _prod(a["shape"])
                N = a["shape"][-1]
                self.emit(f"for (int e = threadIdx.x; e < {E}; e += {NT}) "
                          f"{self.lw(a['base'] + ' + e')} /= {self.lr(a['l'] + f' + e / {N}')};")
                self.sync()
            self.define(p, a["base"], a["shape"], a["axes"], a["origin"])
        self.vals[id(rl)] = self.vals[id(rl.partials[0])]

    def gen_partial(self, c: Compute, a: dict):
        op = c.op
        for key in ("base", "m", "l", "alpha"):
            if a.get(key) is not None:
                self.touch(a[key])
        if op == "matmul":
            x, y = self.view(c.inputs[0]), self.view(c.inputs[1])
            shape = self._mm_shape(x, y)
            self._acc_alloc(a, shape, _value_axes(c), x.origin[:-1] + [y.origin[-1]])
            self.emit_matmul(x, y, shape, a["base"], accumulate=True)
        elif op in ROW_REDUCE_OPS:
            v = self.view(c.inputs[0])
            p = v.axes.index(c.axis)
            shape = list(v.shape)
            L = shape[p]
            shape[p] = 1
            org = list(v.origin)
            org[p] = "0"
            self._acc_alloc(a, shape, v.axes, org)
            self.emit_rowreduce(v, p, L, shape, a["base"], op, acc_mode=True)
        elif op == "softmax_matmul":
            s, v = self.view(c.inputs[0]), self.view(c.inputs[1])
            shape = self._mm_shape(s, v)
            first = a["base"] is None
            self._acc_alloc(a, shape, _value_axes(c), s.origin[:-1] + [v.origin[-1]])
            if first:
                R = _prod(shape[:-1])
                a["m"] = self.alloc([R])
                a["l"] = self.alloc([R])
                a["alpha"] = self.alloc([R])
            self.emit_online_softmax(s, v, shape, a)
        else:
            raise UnsupportedProgram(f"partial op {op!r}")
        self.sync()
        self.vals[id(c)] = (a["base"], tuple(a["shape"]), a["axes"], len(self.loops), a["origin"])

    def _acc_alloc(self, a, shape, axes, origin):
        if a["base"] is None:
            a["base"] = self.alloc(shape)
            a["shape"] = tuple(shape)
            a["axes"] = list(axes)
            # an accumulator never spans its loop's axis: its origin is loop-invariant
            a["origin"] = list(origin)
        elif tuple(shape) != a["shape"]:
            raise UnsupportedProgram("partial shape changes between iterations")

    def emit_online_softmax(self, s, v, shape, a):
        K = s.shape[-1]
        N = shape[-1]
        rshape = list(shape[:-1]) + [1]
        r = len(shape)

        def rows(idx):
            si = idx[:r - 1] + ["k"]
            self.emit("float mt = -GR_INF;")
            self.emit(f"for (int k = 0; k < {K}; ++k) mt = fmaxf(mt, {self.lr(s.addr(si))});")
            self.emit(f"const float mo = {self.lr(a['m'] + ' + e')};")
            self.emit("const float mn = fmaxf(mo, mt);")
            self.emit("const float ms = (mn == -GR_INF) ? 0.f : mn;")
            self.emit("const float al = __expf(mo - ms);")
            self.emit("float ls = 0.f;")
            self.emit(f"for (int k = 0; k < {K}; ++k) ls += __expf({self.lr(s.addr(si))} - ms);")
            self.emit(f"{self.lw(a['m'] + ' + e')} = mn; {self.lw(a['alpha'] + ' + e')} = al;")
            self.emit(f"{self.lw(a['l'] + ' + e')} = {self.lr(a['l'] + ' + e')} * al + ls;")
        self.elem_loop(rshape, rows)
        self.sync()

        def outs(idx):
            si = idx[:r - 1] + ["k"]
            vi = idx[:r - 2] + ["k", idx[r - 1]]
            self.emit(f"const int row = e / {N};")
            self.emit(f"const float mn = {self.lr(a['m'] + ' + row')};")
            self.emit("const float ms = (mn == -GR_INF) ? 0.f : mn;")
            self.emit("float acc = 0.f;")
            self.emit(f"for (int k = 0; k < {K}; ++k) acc = fmaf(__expf({self.lr(s.addr(si))} - ms), "
                      f"{self.lr(v.addr(vi))}, acc);")
            self.emit(f"{self.lw(a['base'] + ' + e')} = {self.lr(a['base'] + ' + e')} * "
                      f"{self.lr(a['alpha'] + ' + row')} + acc;")
        self.elem_loop(shape, outs)

    # -- kernel ----------------------------------------------------------------
    def render(self) -> tuple:
        loop, p = self.loop, self.p
        g_out = p.tensors[loop.out]
        grid = [_cdiv(g, t) for g, t in zip(g_out, loop.tile_shape)]
        kname = f"{_cname(loop.out)}_kernel"
        args = _loop_tensors(loop)
        if args.count(loop.out) > 1:
            raise UnsupportedProgram(f"stage {loop.out} reads its own output")
        # grid decode (row-major, last output dim fastest)
        self.emit("int bid = blockIdx.x;")
        for d in range(len(grid) - 1, -1, -1):
            var = f"b_{_cname(loop.index_vars[d])}"
            if grid[d] == 1:
                self.emit(f"const int {var} = 0;")
            else:
                self.emit(f"const int {var} = bid % {grid[d]}; bid /= {grid[d]};")
            self.scope[loop.index_vars[d]] = var
        self.gen_body(loop.body)
        consts = self.assign_lds()
        if self.nfl * 4 > LDS_LIMIT:
            raise LdsOverflow(loop.out, self.nfl * 4 - LDS_LIMIT)
        # the checking build keeps two shadow words per LDS float behind the tiles
        lds = self.nfl * 4 * (3 if self.check else 1)
        if lds > LDS_LIMIT:
            raise UnsupportedProgram(f"stage {loop.out}: the checking build needs {lds} B of LDS "
                                     f"(three times the tiles' {self.nfl * 4} B); use smaller tiles")
        params = ", ".join(f"{'const ' if a != loop.out else ''}{self.T}* __restrict__ {_cname(a)}" for a in args)
        if self.check:
            params += ", unsigned int* __restrict__ gr_chk"
        code = [f"// stage {loop.out}: generic LDS-tile kernel, tile {tuple(loop.tile_shape)}, "
                f"{self.nfl * 4} B LDS{' (checking build)' if self.check else ''}",
                f'extern "C" __global__ __launch_bounds__({NT}) void {kname}({params}) {{',
                f"  extern __shared__ __attribute__((aligned(16))) float gr_lds[];"]
        code += consts
        if self.check:
            code += [f"  constexpr int gr_nfl = {self.nfl};",
                     "  unsigned int gr_epoch = 1u;",
                     "  unsigned int* const gr_sh = reinterpret_cast<unsigned int*>(gr_lds + gr_nfl);",
                     f"  for (int e = threadIdx.x; e < 2 * gr_nfl; e += {NT}) gr_sh[e] = 0u;",
                     "  __syncthreads();"]
        code += self.lines
        code.append("}")
        return "\n".join(code) + "\n", {"kernel": kname, "grid": [_prod(grid), 1, 1], "block": [NT, 1, 1],
                                          "lds": lds, "args": args + (["__check__"] if self.check else []),
                                          "lowering": "generic"}


def _ew_expr(op, a, const):
    if op == "add":
        return f"{a[0]} + {a[1]}"
    if op == "sub":
        return f"{a[0]} - {a[1]}"
    if op == "mul":
        return f"{a[0]} * {a[1]}"
    if op == "div":
        return f"{a[0]} / {a[1]}"
    if op == "relu":
        return f"fmaxf({a[0]}, 0.f)"
    if op == "exp":
        return f"__expf({a[0]})"
    if op == "sqrt":
        return f"sqrtf({a[0]})"
    if op == "mulc":
        return f"{a[0]} * {_flt(const)}"
    if op == "addc":
        return f"{a[0]} + {_flt(const)}"
    if op == "silu":
        return f"{a[0]} / (1.f + __expf(-{a[0]}))"
    raise UnsupportedProgram(f"op {op!r}")


# ---------------------------------------------------------------------------
# Module
# ---------------------------------------------------------------------------
PLAN_TAG = "GR_PLAN"


def render_module(program: Program, fn_name: str = "fn", check: bool = False) -> str:
    """HIP source of the whole program (one kernel per stage) with its launch
    plan in a trailing comment. check=True: the checking build, whose generic
    stages count out-of-range LDS and global indices and LDS races between
    barriers in a buffer bound as "__check__" (csrc/gr_check.h; the flash,
    GEMM and row lowerings are the same as in the product build)."""
    validate(program)
    shapes = _infer_program(program)
    meta = kernel_meta(program, shapes)
    inputs, inter, outputs = _program_io(program)
    parts = ['#include "gr_gemm_f32.h"'] + (['#include "gr_check.h"'] if check else []) + [
        "", f"// generated from a grammar program: {len(program.body)} stage(s), storage {program.dtype}"
        + (" (checking build)" if check else "")]
    # The fp16 flash kernel pre-scales Q by scale * log2(e) once and rounds it
    # to fp16; with a factor above 1 a finite |q| could overflow, so such a
    # module takes the kernel's per-score scaling instead (any scale is exact).
    flash = [f for f in (_match_flash(l, program) for l in program.body
                         if (getattr(l, "knobs", None) or {}).get("lowering") != "generic") if f is not None]
    if program.dtype == "fp16" and any(f["scale"] * LOG2E > 1.0 for f in flash):
        parts.insert(0, "#define GR_FLASH_OPT 0  // a flash stage's scale * log2(e) exceeds 1: no fp16 Q pre-scale")
    if any(f.get("f32") for f in flash):
        parts.insert(parts.index('#include "gr_gemm_f32.h"') + 1, '#include "gr_flash_f32.h"')
    if any(f.get("W2") and f["D"] == 64 for f in flash):
        parts.insert(parts.index('#include "gr_gemm_f32.h"') + 1, '#include "gr_flash_w2.h"')
    if any(f.get("W2") and f["D"] == 128 for f in flash):
        parts.insert(parts.index('#include "gr_gemm_f32.h"') + 1, '#include "gr_flash_w2h.h"')
    steps = []
    over, excess = [], 0
    matched = []
    for loop in program.body:
        # knobs {"lowering": "generic"} pins a stage to the generic LDS-tile
        # lowering (diagnostics and tests of that lowering)
        generic = (getattr(loop, "knobs", None) or {}).get("lowering") == "generic"
        f = None if generic else _match_flash(loop, program)
        gm = _match_gemm(loop, program) if f is None and not generic else None
        rw = _match_rows(loop, program) if f is None and gm is None and not generic else None
        matched.append((f, gm, rw))
    fused = _split_sums_in_consumers(program, matched, outputs)
    for loop, (f, gm, rw) in zip(program.body, matched):
        try:
            if f is not None:
                code, step = _render_flash(loop, program, f)
            elif gm is not None:
                code, step = _render_gemm(loop, program, gm)
            elif rw is not None:
                code, step = _RowGen(loop, program, rw, fused).render()
            else:
                code, step = _StageGen(loop, program, shapes, check=check).render()
        except LdsOverflow as e:
            over.append(loop.out)
            excess += e.need
            continue
        parts.append(code)
        steps.extend(step if isinstance(step, list) else [step])
    if over:
        raise LdsOverflow(",".join(over), excess)
    plan = {"fn": fn_name, "dtype": program.dtype, "inputs": inputs, "intermediates": inter, "outputs": outputs,
            "tensors": {k: list(v) for k, v in program.tensors.items()}, "steps": steps, "meta": meta}
    if check:
        plan["check"] = True
    parts.append(f"/*{PLAN_TAG} {json.dumps(plan, sort_keys=True)} {PLAN_TAG}*/")
    return "\n".join(parts) + "\n"


def _split_sums_in_consumers(program: Program, matched: list, outputs) -> dict:
    """Split-K fp32 GEMM stages whose second launch can go: the stage has no
    activation (a residual is added by its first K part, alpha by every
    part), its output is an intermediate of the program, and every stage
    that reads it is row-lowered with rows of the same shape, so those
    stages sum the partial products as they load them. Marks the GEMM
    parameters and returns tensor -> (workspace, parts, part stride)."""
    out = {}
    for loop, (_, gm, _) in zip(program.body, matched):
        if not gm or not gm.get("f32") or gm.get("ksplit", 1) <= 1 or (gm["act"] & 3) or loop.out in outputs:
            continue
        readers = [(l, rw) for l, (_, _, rw) in zip(program.body, matched)
                   if l is not loop and any(ld.source == loop.out for ld in _iter_loads(l.body))]
        if not readers or any(rw is None or tuple(rw["out"]) != tuple(program.tensors[loop.out])
                              for _, rw in readers):
            continue
        gm["fuse_reduce"] = True
        out[loop.out] = (f"gr_ws_{_cname(loop.out)}", gm["ksplit"], gm["batch"] * gm["M"] * gm["N"])
    return out


def flash_stage_indices(program: Program) -> set:
    """Indices of the stages whose lowering does not stage per-value tiles in
    LDS: the flash and GEMM kernels (registers and a fixed LDS ring) and the
    row lowering (streams rows through registers)."""
    out = set()
    for i, loop in enumerate(program.body):
        if _match_flash(loop, program) is not None or _match_gemm(loop, program) is not None:
            out.add(i)
        elif _match_rows(loop, program) is not None:
            out.add(i)
    return out


def parse_plan(src: str) -> dict:
    m = re.search(r"/\*" + PLAN_TAG + r" (.*) " + PLAN_TAG + r"\*/", src, re.S)
    if not m:
        raise ValueError("source carries no launch plan")
    return json.loads(m.group(1))
