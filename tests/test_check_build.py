"""CPU checks of the checking build of the generic lowering (csrc/gr_check.h):
every LDS access of a generic stage goes through the checked accessors, every
barrier advances the race detector's interval, the product build's text is
unchanged by the option, and the instrumented modules compile for gfx950."""
import re

import pytest

import grammar_cases as C
from grammar.hip_backend import parse_plan, render_module


def _generic(p):
    for l in p.body:
        l.knobs["lowering"] = "generic"
    return p


def fit_for_check(p, limit=160 * 1024):
    """Halve the output tiles of the stages whose checking build (three times
    the tiles' LDS) does not fit, largest dimension first -- a retiling, as
    the descent's tile sweeps make."""
    from grammar.hip_backend import UnsupportedProgram
    for _ in range(16):
        try:
            return render_module(p, check=True)
        except UnsupportedProgram as e:
            m = re.match(r"stage (\S+): the checking build needs", str(e))
            if not m:
                raise
            loop = next(l for l in p.body if l.out == m.group(1))
            old = tuple(loop.tile_shape)
            for d in sorted((i for i, t in enumerate(old) if t > 1 and t % 2 == 0), key=lambda i: -old[i]):
                loop.tile_shape = old[:d] + (old[d] // 2,) + old[d + 1:]
                try:
                    render_module(p)            # a legal tiling (a row softmax keeps its whole row)
                    break
                except (AssertionError, UnsupportedProgram):
                    loop.tile_shape = old
            else:
                raise AssertionError(f"stage {loop.out}: no smaller tiling renders")
    raise AssertionError("no tile fits the checking build")


def _generic_stage_bodies(src):
    """The text of each generic stage kernel in a rendered module."""
    return re.findall(r"// stage \S+: generic LDS-tile kernel.*?\n}\n", src, re.S)


@pytest.mark.parametrize("name", list(C.REFS))
def test_every_lds_access_is_checked(name):
    p = _generic(C.REFS[name][0]())
    checked = fit_for_check(p)
    plain = render_module(p)
    assert "GR_LR" not in plain and "GR_SYNC" not in plain and "__check__" not in plain
    plan = parse_plan(checked)
    assert plan["check"] is True
    bodies = _generic_stage_bodies(checked)
    assert len(bodies) == len(plan["steps"])
    for body, step in zip(bodies, plan["steps"]):
        assert step["args"][-1] == "__check__"
        # the only raw uses of the LDS array: its declaration and the shadow base
        raw = [l for l in body.splitlines() if "gr_lds[" in l]
        assert raw == ["  extern __shared__ __attribute__((aligned(16))) float gr_lds[];"], raw
        # past the shadow's initialisation every barrier is GR_SYNC
        assert "__syncthreads();" not in body.split("gr_sh[e] = 0u;\n  __syncthreads();", 1)[1]
        assert body.count("GR_SYNC();") == body.count("GR_SYNC") >= 1
        # every global tensor index is range-checked
        loads = re.findall(r"\(float\)\w+\[(.*?)\];", body)
        assert all(x.startswith("GR_GI(") for x in loads), loads
    # the plain build's LDS need tripled (two shadow words per float)
    for s_plain, s_chk in zip(parse_plan(plain)["steps"], plan["steps"]):
        assert s_chk["lds"] == 3 * s_plain["lds"]


@pytest.mark.parametrize("name", ["attention_atomic", "layernorm", "matmul_reduction", "softmax"])
def test_checked_modules_compile(name):
    from grammar import runtime as rt
    key = next(k for k in C.REFS if k == name or k.endswith(name))
    src = fit_for_check(_generic(C.REFS[key][0]()))
    assert rt.compile_source(src, name + "_check.hip")[:4] == b"\x7fELF"


def test_checking_build_refuses_tiles_whose_shadow_does_not_fit():
    from grammar.hip_backend import UnsupportedProgram
    p = _generic(C.p_matmul_full_k())
    # a tile whose plain build fits 160 KiB but not three times over
    for l in p.body:
        l.tile_shape = tuple(min(e, 128) for e in l.tile_shape)
    plain = parse_plan(render_module(p))
    if max(s["lds"] for s in plain["steps"]) * 3 <= 160 * 1024:
        pytest.skip("tile fits three times over")
    with pytest.raises(UnsupportedProgram, match="checking build"):
        render_module(p, check=True)
