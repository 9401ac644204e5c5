"""The descent's checker (grammar/torch_eval.py, whole-tensor semantics) agrees
with each case's closed form and with the tile interpreter (CPU torch)."""
import numpy as np
import pytest

import grammar_cases as C
from grammar.kernel_ast import kernel_meta

torch = pytest.importorskip("torch")


@pytest.mark.parametrize("name", list(C.REFS))
def test_torch_eval_matches_closed_form(name):
    from grammar.torch_eval import evaluate
    build, ref = C.REFS[name]
    p = build()
    ins = C.inputs_for(p, 0)
    out = evaluate(p, {k: torch.from_numpy(v) for k, v in ins.items()})[kernel_meta(p)["output"][0]]
    assert np.allclose(out.numpy(), ref(ins), rtol=1e-3, atol=1e-3)
