"""CPU tests of the ablation tooling: plot_ablation.py summarises RunLogger
logs (best feasible curve as the reference's plot_ablation.py:55-68 reads
it) and draws the figures; run_ablations.py covers every principle that
run_attention_search.principle_config knows (run_attention_search.py:147-166)."""
import json
import math
import os

import grammar_cases as C
from grammar import optimization as O


def _proxy_run(run_dir, principle_rules=O.DEFAULT_RULES, seed=0):
    ev = O.Evaluator(O.EvalConfig(proxy=True, mem_budget=64 * 1024))
    O.autotune(C.p_attention_atomic(), ev, O.SearchConfig(iters=8, N=2, K=3, seed=seed, verbose=False,
                                                          run_dir=run_dir, rules=principle_rules))


def test_summary_and_figures_from_run_logs(tmp_path):
    import plot_ablation as P
    a, b = str(tmp_path / "full"), str(tmp_path / "norev")
    _proxy_run(a)
    _proxy_run(b, seed=1)
    curve = P.feasible_best(P.read_log(a))
    assert [it for it, _ in curve] == list(range(9))
    vals = [v for _, v in curve if v is not None]
    assert vals == sorted(vals, reverse=True)          # the best never gets worse
    md = P.summary_markdown({"full": a, "no_reversibility": b})
    assert "| full |" in md and "| no_reversibility |" in md and "Best feasible ms" in md
    written = P.plot({"full": a, "no_reversibility": b}, a, str(tmp_path))
    assert all(os.path.getsize(p) > 1000 for p in written) and len(written) == 2


def test_never_feasible_run_is_reported(tmp_path):
    import plot_ablation as P
    d = tmp_path / "r"
    d.mkdir()
    with open(d / "log.jsonl", "w") as f:
        for it in range(3):
            f.write(json.dumps({"iter": it, "loss": 1e9 + 5, "best_loss": 1e9 + 5, "n_stages": 8, "flops": 1}) + "\n")
    assert all(v is None for _, v in P.feasible_best(P.read_log(str(d))))
    assert "| r | never |" in P.summary_markdown({"r": str(d)})


def test_run_ablations_covers_every_principle():
    import run_ablations as A
    import run_attention_search as RS
    for p in A.PRINCIPLES:
        cfg = RS.principle_config(p)
        assert set(cfg) >= {"rules", "repairable", "couple_tiles", "reduction_tile"}


def test_reference_rule_set_ablations():
    """--rules reference: the reference's seven rules, and without the inverse
    rules for no_reversibility (reference run_attention_search.py:140-166)."""
    import run_attention_search as RS
    from grammar.optimization import REFERENCE_RULES
    assert RS.principle_config("full", "reference")["rules"] == REFERENCE_RULES
    norev = RS.principle_config("no_reversibility", "reference")["rules"]
    assert "hoist" not in norev and "unwrap_reduction" not in norev and set(norev) < set(REFERENCE_RULES)
    assert RS.principle_config("no_repairability", "reference")["repairable"] is False
    assert "fuse_softmax_chain" in RS.principle_config("full")["rules"]
