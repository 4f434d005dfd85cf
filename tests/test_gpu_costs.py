"""costs.json on the HIP backend (the reference's scripts/time_draft_step.py
layout) feeding CostAwareChain.from_costs (python/woodcock/policies.py:97-101)."""
import json

import pytest

from woodcock_amd.costs import measure
from woodcock_amd.config import tiny_drafter
from woodcock_amd.policies import CostAwareChain
from woodcock_amd.target import TargetConfig

pytestmark = pytest.mark.gpu


def test_costs_layout_and_policy(cuda):
    tcfg = TargetConfig(hidden_size=512, num_heads=4, num_kv_heads=2, head_dim=128, intermediate_size=1024,
                        num_layers=2, vocab_size=1000)
    res = measure(drafter_cfg=tiny_drafter(), target_cfg=tcfg, ctx=64, sizes=(16,), max_n=5, iters=5)
    res = json.loads(json.dumps(res))  # what a costs.json round trip gives
    assert set(res) == {"ctx", "drafter", "verify_ms"} and res["ctx"] == 64
    assert set(res["drafter"]) == {"full", "16"}
    for d in res["drafter"].values():
        assert 0 < d["head_ms"] < d["step_ms"] < 100
    assert sorted(int(n) for n in res["verify_ms"]) == [1, 2, 3, 4, 5]
    assert all(0 < v < 100 for v in res["verify_ms"].values())
    pol = CostAwareChain.from_costs(res, "16")
    assert pol.k_max == 4
    assert 1 <= pol.best_depth(0.8) <= 4
    assert pol.plan(100, stochastic=False).width == 1
