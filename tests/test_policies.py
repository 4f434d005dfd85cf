"""Draft-shape policies (woodcock_amd.policies; python/woodcock/policies.py).

The cost-aware chain is checked against what the mathematics fixes: with a
constant verify cost and no update overhead, its objective E(k) / T(k) is
Leviathan et al.'s walltime-improvement factor (arXiv:2211.17192, Thm. 3.8),
so its choice must be that factor's maximiser; the expected tokens per round
E(k) is the truncated geometric series of the acceptance rate.  The cases
(grids, costs, observation sequences, expected estimates) are the reference
tests' own data, read from tests/golden/reference_cases.json; the checks are
written here.  The static shapes' budgets, frontier and verify-set selection
are checked on hand-made node lists.
"""
import json
from dataclasses import dataclass
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

from woodcock_amd.policies import CostAwareChain, Plan, StaticPolicy, top_by_phat

CASES = json.loads((Path(__file__).parent / "golden" / "reference_cases.json").read_text())["policies"]


def expected_tokens(alpha: float, k: int) -> float:
    """1 + alpha + ... + alpha^k: tokens a chain of k drafts yields per round."""
    return float(sum(alpha ** i for i in range(k + 1)))


def argmax_shortest(scores: dict[int, float]) -> int:
    """Key of the largest score; among (exact) ties, the smallest key."""
    top = max(scores.values())
    return min(k for k, s in scores.items() if s == top)


def flat_verify(ms: float, sizes: int) -> dict[int, float]:
    return {n: ms for n in range(1, sizes + 1)}


LEV = CASES["leviathan"]


@pytest.mark.parametrize("alpha", LEV["alphas"])
@pytest.mark.parametrize("c", LEV["step_costs"])
def test_choice_maximises_leviathan_improvement(alpha, c):
    """t_v constant, t_s = t_h = c (no update overhead): cost(k) = t_v + k c, so
    E(k) / cost(k) is the improvement factor of Thm. 3.8 up to the constant t_v."""
    pol = CostAwareChain(step_ms=c, head_ms=c, verify_ms=flat_verify(LEV["verify_ms"], LEV["verify_sizes"]),
                         k_max=LEV["k_max"])
    factor = {k: expected_tokens(alpha, k) / (1.0 + k * c / LEV["verify_ms"]) for k in range(1, LEV["k_max"] + 1)}
    want = argmax_shortest({k: round(v, 12) for k, v in factor.items()})
    assert pol.best_depth(alpha) == want


def test_geometric_form_of_the_objective():
    """The policy's rate uses the closed form (1 - a^(k+1)) / (1 - a); both agree
    with the series for every length and acceptance on a grid."""
    v = {n: 3.0 + 0.1 * n for n in range(1, 10)}
    pol = CostAwareChain(step_ms=0.3, head_ms=0.1, verify_ms=v)
    for a in np.linspace(0.05, 0.95, 19):
        for k in range(1, pol.k_max + 1):
            closed = (1 - a ** (k + 1)) / (1 - a)
            assert closed == pytest.approx(expected_tokens(a, k), rel=1e-12)
        scores = {k: expected_tokens(a, k) / pol.cost[k] for k in range(1, pol.k_max + 1)}
        assert pol.best_depth(a) == argmax_shortest({k: round(s, 12) for k, s in scores.items()})


MONO = CASES["monotone"]


def test_longer_chains_when_acceptance_rises_or_steps_get_cheaper():
    v = {n: MONO["verify_ms"]["base"] + MONO["verify_ms"]["per_row"] * n for n in range(1, MONO["sizes"] + 1)}
    slow = CostAwareChain(verify_ms=v, **MONO["slow"])
    cheap = CostAwareChain(verify_ms=v, **MONO["cheap"])
    assert slow.best_depth(MONO["alpha_low"]) < slow.best_depth(MONO["alpha_high"])
    assert slow.best_depth(MONO["alpha_mid"]) < cheap.best_depth(MONO["alpha_mid"])
    # and everywhere on a grid: non-decreasing in the acceptance rate
    for pol in (slow, cheap):
        depths = [pol.best_depth(a) for a in np.linspace(0.01, 0.99, 50)]
        assert depths == sorted(depths)


EST = CASES["alpha_estimate"]


def test_acceptance_estimate_over_a_sliding_window():
    """alpha = (successes + prior * alpha0) / (successes + failures + prior) over
    the last `window` rounds, a round of a accepted out of k adding a successes
    and one failure when a < k."""
    pol = CostAwareChain(EST["step_ms"], EST["head_ms"], flat_verify(EST["verify_ms"], EST["sizes"]),
                         alpha0=EST["alpha0"], prior=EST["prior"], window=EST["window"])
    kept: list[tuple[int, int]] = []
    for step in EST["steps"]:
        if step.get("reset"):
            pol.reset()
            kept.clear()
        for a, k in step.get("observe", []):
            pol.observe(a, k, k, 0.0, 0.0)
            kept = (kept + [(a, k)])[-EST["window"]:]
        succ = sum(a for a, _ in kept)
        fail = sum(a < k for a, k in kept)
        exact = (Fraction(succ) + Fraction(EST["prior"]) * Fraction(EST["alpha0"])) / (succ + fail + Fraction(EST["prior"]))
        assert float(exact) == pytest.approx(step["alpha"])
        assert pol.alpha() == pytest.approx(step["alpha"])


@pytest.mark.parametrize("alpha0,want", [(1.0, 0.99), (0.0, 0.01)])
def test_acceptance_estimate_is_clipped(alpha0, want):
    pol = CostAwareChain(1.0, 0.5, flat_verify(10.0, 9), alpha0=alpha0, prior=100.0)
    assert pol.alpha() == want


KM = CASES["k_max"]


def test_lengths_limited_by_the_measured_verify_sizes():
    """A chain of k needs a verify of k + 1 rows: with sizes 1..n measured, k <= n - 1."""
    pol = CostAwareChain(KM["step_ms"], KM["head_ms"], flat_verify(KM["verify_ms"], KM["sizes"]), k_max=KM["k_max"])
    assert pol.k_max == KM["want_k_max"]
    assert set(pol.cost) == set(range(1, KM["want_k_max"] + 1))
    assert pol.best_depth(KM["alpha"]) == KM["want_depth"]


def test_cost_table_and_choice_by_enumeration():
    """cost[k] = t_v(k+1) + k t_s + (t_s - t_h); the choice beats every other length."""
    v = {1: 3.0, 2: 3.1, 3: 3.3, 4: 3.6, 5: 4.0, 6: 4.5}
    pol = CostAwareChain(step_ms=0.4, head_ms=0.15, verify_ms=v, k_max=8)
    assert pol.k_max == 5
    for k in range(1, 6):
        assert pol.cost[k] == pytest.approx(v[k + 1] + 0.4 * k + 0.25)
    for a in (0.2, 0.5, 0.75, 0.95):
        best = pol.best_depth(a)
        for k in range(1, 6):
            assert expected_tokens(a, best) / pol.cost[best] >= expected_tokens(a, k) / pol.cost[k] - 1e-12


def test_plan_records_the_choice_and_reads_a_costs_table():
    costs = {"drafter": {"16384": {"step_ms": 0.05, "head_ms": 0.015}},
             "verify_ms": {str(n): 9.0 + 0.1 * n for n in range(1, 10)}}
    pol = CostAwareChain.from_costs(costs, "16384")
    p = pol.plan(100, stochastic=False)
    assert p.width == 1 and p.max_depth == p.budget == pol.chosen[-1] == pol.best_depth(pol.alpha())


def test_static_defaults_and_children_budget():
    assert StaticPolicy(5).budget == 5
    assert StaticPolicy(6, width=4).budget == 24
    plan = Plan(max_depth=6, width=4, budget=10)
    assert [plan.children_for(1.0, 1) for _ in range(4)] == [4, 4, 2, 0]


@dataclass
class N:
    phat: float
    depth: int


def test_select_verify_keeps_root_and_most_probable_nodes():
    nodes = [N(1.0, 0), N(0.5, 1), N(0.3, 1), N(0.3, 2), N(0.05, 2), N(0.4, 2)]
    assert top_by_phat(nodes, 3) == [0, 1, 2, 5]
    pol = StaticPolicy(2, width=2, budget=3)
    assert pol.select_verify(nodes, 10, stochastic=False) == [0, 1, 2, 5]
    assert pol.select_verify(nodes, 10, stochastic=True) == list(range(6))  # never prune drawn nodes
    # tie on phat: the shallower node first, then the earlier one
    assert top_by_phat([N(1, 0), N(0.3, 2), N(0.3, 1), N(0.3, 1)], 2) == [0, 2, 3]
    assert pol.select_frontier([1, 2, 3, 4, 5], nodes, 2) == [1, 5]
