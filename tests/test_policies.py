"""Draft-shape policies against closed forms (tests/test_policies.py:11-43 of the
reference: Leviathan's Thm. 3.8, monotonicity, the acceptance estimate and the
verify-size limit) plus the static shapes' budgets and node selection."""
from dataclasses import dataclass

import pytest

from woodcock_amd.policies import CostAwareChain, Plan, StaticPolicy, top_by_phat


def leviathan_factor(alpha, gamma, c):
    """arXiv:2211.17192 Thm. 3.8: expected walltime improvement factor."""
    return (1 - alpha ** (gamma + 1)) / ((1 - alpha) * (gamma * c + 1))


@pytest.mark.parametrize("alpha", [0.3, 0.6, 0.8, 0.9])
@pytest.mark.parametrize("c", [0.02, 0.1, 0.3])
def test_reduces_to_leviathan_with_constant_verify_and_no_update(alpha, c):
    pol = CostAwareChain(step_ms=c, head_ms=c, verify_ms={n: 1.0 for n in range(1, 10)}, k_max=8)
    best = max(range(1, 9), key=lambda g: (leviathan_factor(alpha, g, c), -g))
    assert pol.best_depth(alpha) == best


def test_longer_chains_for_higher_acceptance_and_cheaper_steps():
    v = {n: 10.0 + 0.2 * n for n in range(1, 10)}
    pol = CostAwareChain(step_ms=1.5, head_ms=1.1, verify_ms=v)
    cheap = CostAwareChain(step_ms=0.5, head_ms=0.1, verify_ms=v)
    assert pol.best_depth(0.4) < pol.best_depth(0.8)
    assert pol.best_depth(0.7) < cheap.best_depth(0.7)


def test_alpha_estimate_counts_successes_and_failures():
    pol = CostAwareChain(1.0, 0.5, {n: 10.0 for n in range(1, 10)}, alpha0=0.5, prior=2.0, window=3)
    assert pol.alpha() == pytest.approx(0.5)
    pol.observe(4, 4, 4, 0, 0)
    pol.observe(1, 4, 4, 0, 0)
    assert pol.alpha() == pytest.approx((5 + 1) / (5 + 1 + 2))
    for _ in range(3):
        pol.observe(0, 2, 2, 0, 0)
    assert pol.alpha() == pytest.approx(1 / (3 + 2))
    pol.reset()
    assert pol.alpha() == pytest.approx(0.5)


def test_alpha_is_clipped():
    pol = CostAwareChain(1.0, 0.5, {n: 10.0 for n in range(1, 10)}, alpha0=1.0, prior=100.0)
    assert pol.alpha() == 0.99
    pol = CostAwareChain(1.0, 0.5, {n: 10.0 for n in range(1, 10)}, alpha0=0.0, prior=100.0)
    assert pol.alpha() == 0.01


def test_k_max_limited_by_measured_verify_sizes():
    pol = CostAwareChain(0.1, 0.05, {n: 1.0 for n in range(1, 5)}, k_max=8)
    assert pol.k_max == 3 and pol.best_depth(0.99) == 3


def test_cost_model_by_brute_force():
    """cost[k] = t_v(k+1) + k t_s + (t_s - t_h), and the chosen length maximises
    E(k)/cost[k] over every k (checked by enumeration)."""
    v = {1: 3.0, 2: 3.1, 3: 3.3, 4: 3.6, 5: 4.0, 6: 4.5}
    pol = CostAwareChain(step_ms=0.4, head_ms=0.15, verify_ms=v, k_max=8)
    assert pol.k_max == 5
    for k in range(1, 6):
        assert pol.cost[k] == pytest.approx(v[k + 1] + 0.4 * k + 0.25)
    for a in (0.2, 0.5, 0.75, 0.95):
        rates = {k: (1 - a ** (k + 1)) / (1 - a) / pol.cost[k] for k in range(1, 6)}
        assert rates[pol.best_depth(a)] == max(rates.values())


def test_plan_and_from_costs():
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
