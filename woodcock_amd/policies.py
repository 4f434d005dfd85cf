"""Draft-shape policies consulted once per round (python/woodcock/policies.py).

``StaticPolicy`` drafts a fixed shape: a chain of ``depth`` tokens (width 1) or
a width-w tree of which the ``budget`` nodes with the largest path probability
are verified (EAGLE-2, arXiv:2406.16858 §4; policies.py:49-75).
``CostAwareChain`` picks the chain length before each round from measured
costs: gamma* = argmax_k E(k) / T(k) with E(k) = (1 - a^(k+1)) / (1 - a)
(Leviathan et al., arXiv:2211.17192 Eq. 1) and
T(k) = t_v(k+1) + k t_s + (t_s - t_h) (policies.py:78-123); the acceptance a
is a smoothed ratio over the last ``window`` rounds, clipped to [0.01, 0.99],
and ties go to the shorter chain.

Distribution preservation at T > 0: the number of children drawn for a node is
fixed before drawing (``Plan.children_for``) and drawn nodes are never pruned by
their own probability (policies.py:10-15).
"""
from __future__ import annotations

from collections import deque
from dataclasses import dataclass, field


@dataclass
class Plan:
    """Shape of one round's draft (policies.py:24-39)."""

    max_depth: int
    width: int
    budget: int  # draft tokens verified this round at most
    remaining: int = field(init=False)

    def __post_init__(self):
        self.remaining = self.budget

    def children_for(self, phat: float, depth: int) -> int:
        """Children to draw for one node, decided before drawing (stochastic mode)."""
        take = max(0, min(self.width, self.remaining))
        self.remaining -= take
        return take


class Policy:
    """Interface the round loop consults (policies.py:42-55)."""

    def reset(self) -> None:
        pass

    def plan(self, context_len: int, stochastic: bool) -> Plan:
        raise NotImplementedError

    def continue_drafting(self, depth: int, gain: float, context_len: int, num_nodes: int) -> bool:
        return True

    def select_frontier(self, level_nodes, nodes, width):
        """The ``width`` most probable nodes of a level (path probability, then depth)."""
        return sorted(level_nodes, key=lambda v: (-nodes[v].phat, nodes[v].depth))[:width]

    def select_verify(self, nodes, context_len: int, stochastic: bool) -> list[int]:
        raise NotImplementedError

    def observe(self, accepted: int, verified: int, depth: int, t_draft: float, t_verify: float) -> None:
        pass


def top_by_phat(nodes, k: int) -> list[int]:
    """Root plus the k non-root nodes of largest path probability (ties: shallower,
    then earlier), returned in node order (policies.py:73-75)."""
    ranked = sorted(range(1, len(nodes)), key=lambda v: (-nodes[v].phat, nodes[v].depth, v))
    return [0] + sorted(ranked[:k])


class StaticPolicy(Policy):
    """Fixed depth / width / budget; width 1 is a chain of ``depth`` drafts.
    The default budget is depth for a chain, 4 * depth for a tree (policies.py:58-66)."""

    def __init__(self, depth: int, width: int = 1, budget: int | None = None):
        self.depth, self.width = depth, width
        self.budget = budget if budget is not None else (depth if width == 1 else 4 * depth)

    def plan(self, context_len: int, stochastic: bool) -> Plan:
        return Plan(self.depth, self.width, self.budget)

    def select_verify(self, nodes, context_len: int, stochastic: bool) -> list[int]:
        # stochastic rounds verify every drawn node (pruning by drawn probability biases the law)
        if stochastic or len(nodes) - 1 <= self.budget:
            return list(range(len(nodes)))
        return top_by_phat(nodes, self.budget)


class CostAwareChain(StaticPolicy):
    """Chain whose length is re-chosen every round from measured latencies.

    step_ms: one draft step (head + layer); head_ms: the head alone;
    verify_ms[n]: the target forward over n rows.  The lengths considered are
    1..min(k_max, max(verify_ms) - 1), since a chain of k needs verify_ms[k+1]."""

    def __init__(self, step_ms: float, head_ms: float, verify_ms: dict[int, float], k_max: int = 8,
                 alpha0: float = 0.6, prior: float = 4.0, window: int = 16):
        super().__init__(depth=1)
        self.k_max = min(k_max, max(verify_ms) - 1)
        self.alpha0, self.prior = alpha0, prior
        # cost[k] = t_v(k+1) + k t_s + (t_s - t_h): k drafts, the verify of k+1 rows and the update
        self.cost = {k: verify_ms[k + 1] + k * step_ms + (step_ms - head_ms) for k in range(1, self.k_max + 1)}
        self.hist: deque[tuple[int, int]] = deque(maxlen=window)
        self.chosen: list[int] = []

    @classmethod
    def from_costs(cls, costs: dict, head: str, **kw) -> "CostAwareChain":
        """``costs``: {"drafter": {head: {"step_ms", "head_ms"}}, "verify_ms": {n: ms}}
        (the costs.json of scripts/time_draft_step.py)."""
        d = costs["drafter"][head]
        return cls(d["step_ms"], d["head_ms"], {int(n): float(v) for n, v in costs["verify_ms"].items()}, **kw)

    def reset(self) -> None:
        self.hist.clear()

    def alpha(self) -> float:
        """(successes + prior * alpha0) / (successes + failures + prior), clipped."""
        succ = sum(a for a, _ in self.hist)
        fail = sum(1 for a, k in self.hist if a < k)
        return min(0.99, max(0.01, (succ + self.prior * self.alpha0) / (succ + fail + self.prior)))

    def best_depth(self, alpha: float) -> int:
        def rate(k: int) -> float:
            return (1.0 - alpha ** (k + 1)) / (1.0 - alpha) / self.cost[k]

        best = 1
        for k in range(2, self.k_max + 1):
            if rate(k) > rate(best):  # strict: ties keep the shorter chain
                best = k
        return best

    def plan(self, context_len: int, stochastic: bool) -> Plan:
        self.depth = self.budget = self.best_depth(self.alpha())
        self.chosen.append(self.depth)
        return Plan(self.depth, 1, self.depth)

    def observe(self, accepted: int, verified: int, depth: int, t_draft: float, t_verify: float) -> None:
        self.hist.append((accepted, depth))
