"""Pins the tree-drafting restatement (oracle/tree_draft.py) on the CPU.

- the selection rules against hand-worked answers, ties included
  (policies.py:52-53,66-75; spec.py:226-237);
- the drafter tree mask against a hand-drawn matrix, with and without a
  sliding window (spec.py:280-294);
- width 1 reduces tree drafting to the greedy chain: the drafted tokens equal
  argmax drafting with the drafter's own causal forward (spec.py:331-350), on
  the reference-pinned tiny drafter fixture;
- structural invariants of a wider tree (parent closure of the verified set,
  sibling order, phat products);
- sampled drafting (T > 0): one node's draws follow the law of sequential
  draws without replacement (ordered pairs, chi-square), the Plan.children_for
  budget split on a hand-worked case, and the whole sampled-tree round --
  drafting, then recursive rejection -- emits the target's law in the Markov
  world of test_oracle_sampling, while planted slips (one uniform vector shared
  by every node, a draw pruned by its own probability, the Gumbel noise with
  the wrong sign) are caught by the same tests.
"""
import numpy as np
import pytest
from scipy.stats import chisquare

from conftest import load_golden
from oracle import sampling as S
from test_oracle_sampling import BAD_P, OK_P, WORLD
from drafter_replay import fixture_config, fixture_weights
from oracle import core
from oracle import tree_draft as td


def test_top_children_descending_lower_row_on_tie():
    q = np.array([0.1, 0.3, 0.05, 0.3, 0.25], np.float32)
    assert td.top_children(q, 3).tolist() == [1, 3, 4]
    assert td.top_children(q, 1).tolist() == [1]


def test_select_frontier_known_answer():
    phat = {4: 0.2, 5: 0.5, 6: 0.2, 7: 0.1}
    depth = {v: 2 for v in phat}
    # ties keep level order: 4 before 6
    assert td.select_frontier([4, 5, 6, 7], phat, depth, 3) == [5, 4, 6]
    assert td.select_frontier([4, 5, 6, 7], phat, depth, 8) == [5, 4, 6, 7]


def test_top_by_phat_known_answer():
    phat = [1.0, 0.5, 0.3, 0.3, 0.3, 0.05]
    depth = [0, 1, 1, 2, 1, 2]
    # ranked: 1 (0.5), then the 0.3 ties by depth then id: 2, 4, 3; then 5
    assert td.top_by_phat(phat, depth, 3) == [0, 1, 2, 4]
    assert td.select_verify(phat, depth, 5) == [0, 1, 2, 3, 4, 5]
    assert td.select_verify(phat, depth, 2) == [0, 1, 2]


def test_draft_mask_known_answer():
    # context slots [0, 8), root at slot 7; level 1 (nodes 1, 2) was forwarded at
    # slots 8, 9; the frontier [3, 4] (children of 1 and 2) goes to slots 10, 11
    parent = [-1, 0, 0, 1, 2]
    depth = [0, 1, 1, 2, 2]
    cache_idx = {0: 7, 1: 8, 2: 9}
    base, tree_cache = 8, 2
    want = np.zeros((2, 12), bool)
    want[0, :8] = True
    want[0, 8] = True   # ancestor 1
    want[0, 10] = True  # itself
    want[1, :8] = True
    want[1, 9] = True   # ancestor 2
    want[1, 11] = True  # itself
    assert (td.draft_mask(parent, cache_idx, depth, [3, 4], base, tree_cache, None) == want).all()
    # window 3: position base - 1 + depth = 9, so the prefix starts at 9 - 3 + 1 = 7
    want[:, :7] = False
    assert (td.draft_mask(parent, cache_idx, depth, [3, 4], base, tree_cache, 3) == want).all()


def _tiny():
    z = load_golden("drafter_tiny.npz")
    cfg = fixture_config(z)
    w = fixture_weights(z)
    return cfg, w


def test_width_one_tree_is_the_greedy_chain():
    cfg, w = _tiny()
    od = core.Drafter(cfg, w)
    rng = np.random.default_rng(3)
    H = cfg["hidden_size"]
    ctx, K = 6, 4
    cache = od.make_cache(64)
    # a context: forward ctx tokens from random features
    hid, out = od.forward(rng.integers(0, cfg["vocab_size"], ctx), rng.standard_normal((ctx, H)).astype(np.float32),
                          cache)
    root_out, root_fb = out[-1], od.feedback(hid, out)[-1]
    snap = (cache.k[0].copy(), cache.offset)
    tree, _, nodes = td.draft_tree_greedy(od, cache, 7, root_out, root_fb, max_depth=K, width=1, budget=K)
    assert cache.offset == snap[1]
    # the chain: argmax drafting with the causal forward at the cache offset
    cache.k[0][:] = snap[0]
    toks, o, f = [], root_out[None], root_fb[None]
    for k in range(K):
        z = od.logits(o)
        toks.append(int(od.token_ids([core.argmax(z[0])])[0]))
        if k < K - 1:
            h, o = od.forward([toks[-1]], f, cache)
            f = od.feedback(h, o)
    assert tree.tokens == [7] + toks
    assert tree.parents == [-1, 0, 1, 2, 3]
    assert tree.depth == [0, 1, 2, 3, 4]


def test_wider_tree_invariants():
    cfg, w = _tiny()
    od = core.Drafter(cfg, w)
    rng = np.random.default_rng(5)
    H = cfg["hidden_size"]
    cache = od.make_cache(96)
    hid, out = od.forward(rng.integers(0, cfg["vocab_size"], 5), rng.standard_normal((5, H)).astype(np.float32),
                          cache)
    width, depth, budget = 3, 3, 7
    tree, phat, nodes = td.draft_tree_greedy(od, cache, 1, out[-1], od.feedback(hid, out)[-1], depth, width, budget)
    assert len(nodes) == 1 + width + (depth - 1) * width * width
    assert len(tree) == budget + 1
    for i, p in enumerate(tree.parents[1:], start=1):
        assert 0 <= p < i and tree.depth[i] == tree.depth[p] + 1
    # siblings drafted in descending q: phat non-increasing within a parent's children
    for v in range(1, len(nodes), width):
        ph = [nodes[u][3] for u in range(v, v + width)]
        assert ph == sorted(ph, reverse=True)
    # the verified non-root nodes are the budget largest phat
    all_ph = sorted((n[3] for n in nodes[1:]), reverse=True)
    assert sorted(phat[1:], reverse=True) == all_ph[:budget]


# ------------------------------------------------------------------ sampled drafting (T > 0)

SEED = 29


def _pair_law(q: np.ndarray) -> np.ndarray:
    """Ordered pairs (a, b) of two draws without replacement: q_a * q_b / (1 - q_a)."""
    law = q[:, None] * q[None, :] / (1.0 - q[:, None])
    np.fill_diagonal(law, 0.0)
    return law.reshape(-1)


def _pair_pvalue(draw, q: np.ndarray, trials: int) -> float:
    V = q.size
    counts = np.zeros(V * V)
    for t in range(trials):
        a, b = draw(t)
        counts[a * V + b] += 1
    want = _pair_law(q) * trials
    live = want > 0
    if counts[~live].any():
        return 0.0
    return float(chisquare(counts[live], want[live] * counts[live].sum() / want[live].sum()).pvalue)


Q5 = np.array([0.05, 0.4, 0.0, 0.25, 0.3], np.float32)


def test_draws_follow_sequential_sampling_without_replacement():
    # node 3 of round t draws two children; the zero entry is never drawn
    assert _pair_pvalue(lambda t: td.sample_children(Q5, 2, 3, SEED, t, 1).tolist(), Q5.astype(np.float64),
                        20000) > OK_P


def test_control_wrong_sign_noise_is_caught():
    def draw(t):  # log q + log(-log u): the noise favours the unlikely entries
        nz, keys = td.gumbel_keys(Q5, 3, SEED, t, 1)
        noise = np.log(Q5[nz].astype(np.float64)) - keys
        bad = np.log(Q5[nz].astype(np.float64)) + noise
        return nz[np.lexsort((nz, -bad))[:2]].tolist()

    assert _pair_pvalue(draw, Q5.astype(np.float64), 20000) < BAD_P


def test_draw_count_and_zero_entries():
    q = np.array([0.0, 0.7, 0.0, 0.3], np.float32)
    for t in range(50):
        got = td.sample_children(q, 4, 0, SEED, t, 1)
        assert sorted(got.tolist()) == [1, 3]  # only the nonzero entries, each once
    assert td.sample_children(q, 0, 0, SEED, 0, 1).size == 0


def test_budget_split_known_answer():
    """Plan.children_for in frontier order: width 3, budget 7 -> the root draws 3,
    the level-1 frontier rows draw 3, 1, 0, and nothing is left for level 3."""
    V = 6
    Q = np.full((V, V), 1.0 / V, np.float32)
    token, parent, depth, phat, qrow = td.sampled_levels(
        lambda fr, lvl, tok, par, dep: Q[[tok[v] for v in fr]], None, 0, 3, 3, 7, SEED, 5, 1)
    assert depth.count(1) == 3 and depth.count(2) == 4 and depth.count(3) == 0
    kids = [sum(1 for p in parent if p == v) for v in range(1, 4)]
    assert kids == [3, 1, 0]  # frontier = level 1 in phat order; equal phat keeps node order
    # level 3 still runs (the frontier is not empty): its three rows get q and draw nothing
    assert len(token) == 1 + 7 and len(qrow) == 1 + 3 + 3 and {0, 1, 2, 3} <= set(qrow)
    for v in range(1, len(token)):
        assert phat[v] == pytest.approx(phat[parent[v]] / V, rel=1e-6)


class SampledTree:
    """A sampled tree drafted from the Markov world's Q, then the recursive rule."""

    def __init__(self, world, depth: int, width: int, budget: int, sample=None):
        self.w, self.depth, self.width, self.budget = world, depth, width, budget
        self.sample = sample

    def __call__(self, prev, rng):
        w = self.w
        rnd = int(rng.integers(1 << 40))
        Qf = w.Q.astype(np.float32)
        token, parent, depth, phat, qrow = td.sampled_levels(
            lambda fr, lvl, tok, par, dep: Qf[[tok[v] for v in fr]], None, prev, self.depth, self.width,
            self.budget, SEED, rnd, 1)
        tree = S.DraftTree(token, parent, depth)
        p = {v: w.P[t] for v, t in enumerate(token)}
        q = {v: S.scatter_draft_dist(qrow[v], None, w.V) for v in qrow}
        path, nxt = S.verify_tree_stochastic(p, q, tree, core.UniformStream(SEED, rnd, 0))
        return [token[v] for v in path] + [nxt]


@pytest.mark.parametrize("shape", [(2, 2, 4), (3, 2, 3), (3, 1, 3), (2, 3, 5)], ids=lambda s: "d%dw%db%d" % s)
def test_sampled_tree_round_emits_the_target_law(shape):
    assert WORLD.pvalue(WORLD.histogram(SampledTree(WORLD, *shape), 12000)) > OK_P


def test_control_one_uniform_vector_for_every_node_is_caught(monkeypatch):
    """Indexing the uniforms by head row alone makes a node's draws repeat its
    parent's noise: once the walk has gone through a rejection the proposal
    depends on what was already drawn."""
    real = td.sample_children
    monkeypatch.setattr(td, "sample_children", lambda q, m, v, seed, r, purpose: real(q, m, 0, seed, r, purpose))
    assert WORLD.pvalue(WORLD.histogram(SampledTree(WORLD, 3, 2, 6), 12000)) < BAD_P


def test_control_pruning_a_draw_by_its_probability_is_caught(monkeypatch):
    """Dropping a drawn child because its own q is low (policies.py:11-15): the
    children left are no longer draws from q in order."""
    real = td.sample_children

    def pruned(q, m, v, seed, r, purpose):
        rows = real(q, m, v, seed, r, purpose)
        if rows.size > 1 and q[rows[0]] < 0.2:
            rows = rows[1:]
        return rows

    monkeypatch.setattr(td, "sample_children", pruned)
    assert WORLD.pvalue(WORLD.histogram(SampledTree(WORLD, 2, 2, 4), 12000)) < BAD_P
