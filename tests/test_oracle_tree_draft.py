"""Pins the greedy tree-drafting restatement (oracle/tree_draft.py) on the CPU.

- the selection rules against hand-worked answers, ties included
  (policies.py:52-53,66-75; spec.py:226-237);
- the drafter tree mask against a hand-drawn matrix, with and without a
  sliding window (spec.py:280-294);
- width 1 reduces tree drafting to the greedy chain: the drafted tokens equal
  argmax drafting with the drafter's own causal forward (spec.py:331-350), on
  the reference-pinned tiny drafter fixture;
- structural invariants of a wider tree (parent closure of the verified set,
  sibling order, phat products).
"""
import numpy as np

from conftest import load_golden
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
