"""CPU restatement of greedy tree drafting (test infrastructure only).

Follows SpeculativeDecoder._draft in greedy mode with a StaticPolicy
(python/woodcock/spec.py:216-303) and the policy hooks it calls
(python/woodcock/policies.py:25-75): per level the frontier's draft
distributions q = softmax(z) (spec.py:120-121), the `width` most probable head
rows of each frontier node as children with phat = phat(parent) * q
(spec.py:226-237), the next frontier = the `width` level nodes of largest phat
(Policy.select_frontier, policies.py:52-53), one drafter forward over the
frontier with positions n - 1 + depth and the tree mask of _draft_mask
(spec.py:270-294), and finally select_verify / _top_by_phat / _to_tree
(policies.py:66-75; spec.py:297-303).

The reference takes the `width` rows from mx.argpartition, whose order within
the selected set is unspecified; here (as on the device) the children of a
node are in descending q order, the lower head row first on a tie.
"""
from __future__ import annotations

import numpy as np

from . import core
from .sampling import DraftTree, probs_from_logits


def top_children(q_row: np.ndarray, width: int) -> np.ndarray:
    """Head rows of the `width` largest q, descending, lower row first on a tie."""
    rows = np.arange(q_row.size)
    order = np.lexsort((rows, -q_row.astype(np.float64)))
    return order[:width]


def select_frontier(level_nodes, phat, depth, width):
    """Policy.select_frontier (policies.py:52-53): a stable sort by (-phat, depth)."""
    return sorted(level_nodes, key=lambda v: (-phat[v], depth[v]))[:width]


def top_by_phat(phat, depth, k):
    """_top_by_phat (policies.py:73-75): root plus the k best non-root nodes, in node order."""
    order = sorted(range(1, len(phat)), key=lambda v: (-phat[v], depth[v], v))[:k]
    return [0] + sorted(order)


def select_verify(phat, depth, budget):
    """StaticPolicy.select_verify (policies.py:66-69), greedy."""
    if len(phat) - 1 <= budget:
        return list(range(len(phat)))
    return top_by_phat(phat, depth, budget)


def draft_mask(parent, cache_idx, depth, frontier, base, tree_cache, window):
    """SpeculativeDecoder._draft_mask (spec.py:280-294)."""
    m = len(frontier)
    mask = np.zeros((m, base + tree_cache + m), dtype=bool)
    for r, v in enumerate(frontier):
        pos = base - 1 + depth[v]
        lo = 0 if not window else max(0, pos - window + 1)
        mask[r, lo:base] = True
        u = parent[v]
        while u > 0:
            mask[r, cache_idx[u]] = True
            u = parent[u]
        mask[r, base + tree_cache + r] = True
    return mask


def draft_tree_greedy(od: core.Drafter, cache: core.Cache, root_token: int, root_out: np.ndarray,
                      root_fb: np.ndarray, max_depth: int, width: int, budget: int):
    """One greedy tree-drafting phase at drafter context n = cache.offset.
    Returns (DraftTree of the verified nodes, phat of those nodes, every node's
    (token, parent, depth, phat)).  The cache offset is restored on return."""
    n = base = cache.offset
    token, parent, depth, phat = [int(root_token)], [-1], [0], [1.0]
    out = {0: np.asarray(root_out, np.float32).reshape(-1)}
    fb = {0: np.asarray(root_fb, np.float32).reshape(-1)}
    cache_idx = {0: n - 1}
    frontier = [0]
    tree_cache = 0
    d2t = od.d2t
    for lvl in range(1, max_depth + 1):
        z = od.logits(np.stack([out[v] for v in frontier]))
        q = probs_from_logits(z, 1.0)
        first = len(token)
        for r, v in enumerate(frontier):
            for row in top_children(q[r], width):
                token.append(int(d2t[row]) if d2t is not None else int(row))
                parent.append(v)
                depth.append(lvl)
                phat.append(phat[v] * float(q[r, row]))
        level_nodes = list(range(first, len(token)))
        if lvl == max_depth:
            break
        frontier = select_frontier(level_nodes, phat, depth, width)
        if not frontier:
            break
        toks = [token[v] for v in frontier]
        feats = np.stack([fb[parent[v]] for v in frontier])
        pos = [n - 1 + depth[v] for v in frontier]
        mask = draft_mask(parent, cache_idx, depth, frontier, base, tree_cache, od.cfg.get("window"))
        cache.offset = base + tree_cache
        hid, o = od.forward(toks, feats, cache, positions=pos, mask=mask)
        f = od.feedback(hid, o)
        for r, v in enumerate(frontier):
            out[v], fb[v] = o[r], f[r]
            cache_idx[v] = base + tree_cache + r
        tree_cache += len(frontier)
    cache.offset = base
    keep = select_verify(phat, depth, budget)
    remap = {v: i for i, v in enumerate(keep)}
    tree = DraftTree(tokens=[token[v] for v in keep], parents=[remap.get(parent[v], -1) for v in keep],
                     depth=[depth[v] for v in keep])
    return tree, [phat[v] for v in keep], list(zip(token, parent, depth, phat))
