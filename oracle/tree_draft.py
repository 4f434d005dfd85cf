"""CPU restatement of tree drafting, greedy and sampled (test infrastructure only).

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

Sampled drafting (T > 0) follows the stochastic branch (spec.py:238-249): the
frontier's q = softmax(z / T) (spec.py:121-124), per frontier node in order
m = Plan.children_for (policies.py:32-36) children drawn without replacement
by Gumbel-top-m (sampling.py:196-203), phat = phat(parent) * q(x) / sum(q)
(the renormalised, scattered q of spec.py:243-248), every node verified
(policies.py:67-69).  The uniforms follow the HIP kernels' indexing instead of
one sequential generator: head row i of frontier node v reads value
v * H4 + i of the Philox stream (H4 = head rows rounded up to 4).  Each
nonzero entry still gets its own fresh uniform, so the draws have the
reference's law; tests/test_oracle_tree_draft.py pins that law.
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


# ------------------------------------------------------------------ sampled drafting (T > 0)

def gumbel_keys(q_row: np.ndarray, v: int, seed: int, round_: int, purpose: int):
    """(nonzero head rows, their keys log q - log(-log u)) of frontier node v."""
    q32 = np.asarray(q_row, dtype=np.float32)
    h4 = (q32.size + 3) // 4 * 4
    u = core.uniforms(seed, round_, purpose, v * h4, q32.size)
    nz = np.flatnonzero(q32 > 0)
    with np.errstate(divide="ignore"):
        keys = np.log(q32[nz].astype(np.float64)) - np.log(-np.log(u[nz]))
    return nz, keys


def sample_children(q_row: np.ndarray, m: int, v: int, seed: int, round_: int, purpose: int) -> np.ndarray:
    """The m draws of frontier node v, in descending key order (lower row first on a tie)."""
    nz, keys = gumbel_keys(q_row, v, seed, round_, purpose)
    return nz[np.lexsort((nz, -keys))[: min(m, nz.size)]]


def sampled_levels(q_of, d2t, root_token: int, max_depth: int, width: int, budget: int, seed: int, round_: int,
                   purpose: int, follow=None, key_tol: float = 1e-3):
    """The level loop of sampled drafting.  q_of(frontier, level, token, parent,
    depth) -> fp32 q rows of the frontier (it forwards the frontier first when
    level > 1).  follow: the node tokens of another implementation; where its
    draws differ from these, the keys of both choices must agree within key_tol
    (a near-tie under rounding) and its choice is taken.
    Returns (token, parent, depth, phat, {node: q row of its children's draws})."""
    token, parent, depth, phat = [int(root_token)], [-1], [0], [1.0]
    qrow = {}
    frontier = [0]
    remaining = budget
    for lvl in range(1, max_depth + 1):
        q = q_of(frontier, lvl, token, parent, depth)
        first = len(token)
        for r, v in enumerate(frontier):
            qrow[v] = q[r]
            m = max(min(width, remaining), 0)  # Plan.children_for
            remaining -= m
            rows = sample_children(q[r], m, v, seed, round_, purpose)
            if follow is not None:
                theirs = np.asarray(follow[len(token):len(token) + rows.size], dtype=np.int64)
                ours = np.asarray(d2t)[rows] if d2t is not None else rows
                assert theirs.size == rows.size, f"node {v}: {theirs.size} draws vs {rows.size}"
                if not np.array_equal(theirs, ours):
                    nz, keys = gumbel_keys(q[r], v, seed, round_, purpose)
                    their_rows = np.searchsorted(np.asarray(d2t), theirs) if d2t is not None else theirs
                    kmap = dict(zip(nz.tolist(), keys.tolist()))
                    for a, b in zip(rows.tolist(), their_rows.tolist()):
                        assert b in kmap and abs(kmap[a] - kmap[b]) <= key_tol, f"node {v}: draws differ"
                    rows = their_rows
            mass = float(np.asarray(q[r], dtype=np.float64).sum())
            for row in rows.tolist():
                token.append(int(d2t[row]) if d2t is not None else int(row))
                parent.append(v)
                depth.append(lvl)
                phat.append(phat[v] * (float(q[r][row]) / mass))
        level_nodes = list(range(first, len(token)))
        if lvl == max_depth:
            break
        frontier = select_frontier(level_nodes, phat, depth, width)
        if not frontier:
            break
    return token, parent, depth, phat, qrow


def draft_tree_sample(od: core.Drafter, cache: core.Cache, root_token: int, root_out: np.ndarray,
                      root_fb: np.ndarray, max_depth: int, width: int, budget: int, temperature: float, seed: int,
                      round_: int, purpose: int, follow=None, key_tol: float = 1e-3):
    """One sampled tree-drafting phase at drafter context n = cache.offset.
    Returns (DraftTree of every node, phat, {node: fp32 q row over the head
    rows}).  The cache offset is restored on return."""
    n = base = cache.offset
    out = {0: np.asarray(root_out, np.float32).reshape(-1)}
    fb = {0: np.asarray(root_fb, np.float32).reshape(-1)}
    cache_idx = {0: n - 1}
    tree_cache = [0]

    def q_of(frontier, lvl, token, parent, depth):
        if lvl > 1:
            tc = tree_cache[0]
            toks = [token[v] for v in frontier]
            feats = np.stack([fb[parent[v]] for v in frontier])
            pos = [n - 1 + depth[v] for v in frontier]
            mask = draft_mask(parent, cache_idx, depth, frontier, base, tc, od.cfg.get("window"))
            cache.offset = base + tc
            hid, o = od.forward(toks, feats, cache, positions=pos, mask=mask)
            f = od.feedback(hid, o)
            for r, v in enumerate(frontier):
                out[v], fb[v] = o[r], f[r]
                cache_idx[v] = base + tc + r
            tree_cache[0] = tc + len(frontier)
        z = od.logits(np.stack([out[v] for v in frontier]))
        return probs_from_logits(z, temperature)

    token, parent, depth, phat, qrow = sampled_levels(q_of, od.d2t, root_token, max_depth, width, budget, seed,
                                                      round_, purpose, follow, key_tol)
    cache.offset = base
    return DraftTree(tokens=token, parents=parent, depth=depth), phat, qrow
