"""numpy restatement of Woodcock's verification rules (test infrastructure only).

Follows python/woodcock/sampling.py (rules, uniform-consumption order, fp64
decisions, thresholds) and the engine-side handling of draft distributions in
python/woodcock/spec.py:113-125,238-248,316-324.  ``rng`` is anything with a
``random(size=None)`` method: a numpy Generator (the reference's own tests) or
``oracle.core.UniformStream`` (the counter-based stream the HIP kernels read).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np


# ------------------------------------------------------------------ distributions

def probs_from_logits(logits, temperature: float, top_k: int = 0, top_p: float = 1.0) -> np.ndarray:
    """Warped float32 distribution over the last axis (sampling.py:39-55;
    sampling.cpp:9-45).

    x = logits / T in fp32; top-k drops every x below the k-th largest x (ties
    with it stay, sampling.py:41-43); softmax as numpy fp32 (max-shifted exp,
    normalised by the row sum).  Top-p follows the reference runtime's
    arithmetic (sampling.cpp:28-44): in descending order (equal values lower
    index first) an entry stays while the fp64 mass before it is below top_p,
    and the kept entries are divided by their fp64 sum.  (An fp32 running sum,
    as the MLX path forms it, drifts by ~1e-4 over a 10^5-entry row, more than
    the entries at the boundary.)"""
    x = np.asarray(logits, dtype=np.float32) / np.float32(max(temperature, 1e-6))
    if top_k and top_k < x.shape[-1]:
        kth = np.sort(x, axis=-1)[..., -top_k][..., None]
        x = np.where(x < kth, np.float32(-np.inf), x)
    e = np.exp(x - x.max(axis=-1, keepdims=True))
    p = (e / e.sum(axis=-1, keepdims=True)).astype(np.float32)
    if top_p < 1.0:
        order = np.argsort(-p, axis=-1, kind="stable")
        srt = np.take_along_axis(p, order, axis=-1).astype(np.float64)
        before = np.cumsum(srt, axis=-1) - srt
        before[..., 1:] = np.cumsum(srt, axis=-1)[..., :-1]  # the exclusive sums themselves, not a difference
        before[..., 0] = 0.0
        keep_sorted = before < top_p  # the first entry is always kept
        keep = np.zeros_like(p, dtype=bool)
        np.put_along_axis(keep, order, keep_sorted, axis=-1)
        kept = np.where(keep, p, np.float32(0)).astype(np.float64)
        p = (kept / kept.sum(axis=-1, keepdims=True)).astype(np.float32)
    return p


def scatter_draft_dist(q_rows: np.ndarray, d2t: np.ndarray | None, vocab: int) -> np.ndarray:
    """Draft distribution over the restricted head rows -> fp64 over the full
    vocabulary, renormalised (spec.py:240-248)."""
    q_rows = np.asarray(q_rows, dtype=np.float64)
    qv = np.zeros(vocab)
    if d2t is None:
        qv[: q_rows.shape[-1]] = q_rows
    else:
        qv[np.asarray(d2t)] = q_rows
    qv /= qv.sum()
    return qv


# ------------------------------------------------------------------ helpers

def residual(p: np.ndarray, q: np.ndarray) -> np.ndarray:
    """norm(max(p - q, 0)); p itself renormalised when the residual mass is <= 1e-12
    (sampling.py:182-187)."""
    r = np.maximum(p - q, 0.0)
    s = r.sum()
    if s <= 1e-12:
        return p / p.sum()
    return r / s


def sample(p: np.ndarray, rng) -> int:
    """Inverse CDF: first i with cumsum(p)[i] > u * total, clamped (sampling.py:190-193)."""
    c = np.cumsum(np.asarray(p, dtype=np.float64))
    return int(min(np.searchsorted(c, rng.random() * c[-1], side="right"), len(c) - 1))


def sample_without_replacement(q: np.ndarray, k: int, rng) -> list[int]:
    """Gumbel-top-k over the nonzero entries, one uniform per nonzero entry
    (sampling.py:196-203)."""
    q = np.asarray(q, dtype=np.float64)
    nz = np.flatnonzero(q > 0)
    k = min(k, len(nz))
    g = np.log(q[nz]) - np.log(-np.log(rng.random(len(nz))))
    return [int(nz[i]) for i in np.argsort(-g)[:k]]


# ------------------------------------------------------------------ chains

def verify_chain_greedy(target_logits, draft_tokens) -> tuple[int, int]:
    """(n_accepted, next_token) for target logits at [x_n, d_1..d_K] (sampling.py:60-66)."""
    t = np.argmax(np.asarray(target_logits), axis=-1).tolist()
    n = 0
    while n < len(draft_tokens) and t[n] == draft_tokens[n]:
        n += 1
    return n, t[n]


def verify_chain_stochastic(p, q, draft_tokens, rng) -> tuple[int, int]:
    """Leviathan/Chen chain rule (sampling.py:69-82): q_i(x) <= 0 rejects without a
    uniform; otherwise accept iff u < min(1, p/q); the first rejection samples the
    residual; all accepted samples a bonus token from p_K."""
    K = len(draft_tokens)
    for i, x in enumerate(draft_tokens):
        qi = q[i, x]
        accept = False if qi <= 0 else rng.random() < min(1.0, p[i, x] / qi)
        if not accept:
            return i, sample(residual(p[i], q[i]), rng)
    return K, sample(p[K], rng)


# ------------------------------------------------------------------ trees

@dataclass
class DraftTree:
    """Flattened draft tree; node 0 is the root.  children[v] keeps draw order
    (node index order) (sampling.py:87-115)."""

    tokens: list[int]
    parents: list[int]
    depth: list[int]
    children: list[list[int]] = field(default_factory=list)

    def __post_init__(self):
        if not self.children:
            self.children = [[] for _ in self.tokens]
            for v, par in enumerate(self.parents):
                if par >= 0:
                    self.children[par].append(v)

    def __len__(self):
        return len(self.tokens)

    def path_to(self, v: int) -> list[int]:
        out = []
        while v > 0:
            out.append(v)
            v = self.parents[v]
        return out[::-1]


def tree_attention_mask(tree: DraftTree, prefix_len: int) -> np.ndarray:
    """(N, prefix+N) bool: the prefix plus every ancestor, self included (sampling.py:118-128)."""
    N = len(tree)
    m = np.zeros((N, prefix_len + N), dtype=bool)
    m[:, :prefix_len] = True
    for v in range(N):
        u = v
        while u >= 0:
            m[v, prefix_len + u] = True
            u = tree.parents[u]
    return m


def verify_tree_greedy(target_argmax, tree: DraftTree) -> tuple[list[int], int]:
    """Walk from the root taking the first child (draw order) whose token is the
    target argmax (sampling.py:131-140)."""
    v, path = 0, []
    while True:
        want = int(target_argmax[v])
        nxt = next((c for c in tree.children[v] if tree.tokens[c] == want), None)
        if nxt is None:
            return path, want
        path.append(nxt)
        v = nxt


def verify_tree_stochastic(p: dict, q: dict, tree: DraftTree, rng) -> tuple[list[int], int]:
    """Recursive rejection sampling over children drawn without replacement
    (sampling.py:143-177)."""
    v, path = 0, []
    while True:
        kids = tree.children[v]
        p_cur = np.asarray(p[v], dtype=np.float64)
        if not kids:
            return path, sample(p_cur, rng)
        q_cur = np.asarray(q[v], dtype=np.float64).copy()
        accepted = None
        for c in kids:
            x = tree.tokens[c]
            qx = q_cur[x]
            if qx > 0 and rng.random() < min(1.0, p_cur[x] / qx):
                accepted = c
                break
            p_cur = residual(p_cur, q_cur)
            q_cur[x] = 0.0
            s = q_cur.sum()
            if s <= 0:
                break
            q_cur /= s
        if accepted is None:
            return path, sample(p_cur, rng)
        path.append(accepted)
        v = accepted


# ------------------------------------------------------------------ engine-level chain round

def chain_stochastic_round(target_probs, draft_probs, d2t, draft_tokens, rng) -> tuple[int, int]:
    """What the engine does for a width-1 stochastic round: fp32 target probs ->
    fp64 (spec.py:321), draft probs scattered through d2t and renormalised in fp64
    (spec.py:240-248), then verify_tree_stochastic on the chain (spec.py:323-324)."""
    tp = np.asarray(target_probs, dtype=np.float32)
    V = tp.shape[-1]
    K = len(draft_tokens)
    tree = DraftTree([0] + list(draft_tokens), list(range(-1, K)), list(range(K + 1)))
    p = {v: tp[v].astype(np.float64) for v in range(K + 1)}
    q = {v: scatter_draft_dist(np.asarray(draft_probs, dtype=np.float32)[v], d2t, V) for v in range(K)}
    path, nxt = verify_tree_stochastic(p, q, tree, rng)
    return len(path), nxt
