"""The oracle's verification rules against the exact law they must preserve.

Same construction as the reference's distribution tests
(tests/test_sampling.py:1-180): a first-order Markov target P[prev] and drafter
Q[prev] over a 5-token vocabulary make the joint law of the first three emitted
tokens exact; the full draft -> verify -> emit loop runs many times and a
chi-square test compares the histogram with that law.  Negative controls
(biased drafting rules) must fail the same test, which shows it has power.
Known answers (tests/test_sampling.py:185-216) pin the greedy rules, the mask
and the warping; the special cases q(x) = 0, p == q and T -> 0 are checked
against what the rules fix in closed form.
"""
import itertools

import numpy as np
import pytest
from scipy.stats import chisquare

from oracle import core
from oracle import sampling as S

V = 5
N_EMIT = 3
TRIALS = 20000


def _markov(seed, sharp):
    return np.random.default_rng(seed).dirichlet(np.full(V, sharp), size=V)


P = _markov(1, 0.7)
Q = 0.5 * _markov(2, 0.7) + 0.5 * P
Q_TRUNC = Q * (np.arange(V) < 3)
Q_TRUNC /= Q_TRUNC.sum(-1, keepdims=True)


def exact_law(root=0):
    law = np.zeros((V,) * N_EMIT)
    for seq in itertools.product(range(V), repeat=N_EMIT):
        pr, prev = 1.0, root
        for t in seq:
            pr *= P[prev, t]
            prev = t
        law[seq] = pr
    return law.ravel()


def run(gen_round, trials=TRIALS, seed=0):
    rng = np.random.default_rng(seed)
    counts = np.zeros(V ** N_EMIT)
    for _ in range(trials):
        out = []
        while len(out) < N_EMIT:
            prev = out[-1] if out else 0
            out.extend(gen_round(prev, rng))
        counts[np.ravel_multi_index(tuple(out[:N_EMIT]), (V,) * N_EMIT)] += 1
    return counts


def chi2_pvalue(counts):
    exp = exact_law() * counts.sum()
    keep = exp > 0
    return chisquare(counts[keep], exp[keep] * counts[keep].sum() / exp[keep].sum()).pvalue


def chain_round(K, Qm=Q, engine=False):
    def gen(prev, rng):
        toks, qs, ps = [], [], [P[prev]]
        cur = prev
        for _ in range(K):
            x = int(rng.choice(V, p=Qm[cur]))
            qs.append(Qm[cur])
            toks.append(x)
            cur = x
            ps.append(P[cur])
        if engine:  # the engine's path: fp32 probabilities, tree rule at width 1
            n, nxt = S.chain_stochastic_round(np.array(ps, np.float32), np.array(qs, np.float32), None, toks, rng)
        else:
            n, nxt = S.verify_chain_stochastic(np.array(ps), np.array(qs), toks, rng)
        return toks[:n] + [nxt]

    return gen


@pytest.mark.parametrize("K", [1, 3])
def test_chain_stochastic_preserves_target(K):
    assert chi2_pvalue(run(chain_round(K))) > 1e-3


@pytest.mark.parametrize("K", [1, 3])
def test_chain_stochastic_truncated_draft_vocab_preserves_target(K):
    assert chi2_pvalue(run(chain_round(K, Q_TRUNC))) > 1e-3


def test_engine_chain_round_preserves_target():
    assert chi2_pvalue(run(chain_round(3, engine=True))) > 1e-3


def build_tree(prev, rng, depth, width, draw_wor=True, Qm=Q):
    tokens, parents, depths = [prev], [-1], [0]
    frontier = [0]
    for d in range(1, depth + 1):
        nxt = []
        for v in frontier:
            kids = (S.sample_without_replacement(Qm[tokens[v]], width, rng) if draw_wor
                    else list(np.argsort(-Qm[tokens[v]])[:width]))
            for x in kids:
                tokens.append(int(x))
                parents.append(v)
                depths.append(d)
                nxt.append(len(tokens) - 1)
        frontier = nxt
    return S.DraftTree(tokens, parents, depths)


def tree_round(depth, width, draw_wor=True, Qm=Q):
    def gen(prev, rng):
        tree = build_tree(prev, rng, depth, width, draw_wor, Qm)
        p = {v: P[t] for v, t in enumerate(tree.tokens)}
        q = {v: Qm[t] for v, t in enumerate(tree.tokens)}
        path, nxt = S.verify_tree_stochastic(p, q, tree, rng)
        return [tree.tokens[v] for v in path] + [nxt]

    return gen


@pytest.mark.parametrize("depth,width", [(1, 2), (2, 3)])
def test_tree_stochastic_preserves_target(depth, width):
    assert chi2_pvalue(run(tree_round(depth, width), trials=12000)) > 1e-3


def test_tree_stochastic_truncated_draft_vocab_preserves_target():
    assert chi2_pvalue(run(tree_round(2, 2, Qm=Q_TRUNC), trials=12000)) > 1e-3


def test_negative_control_topk_children_is_biased():
    assert chi2_pvalue(run(tree_round(1, 2, draw_wor=False))) < 1e-6


def test_negative_control_stopping_on_current_draw_is_biased():
    def gen(prev, rng):
        x = int(rng.choice(V, p=Q[prev]))
        if Q[prev, x] < 0.3:
            return [int(rng.choice(V, p=P[prev]))]
        n, nxt = S.verify_chain_stochastic(np.array([P[prev], P[x]]), np.array([Q[prev]]), [x], rng)
        return [x, nxt][: n + 1]

    assert chi2_pvalue(run(gen)) < 1e-6


def test_negative_control_planted_bias_in_residual_is_detected():
    """A plausible mistake -- sampling the rejection from p instead of the
    residual -- must fail the law (the oracle's test has power against it)."""
    def gen(prev, rng):
        x = int(rng.choice(V, p=Q[prev]))
        if rng.random() < min(1.0, P[prev, x] / Q[prev, x]):
            return [x]
        return [S.sample(P[prev], rng)]

    assert chi2_pvalue(run(gen)) < 1e-6


def test_stopping_on_past_draws_is_unbiased():
    def gen(prev, rng):
        K = 2 if Q[prev].max() > 0.4 else 1
        return chain_round(K)(prev, rng)

    assert chi2_pvalue(run(gen)) > 1e-3


# ------------------------------------------------------------------ special cases (closed form)

class Counting:
    def __init__(self, values):
        self.values, self.n = list(values), 0

    def random(self, size=None):
        assert size is None
        v = self.values[self.n]
        self.n += 1
        return v


def test_zero_draft_probability_consumes_no_uniform():
    p = np.array([[0.1, 0.2, 0.3, 0.4], [0.25] * 4])
    q = np.array([[0.5, 0.5, 0.0, 0.0]])
    rng = Counting([0.0, 0.99])
    n, nxt = S.verify_chain_stochastic(p, q, [2], rng)
    # rejected without a draw; the residual max(p - q, 0) = [0, 0, .3, .4] / .7 sampled with u = 0.0
    assert (n, nxt, rng.n) == (0, 2, 1)


def test_equal_distributions_accept_and_fall_back_to_p():
    p = np.array([[0.1, 0.2, 0.3, 0.4]] * 2)
    # p == q: every draw is accepted (ratio 1 > u for u < 1)
    rng = Counting([0.999999, 0.5])
    assert S.verify_chain_stochastic(p, p[:1].copy(), [3], rng) == (1, 2) and rng.n == 2
    # the residual of p against itself is empty -> p renormalised (sampling.py:184-185)
    r = S.residual(p[0], p[0])
    np.testing.assert_array_equal(r, p[0] / p[0].sum())


def test_inverse_cdf_boundaries():
    p = np.array([0.0, 0.5, 0.0, 0.5])
    assert S.sample(p, Counting([0.0])) == 1        # first index with c > 0
    assert S.sample(p, Counting([0.5])) == 3        # c = [0, .5, .5, 1]: first c > .5
    assert S.sample(p, Counting([0.9999999])) == 3


def test_low_temperature_is_greedy():
    logits = np.array([[2.0, 5.0, 1.0, 4.99]], np.float32)
    p = S.probs_from_logits(logits, 1e-9)
    assert p.argmax() == 1 and p[0, 1] == 1.0


def test_chain_rule_equals_tree_rule_at_width_one():
    """verify_chain_stochastic and verify_tree_stochastic on a chain consume the
    same uniforms in the same order (sampling.py:69-82 vs 143-177)."""
    r = np.random.default_rng(5)
    for trial in range(300):
        K = int(r.integers(1, 5))
        ps = r.dirichlet(np.full(7, 0.5), size=K + 1)
        qs = r.dirichlet(np.full(7, 0.5), size=K)
        qs[:, r.integers(0, 7)] = 0
        qs /= qs.sum(-1, keepdims=True)
        toks = [int(r.integers(0, 7)) for _ in range(K)]
        a = core.UniformStream(11, trial)
        b = core.UniformStream(11, trial)
        n1, x1 = S.verify_chain_stochastic(ps, qs, toks, a)
        tree = S.DraftTree([0] + toks, list(range(-1, K)), list(range(K + 1)))
        path, x2 = S.verify_tree_stochastic({v: ps[v] for v in range(K + 1)}, {v: qs[v] for v in range(K)}, tree, b)
        assert (n1, x1, a.pos) == (len(path), x2, b.pos)


# ------------------------------------------------------------------ known answers (tests/test_sampling.py:185-216)

def test_greedy_chain_and_tree_known_answers():
    logits = np.log(P[[0, 3, 1]])
    want = np.argmax(P[[0, 3, 1]], axis=-1)
    assert S.verify_chain_greedy(logits, [int(want[0]), int(want[1])]) == (2, want[2])
    assert S.verify_chain_greedy(logits, [int((want[0] + 1) % V), int(want[1])]) == (0, want[0])
    tree = S.DraftTree(tokens=[0, 1, 2, 4], parents=[-1, 0, 0, 2], depth=[0, 1, 1, 2])
    assert S.verify_tree_greedy([2, 9, 4, 3], tree) == ([2, 3], 3)


def test_tree_mask_known_answer():
    tree = S.DraftTree(tokens=[0, 1, 2, 4], parents=[-1, 0, 0, 2], depth=[0, 1, 1, 2])
    m = S.tree_attention_mask(tree, prefix_len=2)
    assert m.shape == (4, 6) and m[:, :2].all()
    assert list(m[3, 2:]) == [True, False, True, True]
    assert list(m[1, 2:]) == [True, True, False, False]


def test_probs_warping_known_answers():
    logits = np.array([[2.0, 1.0, 0.0, -1.0]], np.float32)
    p = S.probs_from_logits(logits, 1.0, top_k=2)
    assert p[0, 2] == 0 and p[0, 3] == 0 and abs(p.sum() - 1) < 1e-6
    p = S.probs_from_logits(logits, 1.0, top_p=0.5)
    assert (p[0] > 0).sum() == 1
    p = S.probs_from_logits(logits, 0.5)
    ref = np.exp(np.array([2, 1, 0, -1.0]) / 0.5)
    np.testing.assert_allclose(p[0], ref / ref.sum(), rtol=1e-5)
