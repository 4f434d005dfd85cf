"""The oracle's verification rules against the law they must preserve.

Speculative sampling is correct when the emitted tokens follow the target's
law exactly.  A first-order Markov target P[prev] over a tiny vocabulary makes
that law computable in closed form for the first few emitted tokens; the
drafter Q[prev] differs from P, so every rejection and residual draw is
exercised.  Each rule below runs the whole draft -> verify -> emit loop many
times, the emitted prefixes are histogrammed, and a chi-square test
(scipy.stats.chisquare) compares the histogram with the closed-form law.
Negative controls -- rules that are wrong in ways an implementation could be --
must fail the same test, which shows it has the power to catch them.

The world's construction (sizes, seeds, concentrations, truncation, chain and
tree shapes, thresholds) and the known answers are the reference tests' data
(tests/golden/reference_cases.json, from the reference's
tests/test_sampling.py); the harness is written here.
"""
import json
from functools import reduce
from pathlib import Path

import numpy as np
import pytest
from scipy.stats import chisquare

from oracle import core
from oracle import sampling as S

DATA = json.loads((Path(__file__).parent / "golden" / "reference_cases.json").read_text())
MK = DATA["markov"]


class MarkovWorld:
    """Target P and drafter Q, both row-stochastic [V][V] (row = previous token)."""

    def __init__(self, spec: dict, truncate: bool = False):
        self.V, self.emit, self.root = spec["vocab"], spec["emit"], spec["root"]
        t, d = spec["target"], spec["draft"]
        self.P = np.random.default_rng(t["seed"]).dirichlet(np.full(self.V, t["concentration"]), size=self.V)
        mix = d["mix_with_target"]
        raw = np.random.default_rng(d["seed"]).dirichlet(np.full(self.V, d["concentration"]), size=self.V)
        self.Q = mix * raw + (1.0 - mix) * self.P
        if truncate:  # a trimmed draft vocabulary: q = 0 on tokens the target still emits
            keep = np.arange(self.V) < spec["truncated_draft_vocab"]
            self.Q = self.Q * keep
            self.Q /= self.Q.sum(axis=1, keepdims=True)

    def law(self) -> np.ndarray:
        """Joint law of the first `emit` tokens after the root, flattened in C order."""
        joint = self.P[self.root]
        for _ in range(self.emit - 1):
            last = np.arange(joint.size) % self.V  # the last token of each prefix
            joint = (joint[:, None] * self.P[last]).reshape(-1)  # append one token
        return joint

    def histogram(self, propose, trials: int, seed: int = 0) -> np.ndarray:
        """Emitted-prefix counts over `trials` independent generations."""
        rng = np.random.default_rng(seed)
        codes = np.empty(trials, np.int64)
        weights = self.V ** np.arange(self.emit - 1, -1, -1)
        for i in range(trials):
            seq = []
            while len(seq) < self.emit:
                seq += propose(seq[-1] if seq else self.root, rng)
            codes[i] = int(np.dot(seq[: self.emit], weights))
        return np.bincount(codes, minlength=self.V ** self.emit).astype(np.float64)

    def pvalue(self, counts: np.ndarray) -> float:
        want = self.law() * counts.sum()
        live = want > 0
        if counts[~live].any():  # a prefix the target cannot produce was emitted
            return 0.0
        return float(chisquare(counts[live], want[live] * counts[live].sum() / want[live].sum()).pvalue)


WORLD = MarkovWorld(MK)
TRUNC = MarkovWorld(MK, truncate=True)
OK_P, BAD_P = MK["accept_pvalue"], MK["reject_pvalue"]


# ------------------------------------------------------------------ proposers (one round each)

class Chain:
    """K drafts from Q along the chain, then the chain rule (or the engine's path:
    fp32 probabilities through the tree rule at width 1)."""

    def __init__(self, world: MarkovWorld, K: int, engine: bool = False):
        self.w, self.K, self.engine = world, K, engine

    def __call__(self, prev, rng):
        w = self.w
        ctx = [prev]
        for _ in range(self.K):
            ctx.append(int(rng.choice(w.V, p=w.Q[ctx[-1]])))
        drafts = ctx[1:]
        p, q = w.P[ctx], w.Q[ctx[:-1]]
        if self.engine:
            n, nxt = S.chain_stochastic_round(p.astype(np.float32), q.astype(np.float32), None, drafts, rng)
        else:
            n, nxt = S.verify_chain_stochastic(p, q, drafts, rng)
        return drafts[:n] + [nxt]


class Tree:
    """A full tree: every node at depth < `depth` gets `width` children, drawn
    from Q[node] without replacement (or, as a control, Q's top entries)."""

    def __init__(self, world: MarkovWorld, depth: int, width: int, children: str = "draw"):
        self.w, self.depth, self.width, self.children = world, depth, width, children

    def _kids(self, tok, rng):
        q = self.w.Q[tok]
        if self.children == "draw":
            return S.sample_without_replacement(q, self.width, rng)
        return list(np.argsort(-q)[: self.width])

    def __call__(self, prev, rng):
        toks, par, dep = [prev], [-1], [0]
        level = [0]
        for d in range(1, self.depth + 1):
            nxt_level = []
            for v in level:
                for x in self._kids(toks[v], rng):
                    toks.append(int(x))
                    par.append(v)
                    dep.append(d)
                    nxt_level.append(len(toks) - 1)
            level = nxt_level
        tree = S.DraftTree(toks, par, dep)
        p = {v: self.w.P[t] for v, t in enumerate(toks)}
        q = {v: self.w.Q[t] for v, t in enumerate(toks)}
        path, nxt = S.verify_tree_stochastic(p, q, tree, rng)
        return [toks[v] for v in path] + [nxt]


# ------------------------------------------------------------------ the law is preserved

@pytest.mark.parametrize("K", MK["chain_lengths"])
@pytest.mark.parametrize("world", [WORLD, TRUNC], ids=["full", "truncated"])
def test_chain_rule_emits_the_target_law(world, K):
    assert world.pvalue(world.histogram(Chain(world, K), 20000)) > OK_P


def test_engine_chain_round_emits_the_target_law():
    assert WORLD.pvalue(WORLD.histogram(Chain(WORLD, max(MK["chain_lengths"]), engine=True), 20000)) > OK_P


@pytest.mark.parametrize("shape", MK["tree_shapes"], ids=lambda s: f"d{s[0]}w{s[1]}")
def test_tree_rule_emits_the_target_law(shape):
    assert WORLD.pvalue(WORLD.histogram(Tree(WORLD, *shape), 12000)) > OK_P


def test_tree_rule_with_a_truncated_draft_vocabulary():
    assert TRUNC.pvalue(TRUNC.histogram(Tree(TRUNC, *MK["truncated_tree_shape"]), 12000)) > OK_P


def test_length_chosen_from_past_tokens_keeps_the_law():
    """A chain length that depends only on what is already committed is fine."""
    rule = MK["past_draw_rule"]

    def propose(prev, rng):
        k = rule["long"] if WORLD.Q[prev].max() > rule["threshold"] else rule["short"]
        return Chain(WORLD, k)(prev, rng)

    assert WORLD.pvalue(WORLD.histogram(propose, 20000)) > OK_P


# ------------------------------------------------------------------ negative controls (must be caught)

def test_control_deterministic_children_are_caught():
    """Top-q children are not draws from q: the rejection correction no longer applies."""
    assert WORLD.pvalue(WORLD.histogram(Tree(WORLD, *MK["topk_control_shape"], children="top"), 20000)) < BAD_P


def test_control_dropping_unlikely_drafts_is_caught():
    """Keeping a draft only when its own q is high makes the proposal depend on the draw."""
    cut = MK["current_draw_control_threshold"]

    def propose(prev, rng):
        x = int(rng.choice(WORLD.V, p=WORLD.Q[prev]))
        if WORLD.Q[prev, x] < cut:
            return [int(rng.choice(WORLD.V, p=WORLD.P[prev]))]
        n, nxt = S.verify_chain_stochastic(WORLD.P[[prev, x]], WORLD.Q[[prev]], [x], rng)
        return [x, nxt][: n + 1]

    assert WORLD.pvalue(WORLD.histogram(propose, 20000)) < BAD_P


def test_control_resampling_from_p_instead_of_the_residual_is_caught():
    """A plausible slip in the rule itself: after a rejection, draw from p rather
    than from norm(max(p - q, 0))."""
    def propose(prev, rng):
        p, q = WORLD.P[prev], WORLD.Q[prev]
        x = int(rng.choice(WORLD.V, p=q))
        return [x] if rng.random() < min(1.0, p[x] / q[x]) else [S.sample(p, rng)]

    assert WORLD.pvalue(WORLD.histogram(propose, 20000)) < BAD_P


# ------------------------------------------------------------------ special cases (closed form)

class Scripted:
    """A uniform source that hands out given values and counts them."""

    def __init__(self, *values):
        self.queue, self.used = list(values), 0

    def random(self, size=None):
        assert size is None
        self.used += 1
        return self.queue.pop(0)


def test_zero_draft_probability_rejects_without_a_uniform():
    p = np.array([[0.1, 0.2, 0.3, 0.4], [0.25] * 4])
    q = np.array([[0.5, 0.5, 0.0, 0.0]])
    src = Scripted(0.0, 0.99)
    # rejected without a draw; then the residual [0, 0, .3, .4] / .7 at u = 0 -> token 2
    assert S.verify_chain_stochastic(p, q, [2], src) == (0, 2) and src.used == 1


def test_identical_distributions_accept_and_residual_falls_back_to_p():
    p = np.array([[0.1, 0.2, 0.3, 0.4]] * 2)
    src = Scripted(0.999999, 0.5)
    assert S.verify_chain_stochastic(p, p[:1].copy(), [3], src) == (1, 2) and src.used == 2
    np.testing.assert_array_equal(S.residual(p[0], p[0]), p[0] / p[0].sum())


def test_inverse_cdf_boundaries():
    p = np.array([0.0, 0.5, 0.0, 0.5])
    assert [S.sample(p, Scripted(u)) for u in (0.0, 0.5, 0.9999999)] == [1, 3, 3]


def test_low_temperature_is_greedy():
    p = S.probs_from_logits(np.array([[2.0, 5.0, 1.0, 4.99]], np.float32), 1e-9)
    assert p.argmax() == 1 and p[0, 1] == 1.0


def test_chain_rule_equals_tree_rule_at_width_one():
    """On a chain the two rules consume the same uniforms in the same order and
    agree on every outcome."""
    r = np.random.default_rng(5)
    for trial in range(300):
        K = int(r.integers(1, 5))
        ps = r.dirichlet(np.full(7, 0.5), size=K + 1)
        qs = r.dirichlet(np.full(7, 0.5), size=K)
        qs[:, r.integers(0, 7)] = 0
        qs /= qs.sum(-1, keepdims=True)
        drafts = [int(r.integers(0, 7)) for _ in range(K)]
        a, b = core.UniformStream(11, trial), core.UniformStream(11, trial)
        chain = S.verify_chain_stochastic(ps, qs, drafts, a)
        tree = S.DraftTree([0] + drafts, list(range(-1, K)), list(range(K + 1)))
        path, nxt = S.verify_tree_stochastic(dict(enumerate(ps)), dict(enumerate(qs)), tree, b)
        assert chain == (len(path), nxt) and a.pos == b.pos


# ------------------------------------------------------------------ known answers

GR = DATA["greedy"]


def test_greedy_known_answers():
    rows = WORLD.P[GR["chain_rows"]]
    top = rows.argmax(axis=1)
    logits = np.log(rows)
    assert S.verify_chain_greedy(logits, [int(top[0]), int(top[1])]) == (2, int(top[2]))
    wrong = int((top[0] + 1) % WORLD.V)
    assert S.verify_chain_greedy(logits, [wrong, int(top[1])]) == (0, int(top[0]))
    tree = S.DraftTree(**GR["tree"])
    assert S.verify_tree_greedy(GR["tree_argmax"], tree) == (GR["tree_path"], GR["tree_next"])


def test_tree_mask_known_answer():
    tree = S.DraftTree(**GR["tree"])
    pre = GR["mask_prefix"]
    m = S.tree_attention_mask(tree, prefix_len=pre)
    assert m.shape == (len(tree), pre + len(tree)) and m[:, :pre].all()
    for row, want in GR["mask_rows"].items():
        assert list(m[int(row), pre:]) == want


def test_warping_known_answers():
    W = DATA["warping"]
    z = np.array([W["logits"]], np.float32)
    p = S.probs_from_logits(z, 1.0, top_k=W["top_k"])
    assert (p[0, W["top_k_zero"]] == 0).all() and abs(p.sum() - 1) < 1e-6
    assert (S.probs_from_logits(z, 1.0, top_p=W["top_p"])[0] > 0).sum() == W["top_p_kept"]
    e = reduce(lambda acc, v: acc + [np.exp(v / W["temperature"])], W["logits"], [])
    np.testing.assert_allclose(S.probs_from_logits(z, W["temperature"])[0], np.array(e) / sum(e), rtol=W["rtol"])
