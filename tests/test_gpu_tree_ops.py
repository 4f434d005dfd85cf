"""Tree helpers and the stochastic tree rule on the GPU, against the oracle.

- wc_tree_mask: byte-exact against the oracle's tree_attention_mask
  (python/woodcock/sampling.py:118-128, pinned by the known answers of
  tests/test_sampling.py:185-216) on random trees, chains and prefixes 0..2048;
- wc_sample_without_replacement: the same tokens, in the same order, and the
  same uniform consumption as the oracle's sample_without_replacement
  (sampling.py:196-203) fed the same Philox stream, rows drawn one after another
  as tree drafting does (spec.py:238-249);
- wc_verify_tree_stochastic: path, next token and uniform count equal the
  oracle's verify_tree_stochastic (sampling.py:143-177) on the full-vocabulary
  workload (Zipf targets, 16384-row draft vocabulary, children drawn without
  replacement from q, some tokens outside the draft vocabulary), round by round;
  a chain equals wc_verify_chain_stochastic; the first emitted token follows
  p(root) over 2*10^4 freshly drawn trees (chi-square); a one-node tree samples
  p[0]; invalid trees raise;
- wc_verify_tree_stochastic_indexed (the verify after sampled tree drafting):
  node v's q at row q_rows[v] of a larger store and the node count read from
  the device, padding rows after it -- the same outcomes as the oracle; a q
  row outside the store or a count outside 1..rows is reported.
Decisions are fp64; sums run in a different order than numpy's, so a decision
could differ only when a uniform falls within rounding of its threshold.
"""
import ctypes as C

import numpy as np
import pytest
import torch
from scipy.stats import chisquare

from oracle import core
from oracle import sampling as S
from woodcock_amd import _lib
from woodcock_amd.runtime import new_verdict, ptr, stream_ptr, workspace
from woodcock_amd.sampling import (DraftTree, PhiloxStream, probs_from_logits, sample_without_replacement_dev,
                                   tree_attention_mask_dev, verify_chain_stochastic, verify_tree_stochastic,
                                   verify_tree_stochastic_dev)
from woodcock_amd.synthetic import stochastic_workload

pytestmark = pytest.mark.gpu

V, H = 151936, 16384
SEED = 4321


def random_parents(n, rng, width=4, depth=6):
    parents, dep, kids = [-1], [0], [0]
    while len(parents) < n:
        cand = [v for v in range(len(parents)) if dep[v] < depth and kids[v] < width]
        v = int(rng.choice(cand))
        parents.append(v)
        dep.append(dep[v] + 1)
        kids.append(0)
        kids[v] += 1
    return parents, dep


# ------------------------------------------------------------------ tree mask

@pytest.mark.parametrize("n,prefix", [(1, 0), (7, 5), (33, 300), (60, 2048), (64, 17)])
def test_tree_mask_matches_oracle(cuda, n, prefix):
    rng = np.random.default_rng(n * 31 + prefix)
    dev = torch.device("cuda", 0)
    for trial in range(3):
        parents, dep = random_parents(n, rng) if trial else (list(range(-1, n - 1)), list(range(n)))
        tree = S.DraftTree([0] * n, parents, dep)
        want = S.tree_attention_mask(tree, prefix).astype(np.uint8)
        out = torch.full((n, prefix + n + 9), 7, dtype=torch.uint8, device=dev)
        tree_attention_mask_dev(torch.tensor(parents, dtype=torch.int32, device=dev), prefix, out[:, : prefix + n])
        got = out.cpu().numpy()
        np.testing.assert_array_equal(got[:, : prefix + n], want)
        assert (got[:, prefix + n:] == 7).all()


# ------------------------------------------------------------------ Gumbel-top-k

@pytest.fixture(scope="module")
def workload(cuda):
    lg, dl, d2t = stochastic_workload(24, V, H, seed=5)
    dev = torch.device("cuda", 0)
    p = probs_from_logits(torch.from_numpy(lg).to(dev), 1.0)
    q = probs_from_logits(torch.from_numpy(dl).to(dev), 1.0)
    torch.cuda.synchronize()
    return p, q, torch.from_numpy(d2t).to(dev), p.cpu().numpy(), q.cpu().numpy(), d2t


def test_sample_without_replacement_matches_oracle(workload):
    p, q, d2, p_np, q_np, d2t = workload
    dev = q.device
    qz = q[:4].clone()
    qz[1, ::3] = 0.0  # zero entries consume no uniform
    qz[2, 100:] = 0.0  # only 100 candidates
    q_host = qz.cpu().numpy()
    k = torch.tensor([4, 3, 16, 1], dtype=torch.int32)
    for rnd, base in ((0, 0), (3, 17), (11, 100_000)):
        st = PhiloxStream(seed=SEED, round=rnd, purpose=2)
        toks, counts = sample_without_replacement_dev(qz, k, st.struct(st.device_round(dev)), d2, uniform_base=base)
        toks, counts = toks.cpu().numpy(), counts.cpu().numpy()
        ost = core.UniformStream(SEED, rnd, 2, start=base)
        for r in range(4):
            want = S.sample_without_replacement(S.scatter_draft_dist(q_host[r], d2t, V), int(k[r]), ost)
            assert counts[r] == len(want)
            assert toks[r, : counts[r]].tolist() == want, (rnd, r)


def test_sample_without_replacement_identity_vocab(cuda):
    dev = torch.device("cuda", 0)
    q = torch.softmax(torch.randn(2, 37, device=dev), -1)
    q[0, 5] = 0.0
    st = PhiloxStream(seed=3, round=9)
    toks, counts = sample_without_replacement_dev(q, 5, st.struct(st.device_round(dev)))
    ost = core.UniformStream(3, 9)
    qn = q.cpu().numpy()
    for r in range(2):
        want = S.sample_without_replacement(S.scatter_draft_dist(qn[r], None, 37), 5, ost)
        assert toks[r].tolist() == want


# ------------------------------------------------------------------ stochastic tree rule

def build_tree(n, q_np, d2t, rng, width=3, depth=5, outside_every=0):
    """Children drawn without replacement from the parent's q (as tree drafting
    does); node v's draft distribution is q row v."""
    tokens, parents, dep = [int(rng.integers(V))], [-1], [0]
    frontier = [0]
    outside = np.setdiff1d(np.arange(2000), d2t)
    while frontier and len(tokens) < n:
        v = frontier.pop(0)
        if dep[v] >= depth:
            continue
        m = min(int(rng.integers(1, width + 1)), n - len(tokens))
        kids = S.sample_without_replacement(S.scatter_draft_dist(q_np[v], d2t, V), m, rng)
        for x in kids:
            if outside_every and rng.integers(outside_every) == 0:
                x = int(outside[rng.integers(len(outside))])
            tokens.append(int(x))
            parents.append(v)
            dep.append(dep[v] + 1)
            frontier.append(len(tokens) - 1)
    return S.DraftTree(tokens, parents, dep)


def oracle_tree(p_np, q_np, d2t, tree, rnd):
    st = core.UniformStream(SEED, rnd)
    p = {v: p_np[v].astype(np.float64) for v in range(len(tree))}
    q = {v: S.scatter_draft_dist(q_np[v], d2t, V) for v in range(len(tree)) if tree.children[v]}
    path, nxt = S.verify_tree_stochastic(p, q, tree, st)
    return path, nxt, st.pos


def test_tree_rounds_equal_oracle(workload):
    p, q, d2, p_np, q_np, d2t = workload
    dev = p.device
    rng = np.random.default_rng(17)
    depths = set()
    for r in range(40):
        n = int(rng.integers(2, 24))
        tree = build_tree(n, q_np, d2t, rng, outside_every=9 if r % 3 == 0 else 0)
        N = len(tree)
        rd = torch.tensor([r], dtype=torch.int32, device=dev)
        verd = verify_tree_stochastic_dev(p[:N], q[:N], torch.tensor(tree.tokens, dtype=torch.int32, device=dev),
                                          torch.tensor(tree.parents, dtype=torch.int32, device=dev),
                                          _lib.Uniforms(SEED, ptr(rd), 0), d2)
        v = verd.cpu().numpy()
        path, nxt, nu = oracle_tree(p_np, q_np, d2t, tree, r)
        a = int(v[_lib.V_N_ACCEPTED])
        got_path = v[_lib.V_KEEP + 1:_lib.V_KEEP + 1 + a].tolist()
        assert v[_lib.V_STATUS] == 0
        assert (got_path, int(v[_lib.V_NEXT]), int(v[_lib.V_N_UNIFORMS])) == (path, nxt, nu), r
        assert v[_lib.V_TOKENS:_lib.V_TOKENS + a + 1].tolist() == [tree.tokens[u] for u in path] + [nxt]
        assert v[_lib.V_KEEP] == 0 and int(v[_lib.V_N_KEEP]) == a + 1
        depths.add(a)
    assert len(depths) >= 3, depths


def test_chain_tree_equals_chain_kernel(workload):
    p, q, d2, p_np, q_np, d2t = workload
    rng = np.random.default_rng(2)
    K = 5
    for r in range(15):
        drafts = [int(d2t[rng.integers(H)]) for _ in range(K)]
        if r % 4 == 0:
            drafts[1] = int(np.argmax(p_np[1]))
        tree = DraftTree([0] + drafts, list(range(-1, K)), list(range(K + 1)))
        a = verify_tree_stochastic(p[:K + 1], q[:K + 1], tree, PhiloxStream(seed=SEED, round=r), d2)
        n, nxt = verify_chain_stochastic(p[:K + 1], q[:K], drafts, PhiloxStream(seed=SEED, round=r), d2)
        assert (len(a[0]), a[1]) == (n, nxt)
        assert a[0] == list(range(1, n + 1))


def test_first_token_follows_root_target(cuda):
    """Depth-1 trees with 3 children drawn without replacement from q: the first
    emitted token is distributed as p(root) (Jeon et al.'s recursive rejection)."""
    dev = torch.device("cuda", 0)
    Vs = 12
    rng = np.random.default_rng(8)
    p0 = rng.dirichlet(np.full(Vs, 0.8))
    q0 = 0.5 * rng.dirichlet(np.full(Vs, 0.8)) + 0.5 * p0
    trials = 20000
    P = torch.from_numpy(np.tile(p0, (4, 1)).astype(np.float32)).to(dev)
    Q = torch.from_numpy(np.tile(q0, (4, 1)).astype(np.float32)).to(dev)
    par = torch.tensor([-1, 0, 0, 0], dtype=torch.int32, device=dev)
    toks = np.zeros((trials, 4), np.int32)
    for t in range(trials):
        toks[t, 1:] = S.sample_without_replacement(q0, 3, rng)
    tt = torch.from_numpy(toks).to(dev)
    rounds = torch.arange(trials, dtype=torch.int32, device=dev)
    verd = torch.zeros(trials, _lib.VERDICT_INTS, dtype=torch.int32, device=dev)
    for t in range(trials):
        verify_tree_stochastic_dev(P, Q, tt[t], par, _lib.Uniforms(99, ptr(rounds[t:t + 1]), 0), verdict=verd[t])
    v = verd.cpu().numpy()
    assert (v[:, _lib.V_STATUS] == 0).all()
    first = v[:, _lib.V_TOKENS]
    counts = np.bincount(first, minlength=Vs).astype(np.float64)
    p32 = P[0].double().cpu().numpy()
    assert chisquare(counts, p32 / p32.sum() * trials).pvalue > 1e-3
    assert 0 < (v[:, _lib.V_N_ACCEPTED] == 1).mean() < 1


def test_single_node_tree_samples_p0(workload):
    p, q, d2, p_np, q_np, d2t = workload
    for r in range(8):
        path, nxt = verify_tree_stochastic(p[:1], None, DraftTree([5], [-1], [0]), PhiloxStream(seed=1, round=r))
        assert path == [] and nxt == S.sample(p_np[0].astype(np.float64), core.UniformStream(1, r))


def test_invalid_tree_is_reported(workload):
    p, q, d2, *_ = workload
    with pytest.raises(ValueError):
        verify_tree_stochastic(p[:3], q[:3], DraftTree([0, 5, 6], [-1, 2, 0], [0, 1, 1]), PhiloxStream(seed=1), d2)
    with pytest.raises(ValueError):
        verify_tree_stochastic(p[:2], q[:2], DraftTree([0, V + 3], [-1, 0], [0, 1]), PhiloxStream(seed=1), d2)


def _indexed(p, store, q_rows, toks, pars, count, rnd, d2):
    dev = p.device
    i32 = lambda x: torch.tensor(x, dtype=torch.int32, device=dev)
    rd, cnt, verd = i32([rnd]), i32([count]), new_verdict(dev)
    qr, tt, pp = i32(q_rows), i32(toks), i32(pars)
    _lib.call("wc_verify_tree_stochastic_indexed", ptr(p), len(toks), p.shape[1], p.stride(0), ptr(store),
              store.shape[0], ptr(qr), store.shape[1], store.stride(0), ptr(d2), ptr(tt), ptr(pp), ptr(cnt),
              C.byref(_lib.Uniforms(SEED, ptr(rd), 0)), ptr(verd), ptr(workspace(dev)), stream_ptr())
    return verd.cpu().numpy()


def test_indexed_rows_and_device_count_equal_oracle(workload):
    p, q, d2, p_np, q_np, d2t = workload
    dev = p.device
    rng = np.random.default_rng(23)
    store = torch.zeros(40, H, dtype=torch.float32, device=dev)
    depths = set()
    for r in range(40):
        tree = build_tree(int(rng.integers(1, 24)), q_np, d2t, rng, outside_every=9 if r % 4 == 1 else 0)
        N = len(tree)
        rows = min(24, N + int(rng.integers(0, 6)))
        slots = rng.permutation(store.shape[0])[:N]
        store.zero_()
        store[torch.from_numpy(slots).to(dev)] = q[:N]
        pad = rows - N
        v = _indexed(p[:rows], store, slots.tolist() + [0] * pad, tree.tokens + [tree.tokens[0]] * pad,
                     tree.parents + [0] * pad, N, r, d2)
        path, nxt, nu = oracle_tree(p_np, q_np, d2t, tree, r)
        a = int(v[_lib.V_N_ACCEPTED])
        assert v[_lib.V_STATUS] == 0
        got = (v[_lib.V_KEEP + 1:_lib.V_KEEP + 1 + a].tolist(), int(v[_lib.V_NEXT]), int(v[_lib.V_N_UNIFORMS]))
        assert got == (path, nxt, nu), r
        depths.add(a)
    assert len(depths) >= 2, depths


def test_indexed_invalid_rows_and_counts_are_reported(workload):
    p, q, d2, *_ = workload
    store = q[:4].contiguous()
    toks, pars = [5, 6, 7], [-1, 0, 0]
    assert _indexed(p[:3], store, [0, 1, 4], toks, pars, 3, 0, d2)[_lib.V_STATUS] == _lib.WC_E_INVALID
    assert _indexed(p[:3], store, [0, 1, -1], toks, pars, 3, 0, d2)[_lib.V_STATUS] == _lib.WC_E_INVALID
    assert _indexed(p[:3], store, [0, 1, 2], toks, pars, 4, 0, d2)[_lib.V_STATUS] == _lib.WC_E_INVALID
    assert _indexed(p[:3], store, [0, 1, 2], toks, pars, 0, 0, d2)[_lib.V_STATUS] == _lib.WC_E_INVALID
    # the rows past the count are never looked at, however invalid
    v = _indexed(p[:3], store, [0, 3, 99], toks, [-1, 0, 7], 2, 0, d2)
    assert v[_lib.V_STATUS] == 0
