"""Stochastic chain verification and the temperature softmax on the GPU.

- probabilities: GPU softmax(logits / T) against the oracle's fp32 restatement
  of probs_from_logits (python/woodcock/sampling.py:39-45), rtol 2e-6; top-k /
  top-p warping (sampling.py:41-54, sampling.cpp:9-45): the kept set equal to the
  oracle's and to the reference runtime's outputs, values within fp32 rounding,
  ties at both boundaries;
- decisions: the accept/reject walk, the uniform count and the emitted token
  equal the oracle's engine-level round (verify_tree_stochastic on the chain,
  python/woodcock/spec.py:316-324) fed the same fp32 p and q and the same
  Philox uniforms, round by round, on the full-vocabulary workload (Zipf target,
  16384-row draft vocabulary);
- the law: first emitted token over 10^5 rounds against p row 0 (chi-square),
  and the exact three-token Markov law of the reference's distribution tests
  (tests/test_sampling.py:33-92) with the GPU rule in the loop;
- special cases: a draft outside the draft vocabulary (q = 0, no uniform), p == q
  (every draft accepted, the bonus token from p_K), K = 0, invalid inputs.
"""
import ctypes as C
import itertools

import numpy as np
import pytest
import torch
from scipy.stats import chisquare

from oracle import core
from oracle import sampling as S
from woodcock_amd import _lib
from woodcock_amd.runtime import new_verdict, ptr
from woodcock_amd.sampling import PhiloxStream, probs_from_logits, verify_chain_stochastic, verify_chain_stochastic_dev
from woodcock_amd.synthetic import draw_rows, stochastic_workload

from conftest import load_golden

pytestmark = pytest.mark.gpu

K, V, H = 5, 151936, 16384
SEED = 1234


@pytest.fixture(scope="module")
def workload(cuda):
    lg, dl, d2t = stochastic_workload(K, V, H, seed=3)
    dev = torch.device("cuda", 0)
    tl, dlg, d2 = torch.from_numpy(lg).to(dev), torch.from_numpy(dl).to(dev), torch.from_numpy(d2t).to(dev)
    p = probs_from_logits(tl, 1.0)
    q = probs_from_logits(dlg, 1.0)
    torch.cuda.synchronize()
    return lg, dl, d2t, tl, dlg, d2, p, q


@pytest.mark.parametrize("temperature", [1.0, 0.7, 1e-7])
def test_probs_match_oracle(workload, temperature):
    lg, dl, _, tl, dlg, _, _, _ = workload
    for host, dev in ((lg, tl), (dl, dlg)):
        got = probs_from_logits(dev, temperature).cpu().numpy()
        want = S.probs_from_logits(host, temperature)
        np.testing.assert_allclose(got, want, rtol=2e-6, atol=1e-12)
        np.testing.assert_allclose(got.sum(-1), 1.0, rtol=1e-5)


@pytest.mark.parametrize("temperature,top_k,top_p", [(1.0, 40, 1.0), (0.7, 0, 0.9), (1.0, 50, 0.8), (0.5, 2000, 0.95),
                                                     (1.0, 1, 1.0), (1.0, 0, 1e-3)])
def test_warped_probs_match_oracle(workload, temperature, top_k, top_p):
    """Top-k / top-p on the full target rows [6, 151936] and the draft rows
    [5, 16384]: the kept set equals the oracle's exactly, the values within fp32
    rounding (fp64 kept mass against numpy's fp32 sum)."""
    from woodcock_amd.sampling import SamplingParams

    lg, dl, _, tl, dlg, _, _, _ = workload
    sp = SamplingParams(temperature=temperature, top_k=top_k, top_p=top_p)
    for host, dev in ((lg, tl), (dl, dlg)):
        got = probs_from_logits(dev, sp).cpu().numpy()
        want = S.probs_from_logits(host, temperature, top_k, top_p)
        np.testing.assert_array_equal(got > 0, want > 0)
        np.testing.assert_allclose(got, want, rtol=4e-6, atol=1e-12)
        np.testing.assert_allclose(got.sum(-1), 1.0, rtol=1e-5)


def test_warped_probs_match_reference_cpp(cuda):
    """The reference's own probs_from_logits outputs (sampling.cpp:9-45) for
    temperature, top-k and top-p cases (tests/golden/verify.npz)."""
    from woodcock_amd.sampling import SamplingParams

    z = load_golden("verify.npz")
    for c in range(5):
        T, k, p = z[f"p{c}.args"].tolist()
        x = torch.from_numpy(z[f"p{c}.z"][None]).to(cuda)
        got = probs_from_logits(x, SamplingParams(temperature=T, top_k=int(k), top_p=p)).cpu().numpy()[0]
        np.testing.assert_array_equal(got > 0, z[f"p{c}.p"] > 0)
        np.testing.assert_allclose(got, z[f"p{c}.p"], rtol=4e-6, atol=1e-9)


def test_warping_ties_and_edges(cuda):
    """Ties at the top-k boundary all stay (x < the k-th largest drops out); at
    the top-p boundary equal values stay lowest index first (four-way, ten-way
    and thousand-way ties); top_p = 0 is rejected."""
    from woodcock_amd.sampling import SamplingParams

    rows = np.full((4, 3000), -2.0, np.float32)
    rows[0, [7, 100, 2999, 5]] = 3.0            # four-way tie for the top
    rows[1, :10] = 0.0                          # ten equal leaders
    rows[1, 10:] = -30.0
    rows[2, ::3] = 1.0                          # a thousand equal entries
    rows[3] = np.linspace(-1, 1, 3000, dtype=np.float32)
    x = torch.from_numpy(rows).to(cuda)
    for sp in (SamplingParams(1.0, top_k=2), SamplingParams(1.0, top_k=4), SamplingParams(1.0, top_p=0.35),
               SamplingParams(0.3, top_k=1000, top_p=0.3005), SamplingParams(1.0, top_p=1.0)):
        got = probs_from_logits(x, sp).cpu().numpy()
        want = S.probs_from_logits(rows, sp.temperature, sp.top_k, sp.top_p)
        np.testing.assert_array_equal(got > 0, want > 0)
        np.testing.assert_allclose(got, want, rtol=4e-6, atol=1e-12)
    got = probs_from_logits(x[:1], SamplingParams(1.0, top_k=2)).cpu().numpy()[0]
    assert sorted(np.flatnonzero(got).tolist()) == [5, 7, 100, 2999]
    got = probs_from_logits(x[1:2], SamplingParams(1.0, top_p=0.35)).cpu().numpy()[0]
    assert np.flatnonzero(got).tolist() == [0, 1, 2, 3]  # ceil(0.35 / 0.1) of the ten, lowest index first
    with pytest.raises(ValueError):
        probs_from_logits(x, SamplingParams(1.0, top_p=0.0))


def test_probs_small_width_and_stride(cuda):
    dev = torch.device("cuda", 0)
    x = torch.randn(3, 40, device=dev) * 4
    out = torch.full((3, 40), -1.0, device=dev)
    probs_from_logits(x[:, :37], 1.3, out=out[:, :37])
    want = S.probs_from_logits(x[:, :37].cpu().numpy(), 1.3)
    np.testing.assert_allclose(out[:, :37].cpu().numpy(), want, rtol=2e-6, atol=1e-12)
    assert (out[:, 37:] == -1).all()


def _oracle_round(p_np, q_np, d2t, drafts, rnd):
    st = core.UniformStream(SEED, rnd)
    n, nxt = S.chain_stochastic_round(p_np, q_np, d2t, list(drafts), st)
    return n, nxt, st.pos


@pytest.mark.parametrize("path", ["probs", "logits"])
def test_rounds_equal_oracle(workload, path):
    """Round by round, (n, next, uniforms consumed) of the two-launch rule on p
    ("probs") and of the one-launch rule straight from the target logits
    ("logits", p formed in place by the same arithmetic as the GPU softmax)
    equal the oracle's engine-level round fed that softmax's fp32 p."""
    from woodcock_amd.sampling import verify_chain_stochastic_logits_dev

    lg, dl, d2t, tl, dlg, d2, p, q = workload
    dev = p.device
    p_np, q_np = p.cpu().numpy(), q.cpu().numpy()
    rng = np.random.default_rng(7)
    rows = draw_rows(q_np, 150, rng)
    drafts = d2t[rows]
    # a few rounds with drafts outside the draft vocabulary (q = 0: rejected, no uniform)
    outside = np.setdiff1d(np.arange(V), d2t)
    drafts[::17, 1] = outside[rng.integers(0, len(outside), size=len(drafts[::17]))]
    rounds = torch.arange(len(drafts), dtype=torch.int32, device=dev)
    dd = torch.from_numpy(drafts).to(dev)
    verd = torch.zeros(len(drafts), _lib.VERDICT_INTS, dtype=torch.int32, device=dev)
    for r in range(len(drafts)):
        u = _lib.Uniforms(SEED, ptr(rounds[r:r + 1]), 0)
        if path == "probs":
            verify_chain_stochastic_dev(p, q, dd[r], u, d2, verdict=verd[r])
        else:
            verify_chain_stochastic_logits_dev(tl, 1.0, q, dd[r], u, d2, verdict=verd[r])
    verd = verd.cpu().numpy()
    assert (verd[:, _lib.V_STATUS] == 0).all()
    seen = set()
    for r in range(len(drafts)):
        n, nxt, nu = _oracle_round(p_np, q_np, d2t, drafts[r], r)
        got = (int(verd[r, _lib.V_N_ACCEPTED]), int(verd[r, _lib.V_NEXT]), int(verd[r, _lib.V_N_UNIFORMS]))
        assert got == (n, nxt, nu), (r, drafts[r], got, (n, nxt, nu))
        toks = verd[r, _lib.V_TOKENS:_lib.V_TOKENS + n + 1].tolist()
        assert toks == list(drafts[r][:n]) + [nxt]
        assert verd[r, _lib.V_KEEP:_lib.V_KEEP + n + 1].tolist() == list(range(n + 1))
        seen.add(n)
    assert len(seen) >= 3, seen  # rejections at several depths are exercised


@pytest.mark.parametrize("path", ["probs", "logits"])
def test_first_token_law_1e5_rounds(workload, path):
    """The first emitted token is distributed as p row 0 (the defining property
    of speculative sampling), over 10^5 rounds of the full-size rule: the
    two-launch rule on p and the one-launch rule from the target logits."""
    from woodcock_amd.sampling import verify_chain_stochastic_logits_dev

    lg, dl, d2t, tl, dlg, d2, p, q = workload
    dev = p.device
    R = 100_000
    q_np = q.cpu().numpy()
    rows = draw_rows(q_np, R, np.random.default_rng(11))
    dd = torch.from_numpy(d2t[rows]).to(dev)
    rounds = torch.arange(R, dtype=torch.int32, device=dev)
    verd = torch.zeros(R, _lib.VERDICT_INTS, dtype=torch.int32, device=dev)
    rr = torch.from_numpy(rows).to(dev)
    for r in range(R):
        u = _lib.Uniforms(SEED + 1, ptr(rounds[r:r + 1]), 0)
        if path == "probs":
            verify_chain_stochastic_dev(p, q, dd[r], u, d2, draft_rows=rr[r], verdict=verd[r])
        else:
            verify_chain_stochastic_logits_dev(tl, 1.0, q, dd[r], u, d2, draft_rows=rr[r], verdict=verd[r])
    v = verd.cpu().numpy()
    assert (v[:, _lib.V_STATUS] == 0).all()
    first = v[:, _lib.V_TOKENS]
    p0 = p[0].double().cpu().numpy()
    top = np.argsort(-p0)[:60]
    counts = np.array([(first == t).sum() for t in top] + [(~np.isin(first, top)).sum()], np.float64)
    exp = np.concatenate([p0[top], [1.0 - p0[top].sum()]]) * R
    assert chisquare(counts, exp * counts.sum() / exp.sum()).pvalue > 1e-3
    # the accepted-length histogram is non-trivial
    assert len(np.unique(v[:, _lib.V_N_ACCEPTED])) >= 4


# ------------------------------------------------------------------ exact Markov law (tests/test_sampling.py:33-92)

MV, N_EMIT = 5, 3


def _markov(seed, sharp):
    return np.random.default_rng(seed).dirichlet(np.full(MV, sharp), size=MV)


MP = _markov(1, 0.7)
MQ = 0.5 * _markov(2, 0.7) + 0.5 * MP


def test_markov_exact_law_with_gpu_rule(cuda):
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(0)
    Kc = 3
    trials = 6000
    counts = np.zeros(MV ** N_EMIT)
    stream = PhiloxStream(seed=77)
    Pt = torch.from_numpy(MP.astype(np.float32)).to(dev)
    Qt = torch.from_numpy(MQ.astype(np.float32)).to(dev)
    for _ in range(trials):
        out = []
        while len(out) < N_EMIT:
            prev = out[-1] if out else 0
            toks, cur = [], prev
            for _ in range(Kc):
                x = int(rng.choice(MV, p=MQ[cur]))
                toks.append(x)
                cur = x
            ctx = [prev] + toks
            p = Pt[ctx]
            q = Qt[ctx[:-1]]
            n, nxt = verify_chain_stochastic(p, q, toks, stream)
            out.extend(toks[:n] + [nxt])
        counts[np.ravel_multi_index(tuple(out[:N_EMIT]), (MV,) * N_EMIT)] += 1
    law = np.zeros((MV,) * N_EMIT)
    for seq in itertools.product(range(MV), repeat=N_EMIT):
        pr, prev = 1.0, 0
        for t in seq:
            pr *= MP[prev, t]
            prev = t
        law[seq] = pr
    exp = law.ravel() * counts.sum()
    keep = exp > 0
    assert chisquare(counts[keep], exp[keep] * counts[keep].sum() / exp[keep].sum()).pvalue > 1e-3


# ------------------------------------------------------------------ special cases

def test_equal_distributions_accept_all_and_sample_bonus(cuda):
    dev = torch.device("cuda", 0)
    p = torch.softmax(torch.randn(4, 300, device=dev), -1)
    q = p[:3].clone()
    drafts = [int(torch.argmax(p[i])) for i in range(3)]
    for r in range(20):
        st = PhiloxStream(seed=5, round=r)
        n, nxt = verify_chain_stochastic(p, q, drafts, st)
        ost = core.UniformStream(5, r)
        want = S.chain_stochastic_round(p.cpu().numpy(), q.cpu().numpy(), None, drafts, ost)
        assert (n, nxt) == want and n == 3


def test_no_drafts_samples_p0(cuda):
    dev = torch.device("cuda", 0)
    p = torch.softmax(torch.randn(1, 1000, device=dev) * 2, -1)
    for r in range(10):
        n, nxt = verify_chain_stochastic(p, torch.empty(0, 1, device=dev), [], PhiloxStream(seed=9, round=r))
        want = S.sample(p[0].cpu().numpy().astype(np.float64), core.UniformStream(9, r))
        assert (n, nxt) == (0, want)


def test_invalid_inputs_raise(cuda):
    dev = torch.device("cuda", 0)
    p = torch.softmax(torch.randn(3, 100, device=dev), -1)
    q = torch.softmax(torch.randn(2, 10, device=dev), -1)
    bad_d2t = torch.tensor([5, 3, 7, 9, 11, 12, 13, 14, 15, 16], dtype=torch.int32, device=dev)
    with pytest.raises(ValueError):
        verify_chain_stochastic(p, q, [5, 7], PhiloxStream(seed=1), d2t=bad_d2t)
    ok_d2t = torch.arange(10, dtype=torch.int32, device=dev) * 3
    with pytest.raises(ValueError):
        verify_chain_stochastic(p, q, [5, 100], PhiloxStream(seed=1), d2t=ok_d2t)
    with pytest.raises(ValueError):
        verify_chain_stochastic(p, q, [5], PhiloxStream(seed=1), d2t=ok_d2t)


@pytest.mark.parametrize("temperature", [1.0, 0.7, 0.5])
def test_logits_path_equals_two_call_path(workload, temperature):
    """wc_verify_chain_stochastic_logits (p formed in place from the logits)
    returns the verdict of wc_probs_from_logits + wc_verify_chain_stochastic,
    every field, over rounds with rejections at every depth and drafts outside
    the draft vocabulary."""
    from woodcock_amd.sampling import verify_chain_stochastic_logits_dev

    lg, dl, d2t, tl, dlg, d2, _, q = workload
    dev = tl.device
    p = probs_from_logits(tl, temperature)
    rng = np.random.default_rng(17)
    rows = draw_rows(q.cpu().numpy(), 120, rng)
    drafts = d2t[rows]
    outside = np.setdiff1d(np.arange(V), d2t)
    drafts[::13, 2] = outside[rng.integers(0, len(outside), size=len(drafts[::13]))]
    dd = torch.from_numpy(drafts).to(dev)
    drows = torch.from_numpy(rows.astype(np.int32)).to(dev)
    rounds = torch.arange(len(drafts), dtype=torch.int32, device=dev)
    v2 = torch.zeros(len(drafts), _lib.VERDICT_INTS, dtype=torch.int32, device=dev)
    v1 = torch.zeros_like(v2)
    for r in range(len(drafts)):
        u = _lib.Uniforms(SEED, ptr(rounds[r:r + 1]), 0)
        verify_chain_stochastic_dev(p, q, dd[r], u, d2, verdict=v2[r])
        verify_chain_stochastic_logits_dev(tl, temperature, q, dd[r], u, d2, verdict=v1[r])
        # with the drafts' head rows given (draft time knows them)
        if r % 3 == 0:
            v3 = torch.zeros_like(v1[r])
            verify_chain_stochastic_logits_dev(tl, temperature, q, dd[r], u, d2, draft_rows=drows[r], verdict=v3)
            assert torch.equal(v3, v1[r]), r
    assert torch.equal(v1, v2)
    # T = 0.5 sharpens p away from q (drawn at T = 1): rejections come early
    assert len(set(v1[:, _lib.V_N_ACCEPTED].tolist())) >= (2 if temperature < 0.6 else 3)


def test_logits_path_no_drafts_and_identity_vocab(cuda):
    """K = 0 draws from softmax(logits_0); without d2t the head rows are the
    first ids of the vocabulary."""
    from woodcock_amd.sampling import verify_chain_stochastic_logits_dev

    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(5)
    lg = torch.randn(4, 9000, generator=g, device=dev) * 3
    q = probs_from_logits(torch.randn(3, 5000, generator=g, device=dev), 1.0)
    rounds = torch.arange(40, dtype=torch.int32, device=dev)
    for r in range(40):
        u = _lib.Uniforms(SEED, ptr(rounds[r:r + 1]), 0)
        d = torch.randint(0, 5000, (3,), generator=g, device=dev, dtype=torch.int32)
        a = verify_chain_stochastic_dev(probs_from_logits(lg, 1.0), q, d, u)
        b = verify_chain_stochastic_logits_dev(lg, 1.0, q, d, u)
        assert torch.equal(a, b), r
        a0 = verify_chain_stochastic_dev(probs_from_logits(lg[:1], 1.0), None, d[:0], u)
        b0 = verify_chain_stochastic_logits_dev(lg[:1], 1.0, None, d[:0], u)
        assert torch.equal(a0, b0), r


def test_logits_path_long_chain_and_invalid_inputs(cuda):
    """K = 9 (beyond the rows a one-launch call holds: the two-launch path)
    equals the two-call path; an invalid d2t or draft sets status WC_E_INVALID
    for that call only, on both paths."""
    from woodcock_amd.sampling import verify_chain_stochastic_logits_dev

    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(11)
    Vs, Hs = 20000, 3000
    d2t = torch.sort(torch.randperm(Vs, generator=g, device=dev)[:Hs])[0].to(torch.int32)
    rounds = torch.arange(30, dtype=torch.int32, device=dev)
    for k in (4, 9):
        lg = torch.randn(k + 1, Vs, generator=g, device=dev) * 2
        q = probs_from_logits(torch.randn(k, Hs, generator=g, device=dev), 1.0)
        p = probs_from_logits(lg, 0.8)
        seen = set()
        for r in range(30):
            u = _lib.Uniforms(SEED, ptr(rounds[r:r + 1]), 0)
            rows = torch.randint(0, Hs, (k,), generator=g, device=dev)
            d = d2t[rows].contiguous()
            if r % 4 == 0:  # shared drafts: the first accepted more often
                d = d2t[torch.argmax(q, dim=1)].to(torch.int32).contiguous()
            a = verify_chain_stochastic_dev(p, q, d, u, d2t)
            b = verify_chain_stochastic_logits_dev(lg, 0.8, q, d, u, d2t)
            assert torch.equal(a, b), (k, r)
            assert int(b[_lib.V_STATUS]) == 0
            seen.add(int(b[_lib.V_N_ACCEPTED]))
        assert len(seen) >= 2, k
        u = _lib.Uniforms(SEED, ptr(rounds[:1]), 0)
        bad_d2t = d2t.clone()
        bad_d2t[7] = bad_d2t[6]
        d = d2t[:k].contiguous()
        v = verify_chain_stochastic_logits_dev(lg, 0.8, q, d, u, bad_d2t)
        assert int(v[_lib.V_STATUS]) == _lib.WC_E_INVALID, k
        v = verify_chain_stochastic_logits_dev(lg, 0.8, q, d, u, d2t)
        assert int(v[_lib.V_STATUS]) == 0, k
        d_out = d.clone()
        d_out[k - 1] = Vs
        v = verify_chain_stochastic_logits_dev(lg, 0.8, q, d_out, u, d2t)
        assert int(v[_lib.V_STATUS]) == _lib.WC_E_INVALID, k
        v = verify_chain_stochastic_logits_dev(lg, 0.8, q, d, u, d2t)
        assert int(v[_lib.V_STATUS]) == 0, k


def test_one_launch_give_up_is_sticky_until_reinit(workload):
    """The one-launch rule's bounded waits, forced to give up from the host
    (spin limit 0: a waiting block stops at its first unsuccessful poll, so
    every kernel ends): the call reports WC_E_HIP; every following call on that
    workspace fails fast -- status WC_E_HIP, no other verdict field written, no
    word of the failed call read -- until wc_workspace_init, after which the
    calls equal the two-launch path again.  A call that did not give up is
    exact."""
    from woodcock_amd.runtime import reset_workspace

    lg, dl, d2t, tl, dlg, d2, p, q = workload
    dev = p.device
    L = _lib.lib()
    n = int(L.wc_workspace_bytes())
    ws = torch.empty((n + 255) // 256 * 256, dtype=torch.uint8, device=dev)
    reset_workspace(ws)
    rows = draw_rows(q.cpu().numpy(), 8, np.random.default_rng(23))
    dd = torch.from_numpy(d2t[rows]).to(dev)
    rounds = torch.arange(8, dtype=torch.int32, device=dev)
    ref = torch.zeros(8, _lib.VERDICT_INTS, dtype=torch.int32, device=dev)
    for r in range(8):
        verify_chain_stochastic_dev(p, q, dd[r], _lib.Uniforms(SEED, ptr(rounds[r:r + 1]), 0), d2, verdict=ref[r])

    def call(r):
        v = torch.zeros(_lib.VERDICT_INTS, dtype=torch.int32, device=dev)
        u = _lib.Uniforms(SEED, ptr(rounds[r:r + 1]), 0)
        _lib.call("wc_verify_chain_stochastic_logits", ptr(tl), K + 1, V, tl.stride(0), 1.0, ptr(q), H, q.stride(0),
                  ptr(d2), ptr(dd[r]), None, C.byref(u), ptr(v), ptr(ws), None)
        torch.cuda.synchronize()
        return v

    gave_up = False
    L.wc_set_spin_limit(0)
    try:
        for attempt in range(8):
            v = call(attempt)
            if int(v[_lib.V_STATUS]) == _lib.WC_E_HIP:
                gave_up = True
                break
            assert torch.equal(v, ref[attempt]), attempt
    finally:
        L.wc_set_spin_limit(-1)
    assert gave_up
    for r in range(3):  # sticky: fails fast without writing anything else
        v = call(r)
        assert int(v[_lib.V_STATUS]) == _lib.WC_E_HIP
        v[_lib.V_STATUS] = 0
        assert not v.any()
    reset_workspace(ws)
    for r in range(8):
        assert torch.equal(call(r), ref[r]), r
