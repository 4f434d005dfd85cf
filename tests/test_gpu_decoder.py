"""The round loop (woodcock_amd.spec.SpeculativeDecoder; python/woodcock/spec.py:151-212)
against oracle loops built from the CPU restatements.

* Auto chain length (CostAwareChain, policies.py:78-123) at the Qwen3-4B drafter
  shape (hidden 2560, 32 / 8 heads, SwiGLU 9728, 16k trimmed head, drafter
  context 4096, bf16 KV) against a synthetic target whose draft positions agree
  with probability 0.68 each: over 24 rounds the chosen chain lengths, drafts,
  accepted counts and tokens equal an oracle loop that runs the same policy
  class on its own accepted counts; the drafter's root and cache rows stay
  within the bf16-cache tolerance.  The same rounds replayed from one captured
  graph per chain length give the same results.
* Greedy tree rounds (spec.py:187-201, 216-329) at the Qwen3-1.7B drafter shape
  (depth 6, width 4, 60 verified rows, context 2048) with a two-layer
  full-width Qwen3-1.7B target forward: the drafted tree, the accepted path
  (planted along a non-contiguous branch), the compacted target KV, and the
  drafter update from the taps at the kept rows, against the oracle's tree
  drafting, target stack, tree walk and compaction on identical inputs.
* Sampled rounds at T > 0 (spec.py:187-201 with the stochastic branches
  238-249 and 320-324) at the same shapes: the drawn tree equals the oracle's
  sampled drafting on the same Philox stream, the target logits and the
  warped target distribution (temperature, top-k) match the oracle's, the
  recursive rejection's path, next token and uniform count equal the oracle
  rule fed the GPU's p and q rows, and the compaction and drafter update follow
  the accepted branch.  Through the loop, chains (a width-1 tree) and trees
  advance every count by the accepted path + 1.
"""
import numpy as np
import pytest
import torch

from oracle import core
from oracle import sampling as S
from oracle import tree_draft as otd
from oracle.target import TargetStack

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


# synthetic latencies (ms): the chosen length moves with the acceptance estimate
COSTS = dict(step_ms=0.1, head_ms=0.03, verify_ms={n: 2.0 + 0.25 * n for n in range(1, 10)})


def _drafter(cuda, cfg, head_rows, seed, kv_dtype=torch.bfloat16):
    from woodcock_amd.config import QWEN3_EOS
    from woodcock_amd.drafter import Drafter
    from woodcock_amd.synthetic import draft_vocab, random_drafter, to_bits

    w = random_drafter(cfg, seed=seed, device=cuda)
    d = Drafter(cfg, w, cuda, kv_dtype)
    ids = draft_vocab(cfg.vocab_size, head_rows, seed=seed, always=QWEN3_EOS)
    d.restrict_vocab(ids)
    bits = {k: to_bits(v) for k, v in d.w.items()}
    bits["lm_head.weight"] = to_bits(d._head)
    od = core.Drafter(cfg.as_dict(), bits)
    od.d2t = ids
    return d, od


def _fill_cache(cuda, caches, ocache, ctx, seed):
    from woodcock_amd.synthetic import to_bits

    g = torch.Generator(device=cuda).manual_seed(seed)
    for i, c in enumerate(caches):
        c.keys[0, :, :ctx] = torch.randn(c.keys[0, :, :ctx].shape, generator=g, device=cuda).bfloat16()
        c.values[0, :, :ctx] = torch.randn(c.values[0, :, :ctx].shape, generator=g, device=cuda).bfloat16()
        ocache.k[i][:] = to_bits(c.keys[0])
        ocache.v[i][:] = to_bits(c.values[0])
    ocache.offset = ctx


def _oracle_chain(od, oc, root_hid, k, logits, taps, gpu_drafts):
    """One fused chain round (spec.py:331-374) on the oracle; where the oracle's
    top-2 margin is below 1e-4 the GPU's (equally valid) choice is followed."""
    eps = od.cfg["rms_norm_eps"]
    out = core.rmsnorm(root_hid, od.w["norm.weight"], eps)
    fb = od.feedback(root_hid, out)
    base = oc.offset
    drafts = []
    for i in range(k):
        z = od.logits(out)[0]
        row = core.argmax(z)
        srt = np.sort(z)
        tok = int(od.d2t[row])
        if tok != gpu_drafts[i]:
            assert srt[-1] - srt[-2] < 1e-4, f"draft {i}: oracle {tok} vs GPU {gpu_drafts[i]}"
            tok = gpu_drafts[i]
        drafts.append(tok)
        if i < k - 1:
            hid, out = od.forward([tok], fb, oc)
            fb = od.feedback(hid, out)
    oc.offset = base
    a, nxt = S.verify_chain_greedy(logits, drafts)
    acc = drafts[:a] + [nxt]
    hid, _ = od.forward(acc, od.fuse([t[: a + 1] for t in taps]), oc)
    return drafts, a, acc, hid[-1:]


@pytest.mark.parametrize("use_graphs", [False, True])
def test_cost_aware_chain_rounds_qwen3_4b(cuda, use_graphs):
    from woodcock_amd.config import qwen3_4b_drafter
    from woodcock_amd.policies import CostAwareChain
    from woodcock_amd.spec import SpeculativeDecoder
    from woodcock_amd.synthetic import SyntheticTarget

    cfg = qwen3_4b_drafter()
    ctx, k_max, rounds = 4096, 8, 24
    d, od = _drafter(cuda, cfg, 16384, seed=41)
    target = SyntheticTarget(k_max, cfg.vocab_size, cfg.target_hidden_size, device=cuda, seed=43, agree_p=0.68)
    dec = SpeculativeDecoder(d, target, CostAwareChain(**COSTS), capacity=ctx + 16 * (k_max + 1), k_max=k_max,
                             use_graphs=use_graphs)
    oc = od.make_cache(ctx + 16 * (k_max + 1), kv_bf16=True)
    _fill_cache(cuda, dec.rnd.cache, oc, ctx, seed=44)
    root = torch.randn(1, cfg.hidden_size, generator=torch.Generator(device=cuda).manual_seed(45), device=cuda)
    x0 = 151643
    dec.start(ctx, x0, root)
    opol = CostAwareChain(**COSTS)
    ohid = root.cpu().numpy()
    n = ctx
    for r in range(rounds):
        res = dec.round()
        k = res.k
        assert k == opol.plan(context_len=n, stochastic=False).max_depth, f"round {r}"
        logits = target.logits[:k + 1].cpu().numpy()
        taps = [t[:k + 1].float().cpu().numpy() for t in target.taps]
        drafts, a, acc, ohid = _oracle_chain(od, oc, ohid, k, logits, taps, dec.rnd.drafts[:k].tolist())
        opol.observe(a, k, k, 0.0, 0.0)
        assert dec.rnd.drafts[:k].tolist() == drafts, f"round {r}"
        assert res.n_accepted == a == target.agreements[-1], f"round {r}"
        assert res.tokens == acc, f"round {r}"
        assert _rel(dec.rnd.upd_hid[a].cpu().numpy(), ohid[0]) < 1e-2, f"round {r}"
        n += a + 1
        assert dec.n == n and dec.x_n == acc[-1]
    assert dec.policy.chosen == opol.chosen
    assert len(set(opol.chosen)) > 1, "the policy never changed the chain length"
    assert dec.rnd.committed() == n
    kg = dec.rnd.cache[0].keys[0, :, ctx:n].float().cpu().numpy()
    assert _rel(kg, oc.keys_f32(0)[:, ctx:n]) < 1e-2
    assert dec.rnd.syncs == rounds


def test_generate_stops_at_eos_and_max_tokens(cuda):
    from woodcock_amd.config import DrafterConfig
    from woodcock_amd.drafter import Drafter
    from woodcock_amd.policies import StaticPolicy
    from woodcock_amd.spec import SpeculativeDecoder
    from woodcock_amd.synthetic import SyntheticTarget, random_drafter

    cfg = DrafterConfig(hidden_size=256, num_layers=1, num_heads=4, num_kv_heads=2, head_dim=64,
                        intermediate_size=512, vocab_size=4096, target_hidden_size=192)
    d = Drafter(cfg, random_drafter(cfg, seed=3, device=cuda), cuda, torch.float32)
    root = torch.randn(1, 256, device=cuda)

    def run(max_new, eos=()):
        # identical state each time: same root, a fresh synthetic target of the same seed
        target = SyntheticTarget(4, cfg.vocab_size, cfg.target_hidden_size, device=cuda, seed=5, agree_p=0.9)
        dec = SpeculativeDecoder(d, target, StaticPolicy(4), capacity=512, k_max=4)
        dec.start(10, 7, root)
        return dec.generate(max_new, eos)

    out, st = run(23)
    assert len(out) == 23 and out[0] == 7 and st.new_tokens == 23
    assert st.rounds == len(st.accepted) and all(k == 4 for k in st.drafted)
    assert sum(a + 1 for a in st.accepted) >= 22
    i = next(j for j in range(3, len(out)) if out[j] not in out[:j])
    out2, st2 = run(100, eos={out[i]})
    assert out2 == out[: i + 1]
    assert st2.rounds <= st.rounds


@pytest.mark.parametrize("layers,ctx,rounds", [(2, 2048, 3), (28, 256, 2)], ids=["2l-ctx2048", "28l-ctx256"])
def test_tree_rounds_qwen3_1p7b(cuda, layers, ctx, rounds):
    """Config-5 tree rounds (depth 6, top-4, 60 nodes) against the oracle: the
    drafted tree, the target's tree-masked logits and taps (2 layers at ctx 2048,
    and the full 28-layer depth at ctx 256), the accepted branch, the target
    and drafter KV compacted along it, and the update pass's last hidden row."""
    from woodcock_amd import _lib
    from woodcock_amd.config import qwen3_1p7b_drafter
    from woodcock_amd.policies import StaticPolicy
    from woodcock_amd.spec import SpeculativeDecoder, TargetRunner
    from woodcock_amd.synthetic import to_bits
    from woodcock_amd.target import TargetConfig, TargetModel, random_target

    dcfg = qwen3_1p7b_drafter()
    tcfg = TargetConfig(num_layers=layers)
    depth, width, budget = 6, 4, 59
    cap = ctx + 128
    feats = (0, 1, 1) if layers == 2 else (2, 14, 25)
    d, od = _drafter(cuda, dcfg, 16384, seed=51)
    tw = random_target(tcfg, seed=52, device=cuda)
    model = TargetModel(tcfg, tw, cuda, max_rows=64, feature_layers=feats)
    tcache = model.make_cache(cap)
    runner = TargetRunner(model, tcache)
    policy = StaticPolicy(depth, width, budget)
    dec = SpeculativeDecoder(d, runner, policy, capacity=cap, k_max=4, max_tree_depth=depth)
    oc = od.make_cache(cap, kv_bf16=True)
    _fill_cache(cuda, dec.rnd.cache, oc, ctx, seed=53)
    ot = TargetStack(tcfg, {k: to_bits(v) for k, v in tw.items()}, feats, cap, kv_bf16=True)
    g = torch.Generator(device=cuda).manual_seed(54)
    for c, o in zip(tcache, ot.caches):
        c.keys[0, :, :ctx] = torch.randn(c.keys[0, :, :ctx].shape, generator=g, device=cuda).bfloat16()
        c.values[0, :, :ctx] = torch.randn(c.values[0, :, :ctx].shape, generator=g, device=cuda).bfloat16()
        o.k[0][:] = to_bits(c.keys[0])
        o.v[0][:] = to_bits(c.values[0])
        o.offset = ctx
    root = torch.randn(1, dcfg.hidden_size, generator=torch.Generator(device=cuda).manual_seed(55), device=cuda)
    dec.start(ctx, 9000, root)
    V = _lib
    rng = np.random.default_rng(56)
    for r in range(rounds):
        n = dec.n
        plan = policy.plan(context_len=n, stochastic=False)
        tree, rows = dec.enqueue_tree_draft(plan)
        logits, taps = dec.enqueue_tree_target(tree, rows)
        torch.cuda.synchronize()
        toks = tree.tokens[:rows].tolist()
        pars = tree.parents[:rows].tolist()
        deps = tree.depth[:rows].tolist()
        # the oracle's tree from the same root, cache and x_n
        root_hid = dec.rnd.upd_hid[int(dec.rnd.verdict[V.V_N_KEEP]) - 1].cpu().numpy()[None]
        root_out = core.rmsnorm(root_hid, od.w["norm.weight"], dcfg.rms_norm_eps)
        otree, _, _ = otd.draft_tree_greedy(od, oc, dec.x_n, root_out, od.feedback(root_hid, root_out), depth,
                                            width, budget)
        assert (otree.tokens, otree.parents, otree.depth) == (toks, pars, deps), f"round {r}"
        assert rows == len(toks) == budget + 1
        # plant a greedy walk down to a deep node whose path is not a prefix of the block
        leaves = [v for v in range(rows) if deps[v] >= 3]
        path = []
        for v in rng.permutation(leaves):
            p, u = [], int(v)
            while u > 0:
                p.append(u)
                u = pars[u]
            p = p[::-1]
            if p != list(range(1, len(p) + 1)):
                path = p
                break
        assert path, "no non-contiguous branch in the tree"
        kids = {u: [v for v in range(rows) if pars[v] == u] for u in range(rows)}
        last = path[-1]
        nxt = next(t for t in range(100, 151936) if t not in {toks[c] for c in kids[last]})
        plant = [(u, toks[c]) for u, c in zip([0] + path[:-1], path)] + [(last, nxt)]
        # oracle target forward over the tree block (positions n + depth, tree mask)
        pos = np.array([n + dd for dd in deps], np.int32)
        mask = S.tree_attention_mask(S.DraftTree(toks, pars, deps), n).astype(np.uint8)
        ologits, otaps = ot.forward(toks, positions=pos, mask=mask)
        assert _rel(logits.cpu().numpy(), ologits) < 1e-3, f"round {r}"
        for t, o in zip(taps, otaps):
            assert _rel(t.cpu().numpy(), o) < 1e-3, f"round {r}"
        for u, t in plant:
            logits[u, t] = 1e4
            ologits[u, t] = 1e4
        # GPU: verify, compaction along the branch, update; one sync
        dec.rnd.enqueue_tree_verify(logits, tree.tokens[:rows], tree.parents[:rows])
        dec.rnd.enqueue_tree_commit(taps, rows, plan.max_depth)
        dec.rnd.enqueue_readback()
        res = dec.rnd.finish()
        keep = dec.rnd.last_keep()
        # oracle: walk, compaction, update
        opath, onext = S.verify_tree_greedy(ologits.argmax(-1).tolist(), S.DraftTree(toks, pars, deps))
        assert opath == path and onext == nxt
        assert keep == [0] + path and res.n_accepted == len(path)
        acc = [toks[v] for v in path] + [nxt]
        assert res.tokens == acc
        ot.compact(n, keep)
        for i in range(tcfg.num_layers):
            gk = tcache[i].keys[0, :, n:n + len(keep)].float().cpu().numpy()
            gv = tcache[i].values[0, :, n:n + len(keep)].float().cpu().numpy()
            assert _rel(gk, ot.caches[i].keys_f32(0)[:, n:n + len(keep)]) < 1e-2, f"round {r} layer {i}"
            assert _rel(gv, ot.caches[i].values_f32(0)[:, n:n + len(keep)]) < 1e-2, f"round {r} layer {i}"
        ohid, _ = od.forward(acc, od.fuse([o[keep] for o in otaps]), oc)
        assert _rel(dec.rnd.upd_hid[len(keep) - 1].cpu().numpy(), ohid[-1]) < 1e-2, f"round {r}"
        dec.n += len(acc)
        dec.x_n = acc[-1]
        assert dec.rnd.committed() == dec.n == oc.offset == ot.offset
        # next round from identical inputs: the oracle takes the GPU's caches and root
        for i, c in enumerate(dec.rnd.cache):
            oc.k[i][:] = to_bits(c.keys[0])
            oc.v[i][:] = to_bits(c.values[0])
        for i, c in enumerate(tcache):
            ot.caches[i].k[0][:] = to_bits(c.keys[0])
            ot.caches[i].v[0][:] = to_bits(c.values[0])


def test_tree_round_through_the_loop(cuda):
    """StaticPolicy with width > 1 takes the tree path of round(): the committed
    count and x_n advance by the accepted path + 1, the drafter cache offset by
    the same, and the target cache offsets follow."""
    from woodcock_amd.config import DrafterConfig
    from woodcock_amd.drafter import Drafter
    from woodcock_amd.policies import StaticPolicy
    from woodcock_amd.spec import SpeculativeDecoder, TargetRunner
    from woodcock_amd.synthetic import random_drafter
    from woodcock_amd.target import TargetConfig, TargetModel, random_target

    dcfg = DrafterConfig(hidden_size=512, num_layers=1, num_heads=4, num_kv_heads=2, head_dim=128,
                         intermediate_size=1024, vocab_size=1000, target_hidden_size=512)
    tcfg = TargetConfig(hidden_size=512, num_heads=4, num_kv_heads=2, head_dim=128, intermediate_size=1024,
                        num_layers=3, vocab_size=1000)
    d = Drafter(dcfg, random_drafter(dcfg, seed=7, device=cuda), cuda, torch.bfloat16)
    model = TargetModel(tcfg, random_target(tcfg, seed=8, device=cuda), cuda, max_rows=64, feature_layers=(0, 1, 2))
    runner = TargetRunner(model, model.make_cache(256))
    dec = SpeculativeDecoder(d, runner, StaticPolicy(3, 3, 10), capacity=256, k_max=3, max_tree_depth=3)
    dec.start(20, 5, torch.randn(1, 512, device=cuda))
    for _ in range(4):
        n0 = dec.n
        res = dec.round()
        assert dec.n == n0 + res.n_accepted + 1 == dec.rnd.committed()
        assert runner.cache[0].offset == dec.n == dec.rnd.cache[0].offset
        assert res.k == 10 and res.depth == 3


def test_sampled_rounds_qwen3_1p7b(cuda):
    from woodcock_amd import _lib
    from woodcock_amd.config import qwen3_1p7b_drafter
    from woodcock_amd.policies import StaticPolicy
    from woodcock_amd.sampling import SamplingParams
    from woodcock_amd.spec import PURPOSE_DRAFT, PURPOSE_VERIFY, S_ROUND, SpeculativeDecoder, TargetRunner
    from woodcock_amd.synthetic import to_bits
    from woodcock_amd.target import TargetConfig, TargetModel, random_target

    dcfg = qwen3_1p7b_drafter()
    tcfg = TargetConfig(num_layers=2)
    ctx, depth, width, budget = 2048, 6, 4, 59
    cap = ctx + 128
    feats = (0, 1, 1)
    # top-k: its boundary is exact on logits / T, so the warped rows can be compared with
    # the oracle's entry for entry (top-p over a near-flat random-init target would put
    # thousands of fp32-equal values at the boundary; the warping tests pin top-p)
    sp = SamplingParams(temperature=0.9, top_k=1000, seed=61)
    d, od = _drafter(cuda, dcfg, 16384, seed=62)
    tw = random_target(tcfg, seed=63, device=cuda)
    model = TargetModel(tcfg, tw, cuda, max_rows=64, feature_layers=feats)
    tcache = model.make_cache(cap)
    runner = TargetRunner(model, tcache)
    policy = StaticPolicy(depth, width, budget)
    dec = SpeculativeDecoder(d, runner, policy, capacity=cap, k_max=4, max_tree_depth=depth, sampling=sp)
    oc = od.make_cache(cap, kv_bf16=True)
    _fill_cache(cuda, dec.rnd.cache, oc, ctx, seed=64)
    ot = TargetStack(tcfg, {k: to_bits(v) for k, v in tw.items()}, feats, cap, kv_bf16=True)
    g = torch.Generator(device=cuda).manual_seed(65)
    for c, o in zip(tcache, ot.caches):
        c.keys[0, :, :ctx] = torch.randn(c.keys[0, :, :ctx].shape, generator=g, device=cuda).bfloat16()
        c.values[0, :, :ctx] = torch.randn(c.values[0, :, :ctx].shape, generator=g, device=cuda).bfloat16()
        o.k[0][:] = to_bits(c.keys[0])
        o.v[0][:] = to_bits(c.values[0])
        o.offset = ctx
    root = torch.randn(1, dcfg.hidden_size, generator=torch.Generator(device=cuda).manual_seed(66), device=cuda)
    dec.start(ctx, 9000, root)
    V = _lib
    d2t = d.vocab_ids.cpu().numpy()
    rng = np.random.default_rng(67)
    paths = []
    for r in range(4):
        n = dec.n
        plan = policy.plan(context_len=n, stochastic=True)
        tree, rows, tdr = dec.enqueue_sampled_draft(plan)
        logits, taps = dec.enqueue_tree_target(tree, rows)
        torch.cuda.synchronize()
        rnd = int(dec.rnd.state[S_ROUND].item())
        cnt = int(tree.count.item())
        toks = tree.tokens[:rows].tolist()
        pars = tree.parents[:rows].tolist()
        deps = tree.depth[:rows].tolist()
        root_hid = dec.rnd.upd_hid[int(dec.rnd.verdict[V.V_N_KEEP]) - 1].cpu().numpy()[None]
        root_out = core.rmsnorm(root_hid, od.w["norm.weight"], dcfg.rms_norm_eps)
        otree, _, oq = otd.draft_tree_sample(od, oc, dec.x_n, root_out, od.feedback(root_hid, root_out), depth, width,
                                             budget, sp.temperature, sp.seed, rnd, PURPOSE_DRAFT,
                                             follow=toks[:cnt])
        assert (otree.tokens, otree.parents, otree.depth) == (toks[:cnt], pars[:cnt], deps[:cnt]), f"round {r}"
        assert rows == budget + 1 and cnt == rows
        pos = np.array([n + dd for dd in deps], np.int32)
        mask = S.tree_attention_mask(S.DraftTree(toks, pars, deps), n).astype(np.uint8)
        ologits, otaps = ot.forward(toks, positions=pos, mask=mask)
        assert _rel(logits.cpu().numpy(), ologits) < 1e-3, f"round {r}"
        for t, o in zip(taps, otaps):
            assert _rel(t.cpu().numpy(), o) < 1e-3, f"round {r}"
        if r % 2 == 0:
            # even rounds: a target that puts all its mass on a deep, non-contiguous
            # branch, so the walk accepts it (p(x) = 1 >= q(x)) and the compaction gathers
            leaves = [v for v in range(rows) if deps[v] >= 3]
            for v in rng.permutation(leaves):
                path, u = [], int(v)
                while u > 0:
                    path.append(u)
                    u = pars[u]
                if path[::-1] != list(range(1, len(path) + 1)):
                    break
            path = path[::-1]
            for u, c in zip([0] + path[:-1], path):
                logits[u, toks[c]] = 1e4
            logits[path[-1], 123] = 1e4
        # GPU: warped target distribution, recursive rejection, compaction, update; one sync
        p = dec.enqueue_sampled_verify(tdr, tree, logits, rows)
        dec.rnd.enqueue_tree_commit(taps, rows, plan.max_depth)
        dec.rnd.enqueue_readback()
        res = dec.rnd.finish()
        keep = dec.rnd.last_keep()
        p_np = p.cpu().numpy()
        wp = S.probs_from_logits(logits.cpu().numpy(), sp.temperature, sp.top_k, sp.top_p)
        assert ((p_np > 0) == (wp > 0)).all(), f"round {r}: top-k kept sets differ"
        assert np.abs(p_np - wp).max() <= 1e-5 * wp.max(), f"round {r}"
        # the oracle rule on the GPU's p and draft rows
        qs = tdr.q_store.cpu().numpy()
        qr = tree.q_rows[:cnt].tolist()
        tr = S.DraftTree(toks, pars, deps)
        pd = {v: p_np[v].astype(np.float64) for v in range(rows)}
        qd = {v: S.scatter_draft_dist(qs[qr[v]], d2t, tcfg.vocab_size) for v in range(rows) if tr.children[v]}
        for v in qd:
            assert np.abs(qs[qr[v]] - oq[v]).max() < 1e-2 * oq[v].max(), f"round {r} node {v}"
        ust = core.UniformStream(sp.seed, rnd, PURPOSE_VERIFY)
        opath, onext = S.verify_tree_stochastic(pd, qd, tr, ust)
        v = _lib.Verdict.from_buffer_copy(dec.rnd.host_verdict.numpy().tobytes())
        assert keep == [0] + opath and res.n_accepted == len(opath), f"round {r}"
        acc = [toks[u] for u in opath] + [onext]
        assert res.tokens == acc and int(v.n_uniforms) == ust.pos
        if r % 2 == 0:
            assert opath == path and onext == 123, f"round {r}"
        paths.append(opath)
        ot.compact(n, keep)
        for i in range(tcfg.num_layers):
            gk = tcache[i].keys[0, :, n:n + len(keep)].float().cpu().numpy()
            assert _rel(gk, ot.caches[i].keys_f32(0)[:, n:n + len(keep)]) < 1e-2, f"round {r} layer {i}"
        ohid, _ = od.forward(acc, od.fuse([o[keep] for o in otaps]), oc)
        assert _rel(dec.rnd.upd_hid[len(keep) - 1].cpu().numpy(), ohid[-1]) < 1e-2, f"round {r}"
        dec.n += len(acc)
        dec.x_n = acc[-1]
        assert dec.rnd.committed() == dec.n == oc.offset == ot.offset
        for i, c in enumerate(dec.rnd.cache):
            oc.k[i][:] = to_bits(c.keys[0])
            oc.v[i][:] = to_bits(c.values[0])
        for i, c in enumerate(tcache):
            ot.caches[i].k[0][:] = to_bits(c.keys[0])
            ot.caches[i].v[0][:] = to_bits(c.values[0])


@pytest.mark.parametrize("shape", [(4, 1, 4), (3, 3, 10)], ids=["chain", "tree"])
def test_sampled_rounds_through_the_loop(cuda, shape):
    from woodcock_amd.config import DrafterConfig
    from woodcock_amd.drafter import Drafter
    from woodcock_amd.policies import StaticPolicy
    from woodcock_amd.sampling import SamplingParams
    from woodcock_amd.spec import SpeculativeDecoder, TargetRunner
    from woodcock_amd.synthetic import random_drafter
    from woodcock_amd.target import TargetConfig, TargetModel, random_target

    dcfg = DrafterConfig(hidden_size=512, num_layers=1, num_heads=4, num_kv_heads=2, head_dim=128,
                         intermediate_size=1024, vocab_size=1000, target_hidden_size=512)
    tcfg = TargetConfig(hidden_size=512, num_heads=4, num_kv_heads=2, head_dim=128, intermediate_size=1024,
                        num_layers=3, vocab_size=1000)
    d = Drafter(dcfg, random_drafter(dcfg, seed=17, device=cuda), cuda, torch.bfloat16)
    model = TargetModel(tcfg, random_target(tcfg, seed=18, device=cuda), cuda, max_rows=64, feature_layers=(0, 1, 2))
    runner = TargetRunner(model, model.make_cache(256))
    depth, width, budget = shape
    dec = SpeculativeDecoder(d, runner, StaticPolicy(depth, width, budget), capacity=256, k_max=4,
                             max_tree_depth=depth, sampling=SamplingParams(temperature=1.0, seed=5))
    dec.start(20, 5, torch.randn(1, 512, device=cuda))
    out, st = dec.generate(24)
    assert len(out) == 24 and st.rounds >= 24 // (depth + 1)
    assert all(0 <= t < 1000 for t in out)
    assert dec.rnd.committed() == dec.n == runner.cache[0].offset == dec.rnd.cache[0].offset
    assert dec.n == 20 + sum(a + 1 for a in st.accepted)
    assert set(st.drafted) == {budget} and max(st.depths) <= depth
