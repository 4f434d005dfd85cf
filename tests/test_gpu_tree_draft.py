"""Greedy tree drafting on the device (woodcock_amd.tree_draft.TreeDrafter:
python/woodcock/spec.py:216-303 with a StaticPolicy) against the oracle
restatement (oracle/tree_draft.py) on identical weights, cache and root:
identical verified trees (tokens, parents, depths, node count), the drafter
cache offset untouched, and the tree entries written to the drafter cache
within the fp32 tolerance.  Shapes: a small drafter with an fp32 and a bf16
cache, and the Qwen3-1.7B drafter with the config-5 tree (depth 6, width 4,
60 verified rows).

Sampled drafting at T > 0 (TreeDrafter(stochastic=True); spec.py:238-249)
against oracle/tree_draft.draft_tree_sample fed the same Philox stream: the
same drawn tree (a draw may differ only where two Gumbel keys agree within
rounding of the fp32 / bf16 forward, and then the GPU's is followed), every
parent's q row within tolerance at the row the tree names, padding rows
after the live count, and the shapes where the counts are data-dependent --
budget-limited levels, a temperature so low that each q has one nonzero entry
(one child per node instead of `width`), and no budget at all."""
import numpy as np
import pytest
import torch

from oracle import core
from oracle import tree_draft as otd

pytestmark = pytest.mark.gpu


def _small_cfg():
    from woodcock_amd.config import DrafterConfig

    return DrafterConfig(hidden_size=256, num_layers=1, num_heads=4, num_kv_heads=2, head_dim=64,
                         intermediate_size=512, vocab_size=4096, target_hidden_size=192, rope_theta=1e6)


def _setup(cuda, cfg, head_rows, ctx, cap, kv_dtype, seed):
    from woodcock_amd.drafter import Drafter
    from woodcock_amd.synthetic import draft_vocab, random_drafter, to_bits

    ids = draft_vocab(cfg.vocab_size, head_rows, seed=seed)
    w = random_drafter(cfg, seed=seed, device=cuda, head_rows=head_rows)
    d = Drafter(cfg, dict(w), cuda, kv_dtype)
    d._vocab_ids = torch.from_numpy(ids).to(cuda)
    d._build_structs(d._rope[0].shape[0])
    cache = d.make_cache(cap)
    od = core.Drafter(cfg.as_dict(), {k: to_bits(v) for k, v in w.items()})
    od.d2t = ids
    oc = od.make_cache(cap, kv_bf16=kv_dtype == torch.bfloat16)
    g = torch.Generator(device=cuda).manual_seed(seed)
    c = cache[0]
    c.keys[0, :, :ctx] = torch.randn(c.keys[0, :, :ctx].shape, generator=g, device=cuda).to(kv_dtype)
    c.values[0, :, :ctx] = torch.randn(c.values[0, :, :ctx].shape, generator=g, device=cuda).to(kv_dtype)
    if kv_dtype == torch.bfloat16:
        oc.k[0][:] = to_bits(c.keys[0])
        oc.v[0][:] = to_bits(c.values[0])
    else:
        oc.k[0][:] = c.keys[0].cpu().numpy()
        oc.v[0][:] = c.values[0].cpu().numpy()
    oc.offset = ctx
    root_out = torch.randn(cfg.hidden_size, generator=g, device=cuda)
    return d, cache, od, oc, root_out


def _run(cuda, cfg, head_rows, ctx, cap, kv_dtype, depth, width, budget, seed, tol):
    from woodcock_amd.tree_draft import TreeDrafter

    d, cache, od, oc, root_out = _setup(cuda, cfg, head_rows, ctx, cap, kv_dtype, seed)
    root_tok = 11
    tdr = TreeDrafter(d, cache, depth, width, budget)
    off = torch.tensor([ctx], dtype=torch.int32, device=cuda)
    tree = tdr.draft(torch.tensor([root_tok], dtype=torch.int32, device=cuda), root_out, root_out, off)
    torch.cuda.synchronize()
    want, _, nodes = otd.draft_tree_greedy(od, oc, root_tok, root_out.cpu().numpy(), root_out.cpu().numpy(),
                                           depth, width, budget)
    n = int(tree.count.item())
    assert n == len(want)
    assert tree.tokens[:n].tolist() == want.tokens
    assert tree.parents[:n].tolist() == want.parents
    assert tree.depth[:n].tolist() == want.depth
    assert int(off.item()) == ctx and oc.offset == ctx
    # tree entries in the drafter cache: (depth - 1) * width forwarded rows after the context
    t = (depth - 1) * width
    k_gpu = cache[0].keys[0, :, ctx:ctx + t].float().cpu().numpy()
    k_ref = oc.keys_f32(0)[:, ctx:ctx + t]
    assert np.abs(k_gpu - k_ref).max() / np.abs(k_ref).max() <= tol
    return tdr, tree


@pytest.mark.parametrize("kv_dtype", [torch.float32, torch.bfloat16])
def test_small_tree_matches_oracle(cuda, kv_dtype):
    _run(cuda, _small_cfg(), 1024, 40, 256, kv_dtype, depth=4, width=3, budget=10, seed=2, tol=1e-5 if
         kv_dtype == torch.float32 else 1e-2)


def test_every_node_kept_when_within_budget(cuda):
    tdr, tree = _run(cuda, _small_cfg(), 1024, 24, 128, torch.float32, depth=3, width=2, budget=64, seed=4, tol=1e-5)
    assert int(tree.count.item()) == tdr.n_nodes == 1 + 2 + 2 * 4


def test_width_one_is_a_chain(cuda):
    _, tree = _run(cuda, _small_cfg(), 1024, 30, 128, torch.float32, depth=4, width=1, budget=4, seed=6, tol=1e-5)
    assert tree.parents[:5].tolist() == [-1, 0, 1, 2, 3]


def test_qwen3_1p7b_config5_tree(cuda):
    from woodcock_amd.config import qwen3_1p7b_drafter

    _run(cuda, qwen3_1p7b_drafter(), 16384, 512, 1024, torch.bfloat16, depth=6, width=4, budget=59, seed=8,
         tol=1e-2)


def test_enqueue_never_synchronises(cuda):
    from woodcock_amd.tree_draft import TreeDrafter

    d, cache, _, _, root_out = _setup(cuda, _small_cfg(), 1024, 20, 128, torch.float32, 9)
    tdr = TreeDrafter(d, cache, 3, 3, 8)
    tok = torch.tensor([3], dtype=torch.int32, device=cuda)
    off = torch.tensor([20], dtype=torch.int32, device=cuda)
    tdr.draft(tok, root_out, root_out, off)  # warm-up
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        tdr.draft(tok, root_out, root_out, off)
    finally:
        torch.cuda.set_sync_debug_mode(0)
    torch.cuda.synchronize()
    assert int(tdr.tree.count.item()) == 9


# ------------------------------------------------------------------ sampled drafting (T > 0)

SEED, PURPOSE = 77, 1


def _run_sampled(cuda, cfg, head_rows, ctx, cap, kv_dtype, depth, width, budget, seed, temperature, tol, rnd=3):
    from woodcock_amd import _lib
    from woodcock_amd.tree_draft import TreeDrafter

    d, cache, od, oc, root_out = _setup(cuda, cfg, head_rows, ctx, cap, kv_dtype, seed)
    root_tok = 11
    tdr = TreeDrafter(d, cache, depth, width, budget, stochastic=True)
    off = torch.tensor([ctx], dtype=torch.int32, device=cuda)
    rd = torch.tensor([rnd], dtype=torch.int32, device=cuda)
    tree = tdr.draft(torch.tensor([root_tok], dtype=torch.int32, device=cuda), root_out, root_out, off,
                     temperature=temperature, rng=_lib.Uniforms(SEED, rd.data_ptr(), PURPOSE))
    torch.cuda.synchronize()
    n = int(tree.count.item())
    toks = tree.tokens.tolist()
    ro = root_out.cpu().numpy()
    want, phat, qrow = otd.draft_tree_sample(od, oc, root_tok, ro, ro, depth, width, budget, temperature, SEED, rnd,
                                             PURPOSE, follow=toks[:n])
    assert n == len(want) <= tdr.max_nodes
    assert toks[:n] == want.tokens
    assert tree.parents[:n].tolist() == want.parents
    assert tree.depth[:n].tolist() == want.depth
    pad = tdr.max_nodes - n
    assert toks[n:] == [root_tok] * pad
    assert tree.parents[n:].tolist() == [0] * pad and tree.depth[n:].tolist() == [1] * pad
    assert int(off.item()) == ctx and oc.offset == ctx
    qr = tree.q_rows[:n].tolist()
    qs = tdr.q_store.cpu().numpy()
    for v, qv in qrow.items():  # the rows the verification reads: nodes with children
        if v in want.parents:
            assert np.abs(qs[qr[v]] - qv).max() <= tol * qv.max(), f"node {v}"
    return tdr, tree, want


@pytest.mark.parametrize("kv_dtype", [torch.float32, torch.bfloat16])
def test_sampled_small_tree_matches_oracle(cuda, kv_dtype):
    for rnd in (1, 2):
        _, _, t = _run_sampled(cuda, _small_cfg(), 1024, 40, 256, kv_dtype, depth=4, width=3, budget=10, seed=2,
                               temperature=1.0, tol=1e-5 if kv_dtype == torch.float32 else 1e-2, rnd=rnd)
        assert len(t) == 11  # 3 + (3 + 3 + 1) draws: the budget runs out in level 2


def test_sampled_budget_beyond_the_shape(cuda):
    # width 2, depth 3: 2 + 4 + 4 draws, budget 20 never binds
    _, tree, t = _run_sampled(cuda, _small_cfg(), 1024, 24, 128, torch.float32, depth=3, width=2, budget=20, seed=4,
                              temperature=0.8, tol=1e-5)
    assert len(t) == 11 and int(tree.count.item()) == 11


def test_sampled_one_child_per_node_at_low_temperature(cuda):
    """T = 1e-6: every q is one-hot, so each node draws one child instead of
    `width` -- the counts differ from the static shape and the tree is the
    greedy chain."""
    _, tree, t = _run_sampled(cuda, _small_cfg(), 1024, 30, 128, torch.float32, depth=4, width=3, budget=12, seed=6,
                              temperature=1e-6, tol=1e-5)
    assert t.parents == [-1, 0, 1, 2, 3]
    _, chain = _run(cuda, _small_cfg(), 1024, 30, 128, torch.float32, depth=4, width=1, budget=4, seed=6,
                    tol=1e-5)
    assert tree.tokens[:5].tolist() == chain.tokens[:5].tolist()


def test_sampled_zero_budget_is_the_root(cuda):
    _, tree, t = _run_sampled(cuda, _small_cfg(), 1024, 20, 128, torch.float32, depth=3, width=2, budget=0, seed=5,
                              temperature=1.0, tol=1e-5)
    assert len(t) == 1 and int(tree.count.item()) == 1


def test_sampled_chain_width_one(cuda):
    _, tree, t = _run_sampled(cuda, _small_cfg(), 1024, 30, 128, torch.float32, depth=5, width=1, budget=5, seed=7,
                              temperature=0.7, tol=1e-5)
    assert t.parents == [-1, 0, 1, 2, 3, 4]


def test_sampled_qwen3_1p7b_config5_shape(cuda):
    from woodcock_amd.config import qwen3_1p7b_drafter

    _, tree, t = _run_sampled(cuda, qwen3_1p7b_drafter(), 16384, 512, 1024, torch.bfloat16, depth=6, width=4,
                              budget=59, seed=8, temperature=1.0, tol=1e-2)
    assert len(t) == 60


def test_sampled_enqueue_never_synchronises(cuda):
    from woodcock_amd import _lib
    from woodcock_amd.tree_draft import TreeDrafter

    d, cache, _, _, root_out = _setup(cuda, _small_cfg(), 1024, 20, 128, torch.float32, 9)
    tdr = TreeDrafter(d, cache, 3, 3, 8, stochastic=True)
    tok = torch.tensor([3], dtype=torch.int32, device=cuda)
    off = torch.tensor([20], dtype=torch.int32, device=cuda)
    rd = torch.tensor([0], dtype=torch.int32, device=cuda)
    u = _lib.Uniforms(1, rd.data_ptr(), PURPOSE)
    tdr.draft(tok, root_out, root_out, off, temperature=1.0, rng=u)  # warm-up
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        tdr.draft(tok, root_out, root_out, off, temperature=1.0, rng=u)
    finally:
        torch.cuda.set_sync_debug_mode(0)
    torch.cuda.synchronize()
    assert int(tdr.tree.count.item()) == 9


@pytest.mark.parametrize("head_rows", [16384, 3001])
def test_expand_from_logits_equals_softmax_then_expand(cuda, head_rows):
    """wc_tree_draft_expand_logits (the children and their q formed from the
    logits by per-part row statistics) against wc_probs_from_logits at T = 1
    followed by wc_tree_draft_expand on the same logits, over two levels (the
    root's children, then a frontier of `width` rows): the same node table
    (tokens, parents, depths of every node), and phat within 1e-6 relative --
    only the association of the softmax sum differs.  3001 head rows: two
    parts, and rows after the first start off the 16-byte vector alignment
    (read element by element)."""
    import ctypes as C

    from woodcock_amd import _lib
    from woodcock_amd.runtime import ptr, stream_ptr, workspace

    width, off = 4, 40
    rng = np.random.default_rng(head_rows)
    d2t = torch.from_numpy(np.sort(rng.choice(151936, head_rows, replace=False)).astype(np.int32)).to(cuda)
    z1 = torch.from_numpy((rng.standard_normal((1, head_rows)) * 3).astype(np.float32)).to(cuda)
    z2 = torch.from_numpy((rng.standard_normal((width, head_rows)) * 3).astype(np.float32)).to(cuda)
    nbytes = int(_lib.lib().wc_tree_draft_state_bytes())
    n = 1 + width + width * width

    def run(fused):
        st = torch.zeros(nbytes, dtype=torch.uint8, device=cuda)
        root = torch.tensor([7], dtype=torch.int32, device=cuda)
        offset = torch.tensor([off], dtype=torch.int32, device=cuda)
        q = torch.empty(width, head_rows, device=cuda)
        s = stream_ptr()

        def expand(z, rows, base):
            if fused:
                _lib.call("wc_tree_draft_expand_logits", ptr(st), ptr(z), rows, head_rows, z.stride(0), ptr(d2t),
                          width, base, s)
            else:
                _lib.call("wc_probs_from_logits", ptr(z), rows, head_rows, z.stride(0), 1.0, 0, 1.0, ptr(q),
                          q.stride(0), ptr(workspace(cuda)), s)
                _lib.call("wc_tree_draft_expand", ptr(st), ptr(q), rows, head_rows, q.stride(0), ptr(d2t), width,
                          base, s)

        _lib.call("wc_tree_draft_begin", ptr(st), ptr(root), s)
        expand(z1, 1, 1)
        tok, feat, pos = (torch.empty(width, dtype=torch.int32, device=cuda) for _ in range(3))
        mask = torch.empty(width, 64, dtype=torch.uint8, device=cuda)
        _lib.call("wc_tree_draft_frontier", ptr(st), 1, 1 + width, width, ptr(offset), 0, 0, 1, ptr(tok), ptr(feat),
                  ptr(pos), ptr(mask), mask.stride(0), s)
        expand(z2, width, 1 + width)
        out = [torch.empty(n, dtype=torch.int32, device=cuda) for _ in range(3)]
        count = torch.empty(1, dtype=torch.int32, device=cuda)
        _lib.call("wc_tree_draft_select", ptr(st), n, n - 1, *[ptr(o) for o in out], ptr(count), s)
        torch.cuda.synchronize()
        phat = st[: 8 * n].view(torch.float64).cpu().numpy()  # the node table's first field
        return [o.cpu().numpy() for o in out], int(count.item()), phat

    (ta, ca, pa), (tb, cb, pb) = run(False), run(True)
    assert ca == cb == n
    for x, y in zip(ta, tb):
        assert (x == y).all()
    assert np.abs(pb - pa).max() <= 1e-6 * np.abs(pa).max()
    assert np.all(pa[1:] > 0) and np.all(pa[1:] < 1)
