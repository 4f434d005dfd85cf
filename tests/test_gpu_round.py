"""The fused greedy chain round (python/woodcock/spec.py:331-374) on the GPU vs an
oracle round built from the CPU drafter restatement, round after round:
identical drafted tokens, accepted lengths and accepted tokens; root outputs
and drafter caches within the fp32 tolerance; exactly one host sync per
round; a captured HIP graph replays to the same results as eager rounds."""
import ctypes as C

import numpy as np
import pytest
import torch

from oracle import core
from oracle import sampling as osamp

pytestmark = pytest.mark.gpu

K = 4


def small_cfg():
    from woodcock_amd.config import DrafterConfig

    return DrafterConfig(hidden_size=256, num_layers=1, num_heads=4, num_kv_heads=2, head_dim=64,
                         intermediate_size=512, vocab_size=4096, target_hidden_size=192, rope_theta=1e6)


def setup(cuda, seed, ctx=40, kv_dtype=torch.float32, cap=256, cfg=None, head_rows=1024, k=K):
    from woodcock_amd.drafter import Drafter
    from woodcock_amd.spec import ChainRound
    from woodcock_amd.synthetic import SyntheticTarget, draft_vocab, random_drafter, to_bits

    cfg = cfg or small_cfg()
    ids = draft_vocab(cfg.vocab_size, head_rows, seed=seed)
    w = random_drafter(cfg, seed=seed, device=cuda, head_rows=head_rows)
    d = Drafter(cfg, dict(w), cuda, kv_dtype)
    d._vocab_ids = torch.from_numpy(ids).to(cuda)
    d._build_structs(d._rope[0].shape[0])
    rnd = ChainRound(d, k, cap)
    od = core.Drafter(cfg.as_dict(), {k: to_bits(v) for k, v in w.items()})
    od.d2t = ids
    oc = od.make_cache(cap, kv_bf16=kv_dtype == torch.bfloat16)
    g = torch.Generator(device=cuda).manual_seed(seed)
    c = rnd.cache[0]
    c.keys[0, :, :ctx] = torch.randn(c.keys[0, :, :ctx].shape, generator=g, device=cuda).to(kv_dtype)
    c.values[0, :, :ctx] = torch.randn(c.values[0, :, :ctx].shape, generator=g, device=cuda).to(kv_dtype)
    if kv_dtype == torch.bfloat16:
        oc.k[0][:] = to_bits(c.keys[0])
        oc.v[0][:] = to_bits(c.values[0])
    else:
        oc.k[0][:] = c.keys[0].cpu().numpy()
        oc.v[0][:] = c.values[0].cpu().numpy()
    oc.offset = ctx
    root = torch.randn(1, cfg.hidden_size, generator=g, device=cuda)  # the root's pre-norm hidden state
    rnd.set_root(ctx, root)
    target = SyntheticTarget(k, cfg.vocab_size, cfg.target_hidden_size, device=cuda, seed=seed + 1)
    return cfg, d, rnd, od, oc, target, root.cpu().numpy()


def oracle_round(od, oc, root_out, root_fb, logits, taps):
    drafts, out, fb = [], root_out, root_fb
    base = oc.offset
    for k in range(K):
        z = od.logits(out)
        drafts.append(int(od.d2t[core.argmax(z[0])]))
        if k < K - 1:
            hid, out = od.forward([drafts[-1]], fb, oc)
            fb = od.feedback(hid, out)
    oc.offset = base
    a, nxt = osamp.verify_chain_greedy(logits, drafts)
    acc = drafts[:a] + [nxt]
    g = od.fuse([t[: a + 1] for t in taps])
    hid, out = od.forward(acc, g, oc)
    return drafts, a, acc, out[-1:], od.feedback(hid[-1:], out[-1:]), hid[-1:]


def gpu_round(rnd, target, n_agree, fused=False):
    rnd.enqueue_draft()
    target.plant(rnd.drafts, n_agree)
    if fused:  # the verify and the fuse of every tap row in one launch
        rnd.enqueue_verify_commit(target.logits, target.taps)
    else:
        rnd.enqueue_verify(target.logits)
        rnd.enqueue_commit(target.taps)
    rnd.enqueue_readback()
    return rnd.finish()


def _rel(a, b):
    return float(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64)).max() / np.abs(b).max())


def test_rounds_match_oracle_round(cuda):
    cfg, d, rnd, od, oc, target, root = setup(cuda, 1)
    root_out = core.rmsnorm(root, od.w["norm.weight"], cfg.rms_norm_eps)
    root_fb = od.feedback(root, root_out)
    pattern = [2, 0, 4, 1, 3, 2, 4, 0]
    for r, n_agree in enumerate(pattern):
        res = gpu_round(rnd, target, n_agree)
        logits = target.logits.cpu().numpy()
        taps = [t.float().cpu().numpy() for t in target.taps]
        drafts, a, acc, root_out, root_fb, root_hid = oracle_round(od, oc, root_out, root_fb, logits, taps)
        assert rnd.drafts.tolist() == drafts, f"round {r}"
        assert res.n_accepted == a == n_agree, f"round {r}"
        assert res.tokens == acc, f"round {r}"
        assert _rel(rnd.upd_hid[a].cpu().numpy(), root_hid[0]) <= 1e-5, f"round {r}"
        n = oc.offset
        assert rnd.committed() == n
        k_gpu = rnd.cache[0].keys[0, :, :n].float().cpu().numpy()
        assert _rel(k_gpu, oc.keys_f32(0)[:, :n]) <= 1e-5, f"round {r}"
    assert rnd.syncs == len(pattern)


@pytest.mark.parametrize("hidden", [2560, 3072])
def test_wide_dual_stream_chain_matches_oracle(cuda, hidden):
    """Drafters wider than 2048 run the dual-stream QKV (the feature row and the
    token's embedding row, each RMS-normed) with x * gain staged once per block
    and the pending head argmax resolved after the weights are requested; 3072
    is six 512-wide steps on the eight-step kernel with the last two masked.
    The pending chain equals the plain chain bit for bit, and both equal the
    oracle's chain from the same root: drafts, and every step's hidden row
    within the fp32 tolerance."""
    from woodcock_amd.config import DrafterConfig

    kk = 5
    cfg = DrafterConfig(hidden_size=hidden, num_layers=1, num_heads=16, num_kv_heads=4, head_dim=128,
                        intermediate_size=1536, vocab_size=8192, target_hidden_size=512, rope_theta=1e6)
    cfg, d, rnd, od, oc, target, root = setup(cuda, 13, ctx=200, kv_dtype=torch.float32, cap=512, cfg=cfg,
                                              head_rows=4096, k=kk)
    assert d.pending_ok
    c = rnd.cache[0]
    k0, v0 = c.keys.clone(), c.values.clone()

    def run(pending):
        c.keys.copy_(k0)
        c.values.copy_(v0)
        rnd.drafts.zero_()
        rnd.step_hid.zero_()
        rnd.pending = pending
        rnd.enqueue_draft()
        torch.cuda.synchronize()
        return rnd.drafts.clone(), rnd.step_hid.clone(), c.keys.clone()

    plain = run(False)
    pend = run(True)
    for a, b, name in zip(plain, pend, ("drafts", "step_hid", "keys")):
        assert torch.equal(a, b), name
    out = core.rmsnorm(root, od.w["norm.weight"], cfg.rms_norm_eps)
    fb = od.feedback(root, out)
    drafts, hids = [], []
    for i in range(kk):
        z = od.logits(out)
        drafts.append(int(od.d2t[core.argmax(z[0])]))
        if i < kk - 1:
            hid, out = od.forward([drafts[-1]], fb, oc)
            fb = od.feedback(hid, out)
            hids.append(hid[0])
    assert plain[0][:kk].tolist() == drafts
    assert len(set(drafts)) > 1
    assert _rel(plain[1][: kk - 1].cpu().numpy(), np.stack(hids)) <= 1e-5


def test_config1_rounds_match_oracle_round(cuda):
    """The benchmarked round at its full shape: Qwen3-1.7B drafter, 16,384-row
    head, bf16 drafter cache at context 512 (capacity 1024), K = 4, the
    update pass at 5 host rows (a + 1 live) -- drafts, accepted lengths and
    tokens equal the oracle round's; root state and appended cache rows within
    the bf16-cache tolerance."""
    from woodcock_amd.config import qwen3_1p7b_drafter

    cfg, d, rnd, od, oc, target, root = setup(cuda, 7, ctx=512, kv_dtype=torch.bfloat16, cap=1024,
                                              cfg=qwen3_1p7b_drafter(), head_rows=16384)
    root_out = core.rmsnorm(root, od.w["norm.weight"], cfg.rms_norm_eps)
    root_fb = od.feedback(root, root_out)
    for r, n_agree in enumerate([2, 4, 0]):
        res = gpu_round(rnd, target, n_agree, fused=True)
        logits = target.logits.cpu().numpy()
        taps = [t.float().cpu().numpy() for t in target.taps]
        drafts, a, acc, root_out, root_fb, root_hid = oracle_round(od, oc, root_out, root_fb, logits, taps)
        assert rnd.drafts.tolist() == drafts, f"round {r}"
        assert res.n_accepted == a == n_agree, f"round {r}"
        assert res.tokens == acc, f"round {r}"
        assert _rel(rnd.upd_hid[a].cpu().numpy(), root_hid[0]) <= 1e-3, f"round {r}"
        n = oc.offset
        assert rnd.committed() == n
        k_gpu = rnd.cache[0].keys[0, :, 512:n].float().cpu().numpy()
        assert _rel(k_gpu, oc.keys_f32(0)[:, 512:n]) <= 1e-2, f"round {r}"
    assert rnd.syncs == 3


@pytest.mark.parametrize("kv,shape,k", [("f32", "small", 4), ("bf16", "small", 4), ("bf16", "qwen3_1p7b", 4),
                                        ("f32", "qwen3_1p7b", 7), ("bf16", "qwen3_1p7b", 8)])
def test_fused_verify_commit_equals_sequential(cuda, kv, shape, k):
    """enqueue_verify_commit (the greedy verify and the fuse of all k + 1 tap
    rows in one launch) leaves the verdict, root rows, drafter cache and device
    state of enqueue_verify + enqueue_commit (the fuse of the kept rows after
    the verdict) bit for bit, eagerly and replayed from captured graphs between
    eager rounds; at the small shape the taps' width takes the two-launch
    fallback, at the Qwen3-1.7B shape the one-launch kernel (k = 4: 250 verify
    units of 3,072 logits over 256 blocks, one each; k = 7: 400, two in some)
    up to its bound of eight rows (k = 8 falls back)."""
    from woodcock_amd.config import qwen3_1p7b_drafter

    kv_dtype = torch.float32 if kv == "f32" else torch.bfloat16
    kw = dict(cfg=qwen3_1p7b_drafter(), head_rows=16384, ctx=512, cap=1024) if shape != "small" else {}
    kw["k"] = k
    pattern = [3, 0, 4, 1, 2] if k == 4 else [k, 0, 5, k - 1, 2]
    _, _, seq, _, _, ts, _ = setup(cuda, 11, kv_dtype=kv_dtype, **kw)
    _, _, fus, _, _, tf, _ = setup(cuda, 11, kv_dtype=kv_dtype, **kw)
    for r, n in enumerate(pattern):
        a = gpu_round(seq, ts, n)
        b = gpu_round(fus, tf, n, fused=True)
        assert (a.n_accepted, a.tokens) == (b.n_accepted, b.tokens) and a.n_accepted == n, f"round {r}"
        assert torch.equal(seq.verdict, fus.verdict), f"round {r}"
        assert torch.equal(seq.state, fus.state), f"round {r}"
        assert torch.equal(seq.upd_hid[: n + 1], fus.upd_hid[: n + 1]), f"round {r}"
        assert torch.equal(seq.cache[0].keys, fus.cache[0].keys), f"round {r}"
        assert torch.equal(seq.cache[0].values, fus.cache[0].values), f"round {r}"
    s = torch.cuda.Stream()
    graphs = {}
    for r, n in enumerate(pattern):
        a = gpu_round(seq, ts, n)
        if n not in graphs:
            s.wait_stream(torch.cuda.current_stream())
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                fus.enqueue_draft()
                tf.plant(fus.drafts, n)
                fus.enqueue_verify_commit(tf.logits, tf.taps)
                fus.enqueue_readback()
            torch.cuda.synchronize()
            graphs[n] = g
        graphs[n].replay()
        b = fus.finish()
        _ = torch.ones(3, device=cuda).sum().item()  # eager work between replays
        assert (a.n_accepted, a.tokens) == (b.n_accepted, b.tokens), f"replay {r}"
        assert torch.equal(seq.verdict, fus.verdict), f"replay {r}"
        assert torch.equal(seq.upd_hid[: n + 1], fus.upd_hid[: n + 1]), f"replay {r}"
        assert torch.equal(seq.cache[0].keys, fus.cache[0].keys), f"replay {r}"


@pytest.mark.parametrize("tap_dtype", ["bf16", "f32"])
def test_verify_fuse_entry_edges(cuda, tap_dtype):
    """wc_verify_chain_greedy_fuse against wc_verify_chain_greedy followed by
    wc_drafter_fuse over the same rows, through the C-ABI, at the Qwen3-1.7B
    fuse shape: rows 1..8 (1 takes the two-call path, 2..8 the one launch), a
    ragged vocab (151,933 logits in rows of 151,936: the last float4 of a row
    is partial), the argmax planted in the last chunk, at index 0 and as ties
    (lowest index wins), and drafts that agree for a chosen prefix.  The
    verdict and the fused rows must be bit-identical."""
    from woodcock_amd import _lib
    from woodcock_amd.config import qwen3_1p7b_drafter
    from woodcock_amd.runtime import new_verdict, ptr, stream_ptr

    _, d, rnd, _, _, _, _ = setup(cuda, 5, cfg=qwen3_1p7b_drafter(), head_rows=16384, ctx=64, cap=128, k=7)
    V, LD, Dt = 151933, 151936, d.cfg.target_hidden_size
    g = torch.Generator(device=cuda).manual_seed(3)
    dt = torch.bfloat16 if tap_dtype == "bf16" else torch.float32
    tdt = _lib.WC_BF16 if tap_dtype == "bf16" else _lib.WC_F32
    ws = [torch.empty_like(rnd.vws) for _ in range(2)]
    for w in ws:
        _lib.call("wc_workspace_init", ptr(w), w.numel(), stream_ptr())
    for rows in range(1, 9):
        for case in range(3):
            buf = torch.randn(rows, LD, generator=g, device=cuda)
            logits = buf[:, :V]
            if case == 0:
                logits[0, V - 1] = 50.0  # the ragged end of row 0
                if rows > 1:
                    logits[1, 0] = 50.0
            elif case == 1:  # ties: the lowest index wins
                logits[:, 1000] = 40.0
                logits[:, 99000] = 40.0
            am = logits.argmax(dim=1).to(torch.int32)
            n_agree = (rows - 1) // 2 if case != 2 else rows - 1
            drafts = am[: rows - 1].clone()  # draft c is checked against row c's argmax
            if n_agree < rows - 1:
                drafts[n_agree] = (drafts[n_agree] + 1) % V
            drafts = drafts if rows > 1 else torch.zeros(1, dtype=torch.int32, device=cuda)
            taps = [torch.randn(rows, Dt, generator=g, device=cuda).to(dt) for _ in range(3)]
            tp = (C.c_void_p * 3)(*[x.data_ptr() for x in taps])
            outs = []
            for which in range(2):
                verdict = new_verdict(cuda)
                gout = torch.full((rows, d.cfg.hidden_size), float("nan"), device=cuda)
                if which == 0:
                    _lib.call("wc_verify_chain_greedy_fuse", ptr(logits), rows, V, LD, ptr(drafts), ptr(verdict),
                              ptr(ws[0]), C.byref(d.dims), C.byref(d.wstruct), tp, tdt, Dt, ptr(gout),
                              d.cfg.hidden_size, ptr(d.ws), stream_ptr())
                else:
                    _lib.call("wc_verify_chain_greedy", ptr(logits), rows, V, LD, ptr(drafts), ptr(verdict),
                              ptr(ws[1]), stream_ptr())
                    _lib.call("wc_drafter_fuse", C.byref(d.dims), C.byref(d.wstruct), tp, tdt, Dt, None, 0, rows,
                              None, ptr(gout), d.cfg.hidden_size, ptr(d.ws), stream_ptr())
                outs.append((verdict, gout))
            torch.cuda.synchronize()
            (v0, g0), (v1, g1) = outs
            assert torch.equal(v0, v1), (rows, case)
            assert int(v0[_lib.V_N_ACCEPTED]) == n_agree, (rows, case)
            assert int(v0[_lib.V_TOKENS + n_agree]) == int(am[n_agree]), (rows, case)
            assert torch.equal(g0, g1), (rows, case)


def test_enqueue_never_synchronises(cuda):
    """Everything between two verdict reads is asynchronous: torch's sync debug
    mode raises on any implicit host synchronisation while a round is enqueued."""
    cfg, d, rnd, od, oc, target, root = setup(cuda, 2)
    gpu_round(rnd, target, 1)  # warm-up (workspaces, attributes)
    torch.cuda.set_sync_debug_mode("error")
    try:
        rnd.enqueue_draft()
        target.plant(rnd.drafts, 2)
        rnd.enqueue_verify(target.logits)
        rnd.enqueue_commit(target.taps)
        rnd.enqueue_readback()
    finally:
        torch.cuda.set_sync_debug_mode(0)
    res = rnd.finish()
    assert res.n_accepted == 2


def test_graph_replay_equals_eager_rounds(cuda):
    """One captured graph per round shape, replayed with host work in between;
    every replay matches the eager round bit for bit."""
    pattern = [2, 3, 0, 4, 2, 1]
    _, _, eager, _, _, te, _ = setup(cuda, 3)
    eager_res = [gpu_round(eager, te, n) for n in pattern]
    eager_k = eager.cache[0].keys.clone()

    _, _, rnd, _, _, tg, _ = setup(cuda, 3)
    gpu_round(rnd, tg, 2)  # warm-up outside capture
    _, _, rnd, _, _, tg, _ = setup(cuda, 3)  # fresh identical state
    n_agree = torch.zeros(1, dtype=torch.int32)
    graphs = {}
    s = torch.cuda.Stream()
    results = []
    for n in pattern:
        if n not in graphs:
            s.wait_stream(torch.cuda.current_stream())
            g = torch.cuda.CUDAGraph()
            # capture without executing: the state must not move
            snap = (rnd.state.clone(), rnd.verdict.clone(), rnd.upd_out.clone(), rnd.upd_hid.clone(),
                    rnd.cache[0].keys.clone(), rnd.cache[0].values.clone(), tg.logits.clone())
            with torch.cuda.graph(g, stream=s):
                rnd.enqueue_draft()
                tg.plant(rnd.drafts, n)
                rnd.enqueue_verify(tg.logits)
                rnd.enqueue_commit(tg.taps)
                rnd.enqueue_readback()
            torch.cuda.synchronize()
            assert torch.equal(snap[0], rnd.state) and torch.equal(snap[4], rnd.cache[0].keys)
            graphs[n] = g
        graphs[n].replay()
        results.append(rnd.finish())
        _ = torch.ones(3, device=cuda).sum().item()  # eager work between replays
    for r, (a, b) in enumerate(zip(results, eager_res)):
        assert (a.n_accepted, a.tokens) == (b.n_accepted, b.tokens), f"replay {r}"
    assert torch.equal(rnd.cache[0].keys, eager_k)
    del n_agree


@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float32])
def test_pending_chain_equals_plain_chain(cuda, kv_dtype):
    """The chain with each head's argmax left pending for the next forward
    (wc_draft_head_norm_pending / wc_drafter_forward_pending) drafts the same
    tokens, hidden rows and drafter KV entries, bit for bit, as the chain of
    standalone heads and forwards; the workspace keys are clear afterwards, so a
    plain head can follow."""
    from woodcock_amd.config import qwen3_1p7b_drafter

    cfg = qwen3_1p7b_drafter()
    cfg, d, rnd, od, oc, target, root = setup(cuda, 11, ctx=300, kv_dtype=kv_dtype, cap=512, cfg=cfg,
                                              head_rows=4096, k=5)
    assert d.pending_ok
    c = rnd.cache[0]
    k0, v0 = c.keys.clone(), c.values.clone()

    def run(pending):
        c.keys.copy_(k0)
        c.values.copy_(v0)
        rnd.drafts.zero_()
        rnd.step_hid.zero_()
        rnd.pending = pending
        rnd.enqueue_draft()
        torch.cuda.synchronize()
        return rnd.drafts.clone(), rnd.step_hid.clone(), rnd.step_out.clone(), c.keys.clone(), c.values.clone()

    plain = run(False)
    pend = run(True)
    again = run(False)  # a plain chain right after the pending one: no stale keys in the workspace
    for a, b, name in zip(plain, pend, ("drafts", "step_hid", "step_out", "keys", "values")):
        assert torch.equal(a, b), name
    for a, b, name in zip(plain, again, ("drafts", "step_hid", "step_out", "keys", "values")):
        assert torch.equal(a, b), name
    assert len(set(plain[0].tolist())) > 1
    rnd.pending = True
