#!/usr/bin/env python3
"""µs per speculative-decoding round on one MI355X (Qwen3-1.7B drafter shape).

Workload (the greedy chain round at the Qwen3-1.7B drafter shape): random-init
bf16 drafter weights N(0, 0.02) (one decoder layer, 16 q / 8 kv heads, head_dim
128, SwiGLU 6144, fc 6144->2048), a 16384-row trimmed head with its d2t map into
the 151936-token vocabulary, drafter KV context 512 (bf16), chain length K=4,
greedy; synthetic target logits [5, 151936] fp32 ~ N(0, 3^2) whose argmax agrees
with the drafts at the first 2 positions; three target taps [5, 2048] bf16; a
28-layer target KV cache (8 kv heads x 128, bf16, context 2048 + 6) compacted
after acceptance.

A "step" is one round: K head+argmax launches, K-1 drafter layers, the fused
target argmax + accept, the target-KV compaction, the fc fusion + drafter update
over the a+1 accepted tokens, and the verdict copy for the round's single host
sync.  Every round starts from the same committed context (n = 512).

Timing: each piece is captured once as a HIP graph; per round the graphs are
replayed behind a short spin kernel (so host submission never shows as GPU idle)
with HIP events on the launch stream around our kernels.  The synthetic-target
stand-in (plant of the agreeing argmax) runs between the two timed graphs and
is reported separately, not in `value`.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

PEAK_HBM_GBS = 8000.0
BASE_CTX = 512
CTX4 = 4096  # drafter context of the Qwen3-4B-shape step
# algorithmic bytes of that step: head 16384 x 2560, the layer (QKV over the fed
# feature and the embedding, o, gate / up, down) and the KV at ctx 4096 + 1
STEP4_BYTES = 83_886_080 + 233_308_160 + 16_781_312
K = 4


_T0 = time.perf_counter()


def log(msg: str) -> None:
    """Progress on stderr (the JSON line stays the only stdout output)."""
    print(f"[bench {time.perf_counter() - _T0:6.1f}s] {msg}", file=sys.stderr, flush=True)


def _sleep_gate():
    import torch

    if hasattr(torch.cuda, "_sleep"):
        torch.cuda._sleep(200_000)


def gpu_time_graphs(graphs_timed, reps, between=None):
    """Replay `graphs_timed` (list of graphs) `reps` times; returns per-rep GPU µs."""
    import torch

    out = []
    for _ in range(reps):
        _sleep_gate()
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(2 * len(graphs_timed))]
        for i, g in enumerate(graphs_timed):
            evs[2 * i].record()
            g.replay()
            evs[2 * i + 1].record()
            if between is not None and i < len(graphs_timed) - 1:
                between[i].replay()
        torch.cuda.synchronize()
        out.append(1e3 * sum(evs[2 * i].elapsed_time(evs[2 * i + 1]) for i in range(len(graphs_timed))))
    return np.array(out)


def capture(fn):
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        fn()
    torch.cuda.synchronize()
    return g


def time_draft_step(d, cache, ctx, reps=32, samples=10, cold_samples=20, evict=None, pending=None):
    """The reference's draft-step unit (scripts/time_draft_step.py:51-56: the
    final norm, head + argmax, one drafter layer; KV rolled back) on drafter d
    at cache offset ctx.  Warm: a graph of `reps` steps replayed back to back
    (median over `samples` replays, per step).  Cold: one step between two
    events after `evict()` streamed 1 GiB (median over `cold_samples`), so the
    drafter's weights come from HBM.  pending (default: what the chain uses):
    the head's argmax is handed to the forward (wc_draft_head_norm_pending /
    wc_drafter_forward_pending)."""
    import ctypes as C

    import torch

    from woodcock_amd import _lib
    from woodcock_amd.runtime import ptr, stream_ptr

    dev = d.device
    dm = d.cfg.hidden_size
    if pending is None:
        pending = d.pending_ok
    dims, W, ws = C.byref(d.dims), C.byref(d.wstruct), ptr(d.ws)
    kp = (C.c_void_p * len(cache))(*[c.keys.data_ptr() for c in cache])
    vp = (C.c_void_p * len(cache))(*[c.values.data_ptr() for c in cache])
    kvdt = _lib.WC_BF16 if cache[0].keys.dtype == torch.bfloat16 else _lib.WC_F32
    g = torch.Generator(device=dev).manual_seed(7)
    hid = torch.randn(1, dm, generator=g, device=dev)
    out = torch.empty_like(hid)
    nxt = torch.empty_like(hid)
    tok = torch.zeros(1, dtype=torch.int32, device=dev)
    off = torch.tensor([ctx], dtype=torch.int32, device=dev)
    fb = out if d.cfg.post_norm else hid

    def one():
        # the layer leaves its final norm to the next head, as in the chain; with
        # pending, the head's argmax is resolved by the forward (the chain's path)
        if pending:
            _lib.call("wc_draft_head_norm_pending", dims, W, ptr(hid), dm, None, 0, ptr(out), dm, None, 0, None, ws,
                      stream_ptr())
            _lib.call("wc_drafter_forward_pending", dims, W, ptr(tok), None, ptr(fb), dm, None, 0, kp, vp, kvdt,
                      cache[0].capacity, ptr(off), 0, None, ptr(nxt), None, None, ws, stream_ptr())
            return
        _lib.call("wc_draft_head_norm", dims, W, ptr(hid), dm, None, 0, ptr(out), dm, None, 0, ptr(tok), None, None,
                  ws, stream_ptr())
        _lib.call("wc_drafter_forward", dims, W, ptr(tok), ptr(fb), dm, None, 0, 1, None, kp, vp, kvdt,
                  cache[0].capacity, ptr(off), 0, None, None, 0, ptr(nxt), None, None, ws, stream_ptr())

    def many():
        for _ in range(reps):
            one()

    many()
    torch.cuda.synchronize()
    gr = capture(many)
    res = {"warm_us": float(np.median(gpu_time_graphs([gr], samples))) / reps}
    if evict is not None:
        t = []
        for _ in range(cold_samples):
            evict()
            _sleep_gate()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            one()
            e1.record()
            torch.cuda.synchronize()
            t.append(1e3 * e0.elapsed_time(e1))
        res["cold_us"] = float(np.median(t))
    return res


def time_head(d, pending, reps=32, samples=10, cold_samples=20, evict=None):
    """The chain's draft head on its own (final norm + 16k-row head GEMV with
    argmax keys; pending: the keys stay in the workspace for the next forward,
    as in every chain step but the last) at one row.  Warm: a graph of `reps`
    launches (median over `samples` replays, per launch).  Cold: one launch
    between two events after `evict()` streamed 1 GiB, behind the spin gate
    (median over `cold_samples`).  A plain head launch afterwards clears the
    pending keys."""
    import ctypes as C

    import torch

    from woodcock_amd import _lib
    from woodcock_amd.runtime import ptr, stream_ptr

    dev = d.device
    dm = d.cfg.hidden_size
    dims, W, ws = C.byref(d.dims), C.byref(d.wstruct), ptr(d.ws)
    g = torch.Generator(device=dev).manual_seed(11)
    hid = torch.randn(1, dm, generator=g, device=dev)
    out = torch.empty_like(hid)
    tok = torch.zeros(1, dtype=torch.int32, device=dev)

    def plain():
        _lib.call("wc_draft_head_norm", dims, W, ptr(hid), dm, None, 0, ptr(out), dm, None, 0, ptr(tok), None, None,
                  ws, stream_ptr())

    def one():
        if pending:
            _lib.call("wc_draft_head_norm_pending", dims, W, ptr(hid), dm, None, 0, ptr(out), dm, None, 0, None, ws,
                      stream_ptr())
        else:
            plain()

    def many():
        for _ in range(reps):
            one()

    many()
    torch.cuda.synchronize()
    gr = capture(many)
    res = {"warm_us": float(np.median(gpu_time_graphs([gr], samples))) / reps}
    if evict is not None:
        t = []
        for _ in range(cold_samples):
            evict()
            _sleep_gate()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            one()
            e1.record()
            torch.cuda.synchronize()
            t.append(1e3 * e0.elapsed_time(e1))
        res["cold_us"] = float(np.median(t))
    if pending:
        plain()
        torch.cuda.synchronize()
    return res


def step_only(args):
    """Only the draft steps of configs 1 and 4, warm and cold; one JSON line."""
    import torch

    from woodcock_amd.config import QWEN3_EOS, qwen3_4b_drafter
    from woodcock_amd.drafter import Drafter
    from woodcock_amd.synthetic import draft_vocab, random_drafter

    cfg, d, ids, rnd, target, init_state, root = build_workload(args.seed)
    flush = torch.zeros(1 << 28, dtype=torch.float32, device=d.device)
    out = {}
    if args.step_config in ("1", "both"):
        out["config1_head"] = time_head(d, pending=d.pending_ok, evict=flush.sum)
        out["config1"] = time_draft_step(d, rnd.cache, BASE_CTX, evict=flush.sum)
        out["config1_plain_head"] = time_draft_step(d, rnd.cache, BASE_CTX, evict=flush.sum, pending=False)
    if args.step_config == "1":
        print(json.dumps({k: {n: round(v, 2) for n, v in t.items()} for k, t in out.items()}), flush=True)
        return
    cfg4 = qwen3_4b_drafter()
    d4 = Drafter(cfg4, random_drafter(cfg4, seed=args.seed + 7, device=d.device), d.device, torch.bfloat16)
    d4.restrict_vocab(draft_vocab(cfg4.vocab_size, 16384, seed=args.seed + 7, always=QWEN3_EOS))
    cache4 = d4.make_cache(CTX4 + 16)
    for c in cache4:
        c.keys.normal_()
        c.values.normal_()
    out["config4"] = time_draft_step(d4, cache4, CTX4, evict=flush.sum)
    out["config4_plain_head"] = time_draft_step(d4, cache4, CTX4, evict=flush.sum, pending=False)
    print(json.dumps({k: {n: round(v, 2) for n, v in t.items()} for k, t in out.items()}), flush=True)


def build_workload(seed=0):
    import torch

    from woodcock_amd.cache import make_cache
    from woodcock_amd.config import QWEN3_EOS, qwen3_1p7b_drafter
    from woodcock_amd.drafter import Drafter
    from woodcock_amd.spec import ChainRound
    from woodcock_amd.synthetic import SyntheticTarget, draft_vocab, random_drafter

    dev = torch.device("cuda", 0)
    cfg = qwen3_1p7b_drafter()
    w = random_drafter(cfg, seed=seed, device=dev)
    d = Drafter(cfg, w, dev, torch.bfloat16)
    ids = draft_vocab(cfg.vocab_size, 16384, seed=seed, always=QWEN3_EOS)
    d.restrict_vocab(ids)
    target_cache = make_cache(28, 8, 128, 2048 + 6, torch.bfloat16, dev)
    rnd = ChainRound(d, K, 1024, target_cache)
    g = torch.Generator(device=dev).manual_seed(seed + 1)
    for c in rnd.cache:
        c.keys[0, :, :BASE_CTX] = torch.randn(c.keys[0, :, :BASE_CTX].shape, generator=g, device=dev).bfloat16()
        c.values[0, :, :BASE_CTX] = torch.randn(c.values[0, :, :BASE_CTX].shape, generator=g, device=dev).bfloat16()
    root = torch.randn(1, cfg.hidden_size, generator=g, device=dev)  # pre-norm hidden state of the last entry
    rnd.set_root(BASE_CTX, root)
    target = SyntheticTarget(K, cfg.vocab_size, cfg.target_hidden_size, device=dev, seed=seed + 2)
    init_state = rnd.state.clone()
    return cfg, d, ids, rnd, target, init_state, root


def bench_gpu(args):
    import ctypes as C

    import torch

    from woodcock_amd import _lib
    from woodcock_amd.runtime import ptr, stream_ptr

    cfg, d, ids, rnd, target, init_state, root = build_workload(args.seed)

    def rewind():
        rnd.state.copy_(init_state)

    def plant():
        target.plant(rnd.drafts, 2)

    def commit():
        rnd.enqueue_verify_commit(target.logits, target.taps)
        rnd.enqueue_readback()

    # eager warm-up round (kernel attributes, allocator), then capture
    rewind()
    rnd.enqueue_draft()
    plant()
    commit()
    res = rnd.finish()
    g_rewind, g_draft, g_plant, g_commit = capture(rewind), capture(rnd.enqueue_draft), capture(plant), capture(commit)

    def one_round():
        g_rewind.replay()
        g_draft.replay()
        g_plant.replay()
        g_commit.replay()
        return rnd.finish()

    log("workload built; warm-up rounds")
    for _ in range(args.warmup):
        one_round()
    # host-observed latency: launch of the round to the verdict on the host (single sync)
    walls, accepted = [], []
    for _ in range(args.steps):
        g_rewind.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        g_draft.replay()
        g_plant.replay()
        g_commit.replay()
        r = rnd.finish()
        walls.append(1e6 * (time.perf_counter() - t0))
        accepted.append(r.n_accepted)
    # GPU time of our kernels per round (events), gated
    rounds_gpu = []
    plants = []
    t_begin = time.perf_counter()
    for _ in range(args.steps):
        g_rewind.replay()
        _sleep_gate()
        e = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
        e[0].record()
        g_draft.replay()
        e[1].record()
        g_plant.replay()
        e[2].record()
        g_commit.replay()
        e[3].record()
        r = rnd.finish()
        rounds_gpu.append(1e3 * (e[0].elapsed_time(e[1]) + e[2].elapsed_time(e[3])))
        plants.append(1e3 * e[1].elapsed_time(e[2]))
    t_timed = time.perf_counter() - t_begin
    assert set(accepted) == {2}, f"accepted lengths {set(accepted)}"
    log(f"{args.steps} timed rounds: median {np.median(rounds_gpu):.1f} us")
    if args.round_only:
        return {"round_gpu_us": float(np.median(rounds_gpu)), "timed_seconds": t_timed}

    # cold start: before each round 1 GiB is read, which evicts the drafter's
    # weights from the 256 MB Infinity Cache as the target forward between
    # rounds does in the product (a read leaves clean lines behind: no
    # write-back competes with the round); the read is outside the timed region
    flush = torch.zeros(1 << 28, dtype=torch.float32, device=rnd.cache[0].keys.device)

    def evict():
        flush.sum()

    cold = []
    for _ in range(max(10, args.steps // 10)):
        g_rewind.replay()
        evict()
        _sleep_gate()
        e = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
        e[0].record()
        g_draft.replay()
        e[1].record()
        g_plant.replay()
        e[2].record()
        g_commit.replay()
        e[3].record()
        rnd.finish()
        cold.append(1e3 * (e[0].elapsed_time(e[1]) + e[2].elapsed_time(e[3])))

    # ---- components, each a graph of REP launches
    REP = 32
    dims, W, ws, s = C.byref(d.dims), C.byref(d.wstruct), ptr(d.ws), stream_ptr
    dm = cfg.hidden_size
    hid1 = rnd.upd_hid[0:1]
    out1 = rnd.upd_out[0:1]
    tok = rnd.drafts[0:1]
    vlog = torch.randn(6, cfg.vocab_size, device=out1.device) * 3
    vdr = torch.randint(0, cfg.vocab_size, (5,), dtype=torch.int32, device=out1.device)
    vverd = torch.zeros(_lib.VERDICT_INTS, dtype=torch.int32, device=out1.device)

    def verifies():
        for _ in range(REP):
            _lib.call("wc_verify_chain_greedy", ptr(vlog), 6, cfg.vocab_size, vlog.stride(0), ptr(vdr), ptr(vverd),
                      ptr(rnd.vws), s())

    # tree-path compaction: keeps with a ~ U{0..5} over a 6-slot verify window at 2048
    rng = np.random.default_rng(args.seed)
    keeps = []
    for _ in range(REP):
        a = int(rng.integers(0, 6))
        keeps.append([0] + sorted(rng.choice(np.arange(1, 6), a, replace=False).tolist()))
    karr = torch.zeros(REP, 8, dtype=torch.int32)
    for i, kp in enumerate(keeps):
        karr[i, 0] = len(kp)
        karr[i, 1] = 2048
        karr[i, 2:2 + len(kp)] = torch.tensor(kp)
    karr = karr.to(out1.device)
    koff = torch.zeros(REP, dtype=torch.int32, device=out1.device)
    tc = rnd.target_cache
    kp_ = (C.c_void_p * len(tc))(*[c.keys.data_ptr() for c in tc])
    vp_ = (C.c_void_p * len(tc))(*[c.values.data_ptr() for c in tc])
    moved_rows = sum(sum(1 for i, k in enumerate(kp) if k != i) for kp in keeps)

    def compacts():
        for i in range(REP):
            _lib.call("wc_kv_compact", kp_, vp_, len(tc), 8, tc[0].capacity, 256, ptr(karr[i, 1:2]),
                      ptr(karr[i, 2:8]), ptr(karr[i, 0:1]), 6, ptr(koff[i:i + 1]), None, s())

    # stochastic accept/reject at k=5 -- target logits [6,151936] straight into the
    # rule; the draft softmax [5,16384] timed on its own
    from woodcock_amd.synthetic import draw_rows, stochastic_workload

    s_lg, s_dl, s_d2t = stochastic_workload(5, cfg.vocab_size, 16384, seed=args.seed + 5)
    s_tl = torch.from_numpy(s_lg).to(out1.device)
    s_dlg = torch.from_numpy(s_dl).to(out1.device)
    s_d2 = torch.from_numpy(s_d2t).to(out1.device)
    s_p = torch.empty_like(s_tl)
    s_q = torch.empty_like(s_dlg)
    from woodcock_amd.sampling import probs_from_logits as _probs

    _probs(s_dlg, 1.0, out=s_q)
    s_rows = draw_rows(s_q.cpu().numpy(), 1, np.random.default_rng(args.seed))[0]
    s_dr = torch.from_numpy(s_d2t[s_rows]).to(out1.device)
    s_round = torch.zeros(1, dtype=torch.int32, device=out1.device)
    s_u = _lib.Uniforms(args.seed, ptr(s_round), 0)
    s_verd = torch.zeros(_lib.VERDICT_INTS, dtype=torch.int32, device=out1.device)
    sws = ptr(rnd.vws)

    def draft_probs():
        # the draft distribution q, formed at draft time in a sampling round
        for _ in range(REP):
            _lib.call("wc_probs_from_logits", ptr(s_dlg), 5, s_dlg.shape[1], s_dlg.stride(0), 1.0, 0, 1.0, ptr(s_q),
                      s_q.stride(0), sws, s())

    def stochastic():
        # the verify step from the target logits: p = softmax(logits / T), accept
        # tests, residual draw (two launches, p never written)
        for _ in range(REP):
            _lib.call("wc_verify_chain_stochastic_logits", ptr(s_tl), 6, s_tl.shape[1], s_tl.stride(0), 1.0,
                      ptr(s_q), 16384, s_q.stride(0), ptr(s_d2), ptr(s_dr), None, C.byref(s_u), ptr(s_verd), sws,
                      s())

    # one Qwen3-1.7B target layer over a 60-node draft tree (depth <= 6) at context
    # 2048 with the tree mask, then the greedy tree verify over [60, 151936] logits
    from woodcock_amd.cache import KVCache
    from woodcock_amd.sampling import DraftTree
    from woodcock_amd.target import TargetConfig, TargetLayer, random_layer

    tcfg = TargetConfig()
    trng = np.random.default_rng(args.seed + 9)
    parents, depth = [-1], [0]
    while len(parents) < 60:
        p_ = int(trng.integers(0, len(parents)))
        if depth[p_] < 6:
            parents.append(p_)
            depth.append(depth[p_] + 1)
    tree = DraftTree([int(t) for t in trng.integers(0, cfg.vocab_size, 60)], parents, depth)
    tl = TargetLayer(tcfg, random_layer(tcfg, seed=args.seed, device=out1.device), out1.device, max_rows=60)
    tcache = KVCache(tcfg.num_kv_heads, tcfg.head_dim, 2048 + 64, torch.bfloat16, out1.device)
    tcache.keys.normal_()
    tcache.values.normal_()
    tx = torch.randn(60, tcfg.hidden_size, device=out1.device)
    toff = torch.tensor([2048], dtype=torch.int32, device=out1.device)
    tpos = torch.tensor([2048 + dd for dd in depth], dtype=torch.int32, device=out1.device)
    tmask = tree_mask_rows(tree, 2048, out1.device)
    tl(tx, tcache, toff, tpos, tmask)  # rope table, workspace touched before capture

    def target_layers():
        for _ in range(REP // 4):
            tl(tx, tcache, toff, tpos, tmask)

    tlog = torch.randn(60, cfg.vocab_size, device=out1.device) * 3
    ttok = torch.tensor(tree.tokens, dtype=torch.int32, device=out1.device)
    tpar = torch.tensor(tree.parents, dtype=torch.int32, device=out1.device)

    def tree_verifies():
        for _ in range(REP):
            _lib.call("wc_verify_tree_greedy", ptr(tlog), 60, cfg.vocab_size, tlog.stride(0), ptr(ttok), ptr(tpar),
                      ptr(vverd), ptr(rnd.vws), s())

    # the whole verify forward of a 28-layer Qwen3-1.7B target (random weights):
    # embedding, layers with the feature taps, final norm + tied head; the chain
    # block (5 rows, causal, context 512) and the 60-node tree block (context 2048)
    from woodcock_amd.target import TargetModel, random_target

    tm = TargetModel(tcfg, random_target(tcfg, seed=args.seed + 5, device=out1.device), out1.device, max_rows=60)
    tm_cache = tm.make_cache(2048 + 64)
    for c in tm_cache:
        c.keys.normal_()
        c.values.normal_()
        c.offset = 512  # the chain block's context (the tree block passes its own offset and mask)
    tm_tok5 = torch.randint(0, tcfg.vocab_size, (5,), dtype=torch.int32, device=out1.device)
    tm_tok60 = torch.tensor(tree.tokens, dtype=torch.int32, device=out1.device)
    tm_off512 = torch.tensor([512], dtype=torch.int32, device=out1.device)
    tm_logits = torch.empty(60, tcfg.vocab_size, device=out1.device)
    tm_taps = [torch.empty(60, tcfg.hidden_size, device=out1.device) for _ in tm.feature_layers]
    tm(tm_tok5, tm_cache, tm_off512, logits=tm_logits[:5], taps=tm_taps)

    def target_chain():
        tm(tm_tok5, tm_cache, tm_off512, logits=tm_logits[:5], taps=tm_taps)

    def target_tree():
        tm(tm_tok60, tm_cache, toff, tpos, tmask, logits=tm_logits, taps=tm_taps)

    # greedy tree drafting on the device at the config-5 shape: depth 6, width 4,
    # 59 verified nodes + root, drafter context 512 (six head + softmax + expand
    # levels, five frontier forwards of 4 rows, the verify-set selection)
    from woodcock_amd.tree_draft import TreeDrafter

    tdr = TreeDrafter(d, rnd.cache, 6, 4, 59)
    td_tok = torch.tensor([7], dtype=torch.int32, device=out1.device)
    td_off = torch.tensor([BASE_CTX], dtype=torch.int32, device=out1.device)
    td_root = torch.randn(cfg.hidden_size, device=out1.device)

    def tree_drafts():
        tdr.draft(td_tok, td_root, td_root, td_off)

    # config 4's draft step: Qwen3-4B drafter shape (hidden 2560, 32 / 8 heads,
    # intermediate 9728, fc 7680 -> 2560), 16k trimmed head, drafter ctx 4096
    from woodcock_amd.config import QWEN3_EOS, qwen3_4b_drafter
    from woodcock_amd.drafter import Drafter
    from woodcock_amd.synthetic import draft_vocab, random_drafter

    cfg4 = qwen3_4b_drafter()
    d4 = Drafter(cfg4, random_drafter(cfg4, seed=args.seed + 7, device=out1.device), out1.device, torch.bfloat16)
    d4.restrict_vocab(draft_vocab(cfg4.vocab_size, 16384, seed=args.seed + 7, always=QWEN3_EOS))
    cache4 = d4.make_cache(CTX4 + 16)
    g4 = torch.Generator(device=out1.device).manual_seed(args.seed + 8)
    for c in cache4:
        c.keys[0, :, :CTX4] = torch.randn(c.keys[0, :, :CTX4].shape, generator=g4, device=out1.device).bfloat16()
        c.values[0, :, :CTX4] = torch.randn(c.values[0, :, :CTX4].shape, generator=g4, device=out1.device).bfloat16()
    log("cold rounds done; component graphs")
    comps = {}
    reps = {"target_layer": REP // 4, "target_chain": 1, "target_tree": 1, "tree_draft": 1}
    for name, fn in (("verify", verifies), ("compact", compacts),
                     ("draft_probs", draft_probs), ("stochastic", stochastic), ("target_layer", target_layers), ("tree_verify", tree_verifies),
                     ("target_chain", target_chain), ("target_tree", target_tree), ("tree_draft", tree_drafts)):
        fn()
        torch.cuda.synchronize()
        g = capture(fn)
        t = gpu_time_graphs([g], max(5, args.steps // 10))
        comps[name] = float(np.median(t)) / reps.get(name, REP)
    rewind()
    torch.cuda.synchronize()
    # the chain's head and draft step (pending argmax hand-over), warm and cold
    # (each cold sample after the 1 GiB read, one launch or step between events)
    head = time_head(d, pending=d.pending_ok, evict=evict)
    head_plain = time_head(d, pending=False, evict=None)
    step = time_draft_step(d, rnd.cache, BASE_CTX, evict=evict)
    step4 = time_draft_step(d4, cache4, CTX4, evict=evict)
    rewind()
    torch.cuda.synchronize()
    del flush
    torch.cuda.empty_cache()
    log("components done; config-4 round loop")
    c4 = bench_config4(args, d4)
    log(f"config-4: mean K {c4['mean_k']:.2f}, {c4['round_us']:.1f} us per round; config-5 tree rounds")
    c5 = bench_tree_round(args, d, tm, tcfg)
    log(f"config-5 tree round {c5['round_us']:.1f} us")

    head_bytes = 16384 * cfg.hidden_size * 2
    layer_bytes = 2 * (cfg.num_heads + 2 * cfg.num_kv_heads) * cfg.head_dim * dm * 2 + \
        dm * cfg.num_heads * cfg.head_dim * 2 + 3 * cfg.intermediate_size * dm * 2
    kv_bytes = (BASE_CTX + 1) * cfg.num_kv_heads * cfg.head_dim * 2 * 2
    step_bytes = head_bytes + layer_bytes + kv_bytes
    compact_bytes = 2 * 28 * 2 * 8 * 256 * moved_rows / REP  # read + write of moved rows
    return {
        "round_gpu_us": float(np.median(rounds_gpu)),
        "round_gpu_us_mean": float(np.mean(rounds_gpu)),
        "round_wall_us": float(np.median(walls)),
        "target_standin_us": float(np.median(plants)),
        "draft_step_us": step["warm_us"],
        "draft_step_us_cold": step["cold_us"],
        "head_us": head["warm_us"],
        "head_us_cold": head["cold_us"],
        "head_plain_us": head_plain["warm_us"],
        "verify_accept_us": comps["verify"],
        "kv_compact_us": comps["compact"],
        "stochastic_us": comps["stochastic"],
        "draft_probs_us": comps["draft_probs"],
        "target_layer_us": comps["target_layer"],
        "tree_verify_us": comps["tree_verify"],
        "target_chain_us": comps["target_chain"],
        "target_tree_us": comps["target_tree"],
        "tree_draft_us": comps["tree_draft"],
        "draft_step_4b_us": step4["warm_us"],
        "draft_step_4b_us_cold": step4["cold_us"],
        "round_gpu_us_cold": float(np.median(cold)),
        "config4": c4,
        "config5": c5,
        "head_bytes": head_bytes,
        "step_bytes": step_bytes,
        "compact_bytes_avg": compact_bytes,
        "accepted": 2,
        "timed_seconds": t_timed,
        "weights": d,
        "ids": ids,
        "root": root,
        "rnd": rnd,
        "target": target,
    }


def bench_config4(args, d4):
    """Auto chain length at the Qwen3-4B drafter shape (drafter context 4096):
    the round loop (SpeculativeDecoder) with CostAwareChain, whose costs are
    measured here -- head and draft step of this drafter, the verify forward
    of a random-init Qwen3-4B-shape target (36 layers) over 1..9 rows -- and
    a synthetic target whose draft positions agree with probability 0.68.
    GPU µs per round exclude the synthetic stand-in (planting the agreement)."""
    import torch

    from woodcock_amd.costs import time_drafter, time_verify
    from woodcock_amd.policies import CostAwareChain
    from woodcock_amd.spec import SpeculativeDecoder
    from woodcock_amd.synthetic import SyntheticTarget
    from woodcock_amd.target import TargetConfig, TargetModel, random_target

    dev = d4.device
    t_d = time_drafter(d4, CTX4, iters=20)
    tcfg4 = TargetConfig(hidden_size=2560, num_heads=32, num_kv_heads=8, head_dim=128, intermediate_size=9728,
                         num_layers=36)
    tm4 = TargetModel(tcfg4, random_target(tcfg4, seed=args.seed + 11, device=dev), dev, max_rows=16)
    verify = time_verify(tm4, CTX4, 9, iters=5)
    del tm4
    torch.cuda.empty_cache()
    policy = CostAwareChain(t_d["step_ms"], t_d["head_ms"], verify)
    syn = SyntheticTarget(8, d4.cfg.vocab_size, d4.cfg.target_hidden_size, device=dev, seed=args.seed + 12,
                          agree_p=0.68)
    warm, rounds = 24, max(40, args.steps // 2)
    dec = SpeculativeDecoder(d4, syn, policy, capacity=CTX4 + 16 + 9 * (warm + rounds), k_max=8, use_graphs=True,
                             timing=True)
    g = torch.Generator(device=dev).manual_seed(args.seed + 13)
    for c in dec.rnd.cache:
        c.keys[0, :, :CTX4] = torch.randn(c.keys[0, :, :CTX4].shape, generator=g, device=dev).bfloat16()
        c.values[0, :, :CTX4] = torch.randn(c.values[0, :, :CTX4].shape, generator=g, device=dev).bfloat16()
    dec.start(CTX4, 151643, torch.randn(1, d4.cfg.hidden_size, generator=g, device=dev))
    for _ in range(warm):  # every length seen here is captured after its first eager round
        dec.round()
    us, ks, acc, full = [], [], [], []
    for _ in range(rounds):
        _sleep_gate()
        res = dec.round()
        t = dec.last_times
        us.append(t["round_us"])
        ks.append(res.k)
        acc.append(res.n_accepted)
        full.append(t["round_us"] + 1e3 * verify[res.k + 1])
    return {"round_us": float(np.mean(us)), "round_us_median": float(np.median(us)), "mean_k": float(np.mean(ks)),
            "k_hist": {int(k): int(n) for k, n in zip(*np.unique(ks, return_counts=True))},
            "mean_accepted": float(np.mean(acc)), "rounds": rounds,
            "head_ms": t_d["head_ms"], "step_ms": t_d["step_ms"],
            "verify_ms_qwen3_4b_36l": {int(n): round(v, 4) for n, v in verify.items()},
            "round_us_incl_target_forward": float(np.mean(full)),
            "tokens_per_s_incl_target_forward": float((np.mean(acc) + 1) / (np.mean(full) * 1e-6))}


def bench_tree_round(args, d, tm, tcfg):
    """The config-5 tree round through the round loop: greedy tree drafting
    (depth 6, width 4, 60 verified rows) at drafter context 2048, the 28-layer
    Qwen3-1.7B target forward over the tree block (tree mask, context 2048),
    the tree walk, the target KV compaction along the accepted branch and the
    drafter update; one host sync.  Per-phase GPU µs from events."""
    import torch

    from woodcock_amd.policies import StaticPolicy
    from woodcock_amd.spec import SpeculativeDecoder, TargetRunner

    dev = d.device
    ctx, rounds = 2048, 12
    cap = ctx + 64 + 8 * (rounds + 3)
    tcache = tm.make_cache(cap)
    for c in tcache:
        c.keys.normal_()
        c.values.normal_()
    dec = SpeculativeDecoder(d, TargetRunner(tm, tcache), StaticPolicy(6, 4, 59), capacity=cap, k_max=4,
                             max_tree_depth=6, timing=True)
    g = torch.Generator(device=dev).manual_seed(args.seed + 21)
    for c in dec.rnd.cache:
        c.keys[0, :, :ctx] = torch.randn(c.keys[0, :, :ctx].shape, generator=g, device=dev).bfloat16()
        c.values[0, :, :ctx] = torch.randn(c.values[0, :, :ctx].shape, generator=g, device=dev).bfloat16()
    dec.start(ctx, 151643, torch.randn(1, d.cfg.hidden_size, generator=g, device=dev))
    for _ in range(3):
        dec.round()
    ph = {"draft_us": [], "target_us": [], "verify_commit_us": []}
    for _ in range(rounds):
        if hasattr(torch.cuda, "_sleep"):
            torch.cuda._sleep(4_000_000)  # the host enqueues the whole round before the GPU reaches it
        dec.round()
        for k in ph:
            ph[k].append(dec.last_times[k])
    out = {k: float(np.median(v)) for k, v in ph.items()}
    out["round_us"] = out["draft_us"] + out["target_us"] + out["verify_commit_us"]
    out["round_us_excl_target_forward"] = out["draft_us"] + out["verify_commit_us"]
    out["rounds"] = rounds
    del tcache, dec
    torch.cuda.empty_cache()
    return out


# ---------------------------------------------------------------- HBM traffic
# The head GEMV's HBM bytes per launch come from two rocprofv3 counter passes
# over `bench.py --pmc-probe` (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch),
# each scaled by what the same counter reads for a plain copy kernel of known
# size run in the same process.  `bench.py --pmc-summary FETCH_DIR WRITE_DIR`
# turns the two counter CSVs into the committed summary that later runs read.
HEAD_KERNEL = "k_gemv1s<2, false, 1, 4, 0, 1>"
PROBE_HEADS = 16
PROBE_COPIES = 4
PROBE_COPY_FLOATS = 64 << 20  # 256 MiB read + 256 MiB written per copy
TRAFFIC_SUMMARY = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                               "draft_head_gemv_16384x2048_hbm_traffic.md")


def pmc_probe(seed=0):
    """Launch only what the counter passes read: PROBE_HEADS head launches of the
    benchmark workload, then PROBE_COPIES copies (torch.neg, fp32) of known size."""
    import ctypes as C

    import torch

    from woodcock_amd import _lib
    from woodcock_amd.runtime import ptr, stream_ptr

    cfg, d, ids, rnd, target, init_state, root = build_workload(seed)
    dims, W, ws = C.byref(d.dims), C.byref(d.wstruct), ptr(d.ws)
    dm = cfg.hidden_size
    x = torch.randn(PROBE_COPY_FLOATS, device="cuda")
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    for _ in range(PROBE_HEADS):
        _lib.call("wc_draft_head_norm", dims, W, ptr(rnd.upd_hid[0:1]), dm, None, 0, ptr(rnd.upd_out[0:1]), dm,
                  None, 0, ptr(rnd.drafts[0:1]), None, None, ws, stream_ptr())
    torch.cuda.synchronize()
    for _ in range(PROBE_COPIES):
        torch.neg(x, out=y)
    torch.cuda.synchronize()
    print(f"pmc probe: {PROBE_HEADS} head launches, {PROBE_COPIES} copies of {4 * PROBE_COPY_FLOATS} bytes",
          flush=True)


# Counter probe over the round's kernels: phases separated by a one-element
# torch.abs marker -- heads, draft-step layers (M = 1), update passes (verify +
# fuse, then the layer at 5 rows, 3 live), verify-width target layers (M = 60,
# tree mask) --
# then the calibration copies.  Per launch of each phase the same kernels run
# in the same order, so dispatch j of a repeat is one kernel (the table below
# names it and gives its algorithmic bytes).
PROBE_REPS = 8
_D, _HKV, _F, _HD = 2048, 8, 6144, 2048  # Qwen3-1.7B drafter: hidden, kv heads, intermediate, q width
PHASES = {
    "head": [("head GEMV + argmax 16384 x 2048", 16384 * _D * 2)],
    "draft layer (M = 1, ctx 512)": [
        ("QKV, two streams, 4096 x (2048 + 2048)", 2 * (_HD + 2 * _HKV * 128) * _D * 2),
        ("decode attention, 513 keys", 2 * 513 * _HKV * 128 * 2),
        ("o_proj + residual 2048 x 2048", _D * _HD * 2),
        ("gate / up + SiLU 2 x 6144 x 2048", 2 * _F * _D * 2),
        ("down + residual 2048 x 6144", _D * _F * 2)],
    "update pass (5 rows, 3 live)": [
        ("greedy verify of [5, 151936] fp32 logits + fuse 2048 x 6144, one launch", 5 * 151936 * 4 + _D * 3 * _D * 2),
        ("QKV, two streams", 2 * (_HD + 2 * _HKV * 128) * _D * 2),
        ("attention, 3 rows (row groups, merged in the launch)", 2 * 515 * _HKV * 128 * 2),
        ("o_proj", _D * _HD * 2),
        ("gate / up", 2 * _F * _D * 2),
        ("down", _D * _F * 2)],
    "target layer (M = 60, ctx 2048, tree mask)": [
        ("input -> fragment-order bf16 hi / lo", 60 * _D * 4 + 60 * _D * 4),
        ("QKV 4096 x 2048, K split", (_HD + 2 * _HKV * 128) * _D * 2),
        ("QKV fix-up (+ q/k norm, RoPE, K/V append)", 0),
        ("tree attention, 2048 + 60 keys, 16-byte mask rows", 2 * 2108 * _HKV * 128 * 2),
        ("attention merge (11 splits)", 0),
        ("o_proj 2048 x 2048, K split", _D * _HD * 2),
        ("o_proj fix-up (+ residual, next activations)", 0),
        ("gate / up 2 x 6144 x 2048, K unsplit, SiLU * up and next activations in the block", 2 * _F * _D * 2),
        ("down 2048 x 6144, K split", _D * _F * 2),
        ("down fix-up (+ residual)", 0)],
}


def pmc_probe2(seed=0):
    """The launches of the counter passes over the round's kernels (see PHASES)."""
    import ctypes as C

    import torch

    from woodcock_amd import _lib
    from woodcock_amd.cache import KVCache
    from woodcock_amd.runtime import ptr, stream_ptr
    from woodcock_amd.sampling import DraftTree
    from woodcock_amd.target import TargetConfig, TargetLayer, random_layer

    cfg, d, ids, rnd, target, init_state, root = build_workload(seed)
    dev = rnd.cache[0].keys.device
    dims, W, ws = C.byref(d.dims), C.byref(d.wstruct), ptr(d.ws)
    dm = cfg.hidden_size
    mark = torch.zeros(1, device=dev)
    tcfg = TargetConfig()
    trng = np.random.default_rng(seed + 9)
    parents, depth = [-1], [0]
    while len(parents) < 60:
        p_ = int(trng.integers(0, len(parents)))
        if depth[p_] < 6:
            parents.append(p_)
            depth.append(depth[p_] + 1)
    tree = DraftTree([int(t) for t in trng.integers(0, cfg.vocab_size, 60)], parents, depth)
    tl = TargetLayer(tcfg, random_layer(tcfg, seed=seed, device=dev), dev, max_rows=60)
    tcache = KVCache(tcfg.num_kv_heads, tcfg.head_dim, 2048 + 64, torch.bfloat16, dev)
    tx = torch.randn(60, tcfg.hidden_size, device=dev)
    toff = torch.tensor([2048], dtype=torch.int32, device=dev)
    tpos = torch.tensor([2048 + dd for dd in depth], dtype=torch.int32, device=dev)
    tmask = tree_mask_rows(tree, 2048, dev)
    off = init_state[0:1]
    hid_s = torch.empty(1, dm, device=dev)
    x = torch.randn(PROBE_COPY_FLOATS, device=dev)
    y = torch.empty_like(x)
    rows = torch.tensor([3], dtype=torch.int32, device=dev)
    tp = (C.c_void_p * 3)(*[t.data_ptr() for t in target.taps])
    g = torch.empty(5, dm, device=dev)
    hid5 = torch.empty(5, dm, device=dev)
    tl(tx, tcache, toff, tpos, tmask)
    torch.cuda.synchronize()
    s = stream_ptr()
    torch.abs(mark, out=mark)
    for _ in range(PROBE_REPS):
        _lib.call("wc_draft_head_norm", dims, W, ptr(rnd.upd_hid[0:1]), dm, None, 0, ptr(rnd.upd_out[0:1]), dm,
                  None, 0, ptr(rnd.drafts[0:1]), None, None, ws, s)
    torch.abs(mark, out=mark)
    for _ in range(PROBE_REPS):
        _lib.call("wc_drafter_forward", dims, W, ptr(rnd.drafts[0:1]), ptr(rnd.upd_out[0:1]), dm, None, 0, 1, None,
                  rnd._kp, rnd._vp, rnd._kvdt, rnd.cache[0].capacity, ptr(off), 0, None, None, 0, ptr(hid_s), None,
                  None, ws, s)
    torch.abs(mark, out=mark)
    for _ in range(PROBE_REPS):
        _lib.call("wc_verify_chain_greedy_fuse", ptr(target.logits), 5, target.logits.shape[1],
                  target.logits.stride(0), ptr(rnd.drafts), ptr(rnd.verdict), ptr(rnd.vws), dims, W, tp, _lib.WC_BF16,
                  target.taps[0].stride(0), ptr(g), dm, ws, s)
        _lib.call("wc_drafter_forward", dims, W, ptr(rnd.seq), ptr(g), dm, None, 0, 5, ptr(rows), rnd._kp, rnd._vp,
                  rnd._kvdt, rnd.cache[0].capacity, ptr(off), 0, None, None, 0, ptr(hid5), None, None, ws, s)
    torch.abs(mark, out=mark)
    for _ in range(PROBE_REPS // 2):
        tl(tx, tcache, toff, tpos, tmask)
    torch.abs(mark, out=mark)
    torch.cuda.synchronize()
    for _ in range(PROBE_COPIES):
        torch.neg(x, out=y)
    torch.cuda.synchronize()
    print(f"pmc probe over the round kernels: {PROBE_REPS} repeats per phase, {PROBE_COPIES} copies", flush=True)


def target_chain_only(seed=0, calls=20):
    """The 28-layer Qwen3-1.7B target forward over a 5-row chain block at
    context 512 (the few-row path), called `calls` times (for a kernel trace)."""
    import torch

    from woodcock_amd.target import TargetConfig, TargetModel, random_target

    dev = torch.device("cuda", 0)
    tcfg = TargetConfig()
    tm = TargetModel(tcfg, random_target(tcfg, seed=seed + 5, device=dev), dev, max_rows=8)
    cache = tm.make_cache(2048 + 64)
    for c in cache:
        c.keys.normal_()
        c.values.normal_()
        c.offset = 512
    tok = torch.randint(0, tcfg.vocab_size, (5,), dtype=torch.int32, device=dev)
    off = torch.tensor([512], dtype=torch.int32, device=dev)
    logits = torch.empty(5, tcfg.vocab_size, device=dev)
    taps = [torch.empty(5, tcfg.hidden_size, device=dev) for _ in tm.feature_layers]
    for _ in range(calls):
        tm(tok, cache, off, logits=logits, taps=taps)
    torch.cuda.synchronize()
    print(json.dumps({"target_chain_calls": calls}), flush=True)


def target_verify_only(seed=0, calls=10, rows=8):
    """The 36-layer Qwen3-4B-shape target forward over an 8-row verify block at
    context 4096 (more query vectors than the few-row path takes, so the
    verify-width GEMMs and the tree attention run), called `calls` times (for
    a kernel trace)."""
    import torch

    from woodcock_amd.target import TargetConfig, TargetModel, random_target

    dev = torch.device("cuda", 0)
    tcfg = TargetConfig(hidden_size=2560, num_heads=32, num_kv_heads=8, head_dim=128, intermediate_size=9728,
                        num_layers=36)
    tm = TargetModel(tcfg, random_target(tcfg, seed=seed + 11, device=dev), dev, max_rows=16)
    cache = tm.make_cache(CTX4 + 32)
    for c in cache:
        c.keys[0, :, :CTX4].normal_()
        c.values[0, :, :CTX4].normal_()
        c.offset = CTX4
    tok = torch.randint(0, tcfg.vocab_size, (rows,), dtype=torch.int32, device=dev)
    off = torch.tensor([CTX4], dtype=torch.int32, device=dev)
    logits = torch.empty(rows, tcfg.vocab_size, device=dev)
    taps = [torch.empty(rows, tcfg.hidden_size, device=dev) for _ in tm.feature_layers]
    tm(tok, cache, off, logits=logits, taps=taps)  # weight layout and first-call set-up outside the timed calls
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(calls):
        tm(tok, cache, off, logits=logits, taps=taps)
    e1.record()
    torch.cuda.synchronize()
    print(json.dumps({"target_verify_calls": calls, "rows": rows, "ctx": CTX4,
                      "ms_per_forward": round(e0.elapsed_time(e1) / calls, 4)}), flush=True)


def tree_mask_rows(tree, prefix, device):
    """The tree attention mask [N, prefix + N] as a row view of a buffer whose
    rows are padded to 16 bytes -- the layout the tree round's mask buffer has."""
    import torch

    from woodcock_amd.sampling import tree_attention_mask

    m = torch.from_numpy(tree_attention_mask(tree, prefix).astype(np.uint8))
    buf = torch.zeros(m.shape[0], (m.shape[1] + 15) // 16 * 16, dtype=torch.uint8, device=device)
    buf[:, : m.shape[1]] = m.to(device)
    return buf[:, : m.shape[1]]


def target_layer_only(seed=0, calls=45):
    """The config-5 target layer alone (Qwen3-1.7B shape, a 60-node tree of depth
    <= 6 at context 2048 with its mask, bf16 KV), called `calls` times."""
    import torch

    from woodcock_amd.cache import KVCache
    from woodcock_amd.sampling import DraftTree
    from woodcock_amd.target import TargetConfig, TargetLayer, random_layer

    dev = torch.device("cuda", 0)
    tcfg = TargetConfig()
    trng = np.random.default_rng(seed + 9)
    parents, depth = [-1], [0]
    while len(parents) < 60:
        p_ = int(trng.integers(0, len(parents)))
        if depth[p_] < 6:
            parents.append(p_)
            depth.append(depth[p_] + 1)
    tree = DraftTree([int(t) for t in trng.integers(0, tcfg.vocab_size, 60)], parents, depth)
    tl = TargetLayer(tcfg, random_layer(tcfg, seed=seed, device=dev), dev, max_rows=60)
    tcache = KVCache(tcfg.num_kv_heads, tcfg.head_dim, 2048 + 64, torch.bfloat16, dev)
    tcache.keys.normal_()
    tcache.values.normal_()
    tx = torch.randn(60, tcfg.hidden_size, device=dev)
    toff = torch.tensor([2048], dtype=torch.int32, device=dev)
    tpos = torch.tensor([2048 + dd for dd in depth], dtype=torch.int32, device=dev)
    tmask = tree_mask_rows(tree, 2048, dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(calls):
        tl(tx, tcache, toff, tpos, tmask)
    e1.record()
    torch.cuda.synchronize()
    print(json.dumps({"target_layer_us": round(1e3 * e0.elapsed_time(e1) / calls, 2), "calls": calls}), flush=True)


def pmc_summary2(fetch_dir, write_dir, mfma_dir):
    """Per-kernel HBM bytes (FETCH_SIZE + WRITE_SIZE, copy-calibrated) and MFMA
    busy (SQ_VALU_MFMA_BUSY_CYCLES over 1024 SIMDs / (GRBM_GUI_ACTIVE per XCD),
    the MfmaUtil metric) of the pmc_probe2 phases, as a markdown table."""
    copy_bytes = 4 * PROBE_COPY_FLOATS

    def phases(d, counter):
        disp = _per_dispatch(_counter_rows(d), counter)
        order = sorted(disp)
        names = [disp[i][0] for i in order]
        vals = [disp[i][1] for i in order]
        marks = [i for i, n in enumerate(names) if "abs" in n.lower() and "kernel" in n.lower()]
        if len(marks) != 5:
            raise SystemExit(f"{counter}: expected 5 phase markers, found {len(marks)}")
        copies = [v for n, v in zip(names[marks[-1] + 1:], vals[marks[-1] + 1:]) if "neg" in n.lower()]
        out = []
        for a, b in zip(marks, marks[1:]):
            out.append(list(zip(names[a + 1:b], vals[a + 1:b])))
        return out, (float(np.mean(copies)) if copies else None)

    fetch, fcopy = phases(fetch_dir, "FETCH_SIZE")
    write, wcopy = phases(write_dir, "WRITE_SIZE")
    busy, _ = phases(mfma_dir, "SQ_VALU_MFMA_BUSY_CYCLES")
    gui, _ = phases(mfma_dir, "GRBM_GUI_ACTIVE")
    ff, wf = copy_bytes / (fcopy * 1024.0), copy_bytes / (wcopy * 1024.0)
    lines = [f"Calibration: a {copy_bytes >> 20} MiB copy reads {fcopy:.0f} KiB by FETCH_SIZE (scale {ff:.4f}) and "
             f"writes {wcopy:.0f} KiB by WRITE_SIZE (scale {wf:.4f}).", "",
             "| Phase | Kernel | Work | Algorithmic bytes | HBM bytes (fetch + write) | ratio | MFMA busy % |",
             "|---|---|---|---:|---:|---:|---:|"]
    for (title, table), F, Wr, B, G in zip(PHASES.items(), fetch, write, busy, gui):
        per = len(table)
        reps = len(F) // per
        for j in range(per):
            idx = [j + r * per for r in range(reps) if j + r * per < len(F)]
            name = F[idx[0]][0]
            short = name if len(name) < 60 else name[:57] + "..."
            fb = np.mean([F[i][1] for i in idx]) * 1024.0 * ff
            wb = np.mean([Wr[i][1] for i in idx]) * 1024.0 * wf
            # the CSV's GRBM_GUI_ACTIVE is summed over the 8 XCDs; MFMA busy cycles over the 1024 SIMDs
            util = 100.0 * np.mean([B[i][1] for i in idx]) / max(np.mean([G[i][1] for i in idx]) / 8.0 * 1024.0, 1.0)
            work, algo = table[j]
            ratio = f"{(fb + wb) / algo:.3f}" if algo else ""
            lines.append(f"| {title} | `{short}` | {work} | {algo or ''} | {fb + wb:.0f} | {ratio} | {util:.1f} |")
    print("\n".join(lines))


def pmc_valu_summary(valu_dir):
    """VALU busy per launch of the pmc_probe2 phases: 100 x SQ_ACTIVE_INST_VALU x 4
    cycles / 1024 SIMDs / (GRBM_GUI_ACTIVE / 8 XCDs), as a markdown table."""
    def phases(counter):
        disp = _per_dispatch(_counter_rows(valu_dir), counter)
        order = sorted(disp)
        names = [disp[i][0] for i in order]
        vals = [disp[i][1] for i in order]
        marks = [i for i, n in enumerate(names) if "abs" in n.lower() and "kernel" in n.lower()]
        if len(marks) != 5:
            raise SystemExit(f"{counter}: expected 5 phase markers, found {len(marks)}")
        return [list(zip(names[a + 1:b], vals[a + 1:b])) for a, b in zip(marks, marks[1:])]

    valu, gui = phases("SQ_ACTIVE_INST_VALU"), phases("GRBM_GUI_ACTIVE")
    lines = ["| Phase | Kernel | Work | VALU busy % |", "|---|---|---|---:|"]
    for (title, table), V, G in zip(PHASES.items(), valu, gui):
        per = len(table)
        reps = len(V) // per
        for j in range(per):
            idx = [j + r * per for r in range(reps) if j + r * per < len(V)]
            name = V[idx[0]][0]
            short = name if len(name) < 60 else name[:57] + "..."
            busy = 100.0 * 4.0 * np.mean([V[i][1] for i in idx]) / 1024.0 / max(np.mean([G[i][1] for i in idx]) / 8.0, 1.0)
            lines.append(f"| {title} | `{short}` | {table[j][0]} | {busy:.1f} |")
    print("\n".join(lines))


def _counter_rows(d):
    import csv
    import glob

    files = sorted(glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True))
    if not files:
        raise SystemExit(f"no *counter_collection.csv under {d}")
    with open(files[0], newline="") as f:
        return list(csv.DictReader(f))


def _per_dispatch(rows, counter):
    """{dispatch id: (kernel name, value)} for one counter (summed over its instances)."""
    out = {}
    for r in rows:
        if r["Counter_Name"] != counter:
            continue
        did = int(r["Dispatch_Id"])
        name, v = out.get(did, (r["Kernel_Name"], 0.0))
        out[did] = (name, v + float(r["Counter_Value"]))
    return out


def pmc_summary(fetch_dir, write_dir):
    """Markdown summary of the two counter passes (printed; commit it under profiles/)."""
    copy_bytes = 4 * PROBE_COPY_FLOATS
    res = {}
    for counter, d in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        disp = _per_dispatch(_counter_rows(d), counter)
        order = sorted(disp)
        head = [disp[i][1] for i in order if HEAD_KERNEL in disp[i][0]]
        copies = [disp[i] for i in order[-PROBE_COPIES:]]
        if len(head) != PROBE_HEADS or any("neg" not in n for n, _ in copies):
            raise SystemExit(f"{counter}: expected {PROBE_HEADS} head dispatches and {PROBE_COPIES} trailing neg "
                             f"copies, got {len(head)} / {[n[:60] for n, _ in copies]}")
        copy_kib = float(np.mean([v for _, v in copies]))
        factor = copy_bytes / (copy_kib * 1024.0)
        res[counter] = (float(np.mean(head)), copy_kib, factor)
    fetch = res["FETCH_SIZE"][0] * 1024.0 * res["FETCH_SIZE"][2]
    write = res["WRITE_SIZE"][0] * 1024.0 * res["WRITE_SIZE"][2]
    algo = 16384 * 2048 * 2 + 2048 * 4 + 2048 * 2
    lines = [
        "# Draft head GEMV + argmax (16384 x 2048 bf16): HBM traffic per launch",
        "",
        "Commands (from the repository root on the GPU host):",
        "",
        "```",
        "cd /tmp && export TMPDIR=/tmp",
        "timeout -s KILL 90 rocprofv3 --pmc FETCH_SIZE --output-format csv -d $R/gpurun_out/pmc_fetch -o pmc "
        "-- python3 $R/bench.py --pmc-probe",
        "timeout -s KILL 90 rocprofv3 --pmc WRITE_SIZE --output-format csv -d $R/gpurun_out/pmc_write -o pmc "
        "-- python3 $R/bench.py --pmc-probe",
        "python3 bench.py --pmc-summary gpurun_out/pmc_fetch gpurun_out/pmc_write",
        "```",
        "",
        f"Probe: {PROBE_HEADS} launches of `{HEAD_KERNEL}` (the draft head with the fused final norm), then "
        f"{PROBE_COPIES} launches of torch.neg over {copy_bytes >> 20} MiB fp32 (reads and writes {copy_bytes} "
        "bytes each) as the calibration copy.",
        "",
        "| counter | head, KiB/dispatch (mean) | copy, KiB/dispatch (mean) | scale (copy bytes / counter bytes) "
        "| head bytes/launch |",
        "|---|---|---|---|---|",
        f"| FETCH_SIZE | {res['FETCH_SIZE'][0]:.1f} | {res['FETCH_SIZE'][1]:.1f} | {res['FETCH_SIZE'][2]:.4f} "
        f"| {fetch:.0f} |",
        f"| WRITE_SIZE | {res['WRITE_SIZE'][0]:.1f} | {res['WRITE_SIZE'][1]:.1f} | {res['WRITE_SIZE'][2]:.4f} "
        f"| {write:.0f} |",
        "",
        f"Algorithmic bytes per launch: {algo} (head weights 16384 x 2048 bf16, the fp32 input row, the final-norm "
        f"gain); measured / algorithmic = {(fetch + write) / algo:.4f}.",
        "",
        f"traffic_bytes_per_launch: {fetch + write:.0f}",
        "",
    ]
    print("\n".join(lines))


def forward_trace_summary(trace_dir: str, calls: int = 10) -> None:
    """Markdown table of the timed target forwards of `bench.py
    --target-verify-only` from a rocprofv3 kernel trace: every dispatch from the
    second embedding launch on (the first forward is the untimed set-up call),
    per forward."""
    import csv
    import glob

    files = sorted(glob.glob(os.path.join(trace_dir, "**", "*kernel_trace.csv"), recursive=True))
    if not files:
        raise SystemExit(f"no *kernel_trace.csv under {trace_dir}")
    with open(files[0], newline="") as f:
        rows = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))
    starts = [i for i, r in enumerate(rows) if "k_embed_rows" in r["Kernel_Name"]]
    if len(starts) != calls + 1:
        raise SystemExit(f"expected {calls + 1} forwards, found {len(starts)}")
    sel = rows[starts[1]:]
    agg: dict[str, list] = {}
    for r in sel:
        d = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        a = agg.setdefault(r["Kernel_Name"], [0, 0.0, float("inf"), 0.0])
        a[0] += 1
        a[1] += d
        a[2] = min(a[2], d)
        a[3] = max(a[3], d)
    tot = sum(a[1] for a in agg.values()) / calls
    span = (int(sel[-1]["End_Timestamp"]) - int(sel[0]["Start_Timestamp"])) / 1e3 / calls
    print("| Kernel | Calls / forward | Avg µs | Min | Max | µs / forward | % of kernels |")
    print("|---|---:|---:|---:|---:|---:|---:|")
    for name, a in sorted(agg.items(), key=lambda kv: -kv[1][1]):
        nm = name if len(name) <= 90 else name[:87] + "..."
        print(f"| `{nm}` | {a[0] / calls:.2f} | {a[1] / a[0]:.2f} | {a[2]:.2f} | {a[3]:.2f} | {a[1] / calls:.1f} "
              f"| {100 * a[1] / calls / tot:.1f} |")
    print(f"| **all kernels** | {sum(a[0] for a in agg.values()) / calls:.1f} | | | | **{tot:.1f}** | 100 |")
    print()
    print(f"First launch to last end, per forward: {span:.1f} µs.")
    # a kernel launched several times per layer (36 layers), by its place in the layer
    layers = 36
    per_fwd: dict[str, list[float]] = {}
    for r in sel:
        per_fwd.setdefault(r["Kernel_Name"], []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    for name, ds in per_fwd.items():
        n = len(ds) // calls
        if len(ds) % calls or n % layers or n // layers < 2:
            continue
        k = n // layers
        print()
        print(f"`{name}`, {k} launches per layer, by their order in the layer:")
        print()
        print("| Place in the layer | Avg µs | Min | Max |")
        print("|---:|---:|---:|---:|")
        for j in range(k):
            v = [ds[f * n + l * k + j] for f in range(calls) for l in range(layers)]
            print(f"| {j + 1} | {sum(v) / len(v):.2f} | {min(v):.2f} | {max(v):.2f} |")


def trace_summary(trace_dir: str, steps: int) -> None:
    """Markdown table of the event-timed rounds of `bench.py --round-only` from a
    rocprofv3 kernel trace: every dispatch after the first spin kernel (the timed
    loop gates each round behind one), our kernels (wc::) per round and the rest
    (torch: the rewind of the state, the synthetic target's plant, the spin)."""
    import csv
    import glob

    files = sorted(glob.glob(os.path.join(trace_dir, "**", "*kernel_trace.csv"), recursive=True))
    if not files:
        raise SystemExit(f"no *kernel_trace.csv under {trace_dir}")
    with open(files[0], newline="") as f:
        rows = sorted(csv.DictReader(f), key=lambda r: int(r["Dispatch_Id"]))
    first = next(i for i, r in enumerate(rows) if "spin_kernel" in r["Kernel_Name"])
    rows = rows[first:]
    agg: dict[str, list[float]] = {}
    for r in rows:
        us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        agg.setdefault(r["Kernel_Name"], []).append(us)

    def short(n: str) -> str:
        return n if len(n) <= 90 else n[:87] + "..."

    ours = {k: v for k, v in agg.items() if "wc::" in k}
    rest = {k: v for k, v in agg.items() if "wc::" not in k}
    tot = sum(sum(v) for v in ours.values())
    lines = ["| Kernel | Calls / round | Avg µs | Min | Max | µs / round | % of round kernels |",
             "|---|---:|---:|---:|---:|---:|---:|"]
    for k, v in sorted(ours.items(), key=lambda kv: -sum(kv[1])):
        lines.append(f"| `{short(k)}` | {len(v) / steps:.2f} | {np.mean(v):.2f} | {min(v):.2f} | {max(v):.2f} "
                     f"| {sum(v) / steps:.2f} | {100 * sum(v) / tot:.1f} |")
    lines.append(f"| **all round kernels** | {sum(len(v) for v in ours.values()) / steps:.2f} | | | | "
                 f"**{tot / steps:.2f}** | 100 |")
    lines += ["", "Outside the measured round (rewind of the device state, the synthetic target's plant, the "
              "spin gate):", "", "| Kernel | Calls / round | Avg µs |", "|---|---:|---:|"]
    for k, v in sorted(rest.items(), key=lambda kv: -sum(kv[1])):
        lines.append(f"| `{short(k)}` | {len(v) / steps:.2f} | {np.mean(v):.2f} |")
    print("\n".join(lines))


def cold_trace_summary(trace_dir: str) -> None:
    """Markdown table of our kernels (wc::) in a rocprofv3 kernel trace, split
    into cold launches -- the first launch of a kind after a 1 GiB flush (a
    torch reduction of >= 50 µs), up to the next flush -- and warm launches
    (all others, e.g. inside the replayed graphs)."""
    import csv
    import glob

    files = sorted(glob.glob(os.path.join(trace_dir, "**", "*kernel_trace.csv"), recursive=True))
    if not files:
        raise SystemExit(f"no *kernel_trace.csv under {trace_dir}")
    with open(files[0], newline="") as f:
        rows = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))
    cold: dict[str, list[float]] = {}
    warm: dict[str, list[float]] = {}
    seen = None  # kernel kinds launched since the last flush, or None before the first
    for r in rows:
        name, us = r["Kernel_Name"], (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        if "reduce_kernel" in name and us >= 50.0:
            seen = set()
            continue
        if "wc::" not in name:
            continue
        if seen is not None and name not in seen:
            seen.add(name)
            cold.setdefault(name, []).append(us)
        else:
            warm.setdefault(name, []).append(us)

    def short(n: str) -> str:
        return n if len(n) <= 90 else n[:87] + "..."

    lines = ["| Kernel | Cold launches | Cold avg µs | Cold min | Warm launches | Warm avg µs | Warm min |",
             "|---|---:|---:|---:|---:|---:|---:|"]
    for k in sorted(set(cold) | set(warm), key=lambda k: -np.mean(cold.get(k, warm.get(k)))):
        c, w = cold.get(k, []), warm.get(k, [])
        cs = f"{len(c)} | {np.mean(c):.2f} | {min(c):.2f}" if c else "0 | | "
        ws = f"{len(w)} | {np.mean(w):.2f} | {min(w):.2f}" if w else "0 | | "
        lines.append(f"| `{short(k)}` | {cs} | {ws} |")
    print("\n".join(lines))


def head_traffic():
    """HBM bytes per head launch from the committed counter summary, or None."""
    try:
        with open(TRAFFIC_SUMMARY) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        return None
    return None


def _oracle_rounds(gpu, seconds: float, threads: int):
    """Whole config-1 rounds on the oracle (C restatement of the reference's
    arithmetic, OpenMP over output rows): K heads, K-1 layers, the greedy
    verify, the update (fuse + a 3-row layer pass).  Median µs over a bounded
    sample, and the sample size."""
    from oracle import core
    from oracle import sampling as osamp
    from woodcock_amd.synthetic import to_bits

    core.set_threads(threads)
    d = gpu["weights"]
    w = {k: to_bits(v) for k, v in d.w.items()}
    w["lm_head.weight"] = to_bits(d._head)
    od = core.Drafter(d.cfg.as_dict(), w)
    od.d2t = gpu["ids"]
    rnd = gpu["rnd"]
    oc = od.make_cache(1024, kv_bf16=True)
    oc.k[0][:] = to_bits(rnd.cache[0].keys[0])
    oc.v[0][:] = to_bits(rnd.cache[0].values[0])
    logits = gpu["target"].logits.cpu().numpy()
    taps = [t.float().cpu().numpy() for t in gpu["target"].taps]
    root = gpu["root"].cpu().numpy()
    times = []
    t_end = time.perf_counter() + seconds
    while (time.perf_counter() < t_end or len(times) < 2) and len(times) < 200:
        oc.offset = BASE_CTX
        t0 = time.perf_counter()
        out = core.rmsnorm(root, od.w["norm.weight"], d.cfg.rms_norm_eps)
        fb = od.feedback(root, out)
        drafts = []
        for k in range(K):
            z = od.logits(out)
            drafts.append(int(od.d2t[core.argmax(z[0])]))
            if k < K - 1:
                hid, out = od.forward([drafts[-1]], fb, oc)
                fb = od.feedback(hid, out)
        oc.offset = BASE_CTX
        a, nxt = osamp.verify_chain_greedy(logits, drafts)
        acc = drafts[:a] + [nxt]
        g = od.fuse([t[: a + 1] for t in taps])
        od.forward(acc, g, oc)
        times.append(1e6 * (time.perf_counter() - t0))
    return float(np.median(times)), len(times)


def _reference_cpp_step(gpu, seconds: float):
    """The reference's own C++ runtime (oracle/_ref/libwcref.so, compiled from its
    sources: Drafter::forward + Drafter::logits + argmax, src/core/drafter.cpp,
    single-threaded, fp32, no BLAS) on the draft-step unit of
    scripts/time_draft_step.py: one token at drafter context 512, the full
    151,936-row head (its C++ drafter has no restricted head).  The head rows
    are the embedding table's values (timing does not depend on them)."""
    import tempfile

    from oracle import refcpp
    from woodcock_amd.synthetic import to_bits

    if not refcpp.available():
        return None
    d = gpu["weights"]
    w = {k: to_bits(v) for k, v in d.w.items()}
    w["lm_head.weight"] = w["embed_tokens.weight"].copy()
    cfg = d.cfg.as_dict()
    rd = refcpp.RefDrafter(cfg, w)
    cache = rd.make_cache()
    row = cfg["num_kv_heads"] * cfg["head_dim"]
    rng = np.random.default_rng(0)
    kv = rng.standard_normal((BASE_CTX, row)).astype(np.float32)
    cache.append(0, kv, kv, BASE_CTX)
    cache.commit(BASE_CTX)
    feat = rng.standard_normal((1, cfg["hidden_size"])).astype(np.float32)
    times = []
    t_end = time.perf_counter() + seconds
    while (time.perf_counter() < t_end or len(times) < 3) and len(times) < 200:
        t0 = time.perf_counter()
        _, out = rd.forward([17], feat, cache)
        z = rd.logits(out)
        refcpp.argmax(z[0])
        times.append(1e3 * (time.perf_counter() - t0))
        cache.trim_to(BASE_CTX)
    rd.close()
    del tempfile
    return {"value": float(np.median(times)), "unit": "ms", "cores": 1, "kind": "reference",
            "sample": f"{len(times)} draft steps (one token at drafter context {BASE_CTX}, full 151936-row head, "
                      "argmax), median; the reference's C++ runtime compiled from its sources"}


def cpu_baseline(gpu, seconds: float):
    """CPU restatement of the reference's semantics (the oracle port) on the same
    config-1 rounds, at all of the host's cores and at one thread, plus the
    reference's own compiled C++ draft step when its library is present."""
    from oracle import core

    threads = core.default_threads()
    log(f"CPU baseline: oracle rounds at {threads} threads")
    v_all, n_all = _oracle_rounds(gpu, 0.5 * seconds, threads)
    log("CPU baseline: oracle rounds at 1 thread")
    v_one, n_one = _oracle_rounds(gpu, 0.25 * seconds, 1)
    core.set_threads(threads)
    log("CPU baseline: the reference's C++ draft step (loading its weights)")
    ref = _reference_cpp_step(gpu, 0.25 * seconds)
    out = {"value": v_all, "unit": "µs", "cores": threads, "kind": "port",
           "sample": f"{n_all} whole config-1 rounds (CPU restatement of reference semantics: drafter in C, numpy "
                     f"verify), median, {threads} OpenMP threads",
           "single_thread": {"value": v_one, "unit": "µs", "cores": 1,
                             "sample": f"{n_one} whole rounds, median, 1 thread"}}
    if ref is not None:
        out["reference_cpp_draft_step_full_head"] = ref
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200, help="timed rounds")
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-seconds", type=float, default=24.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--pmc-probe", action="store_true", help="only the launches the counter passes read")
    ap.add_argument("--pmc-probe2", action="store_true", help="the launches of the round-kernel counter passes")
    ap.add_argument("--pmc-summary2", nargs=3, metavar=("FETCH_DIR", "WRITE_DIR", "MFMA_DIR"),
                    help="summarise the three counter passes over --pmc-probe2 (no GPU needed)")
    ap.add_argument("--target-chain-only", action="store_true",
                    help="only the 28-layer target forward over a 5-row chain block, 20 calls (for a kernel trace)")
    ap.add_argument("--target-verify-only", action="store_true",
                    help="only the 36-layer Qwen3-4B-shape forward over an 8-row verify block at context 4096, "
                         "10 calls (for a kernel trace)")
    ap.add_argument("--forward-trace-summary", metavar="TRACE_DIR",
                    help="summarise a kernel trace of --target-verify-only (no GPU needed)")
    ap.add_argument("--target-layer-only", action="store_true",
                    help="only the M = 60 verify-width target layer, 45 calls (for a kernel trace of the layer)")
    ap.add_argument("--step-only", action="store_true",
                    help="only the draft steps of configs 1 and 4, warm and cold")
    ap.add_argument("--step-config", choices=("1", "4", "both"), default="both",
                    help="with --step-only: the drafter shapes to time")
    ap.add_argument("--round-only", action="store_true",
                    help="only the timed config-1 rounds (for a kernel trace of the round alone)")
    ap.add_argument("--cold-trace-summary", metavar="TRACE_DIR",
                    help="print the cold / warm split of our kernels in a rocprofv3 kernel trace")
    ap.add_argument("--trace-summary", metavar="TRACE_DIR",
                    help="summarise a rocprofv3 kernel trace of --round-only (no GPU needed); --steps as in that run")
    ap.add_argument("--pmc-valu-summary", metavar="VALU_DIR",
                    help="summarise the VALU-busy counter pass over --pmc-probe2 (no GPU needed)")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="summarise two rocprofv3 counter passes over --pmc-probe (no GPU needed)")
    args = ap.parse_args()
    if args.pmc_summary:
        pmc_summary(*args.pmc_summary)
        return
    if args.pmc_valu_summary:
        pmc_valu_summary(args.pmc_valu_summary)
        return
    if args.pmc_summary2:
        pmc_summary2(*args.pmc_summary2)
        return
    if args.trace_summary:
        trace_summary(args.trace_summary, args.steps)
        return
    if args.cold_trace_summary:
        cold_trace_summary(args.cold_trace_summary)
        return
    if args.forward_trace_summary:
        forward_trace_summary(args.forward_trace_summary)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the round is a batch-1, single-device path with no collective; "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    if args.pmc_probe:
        pmc_probe(args.seed)
        return
    if args.pmc_probe2:
        pmc_probe2(args.seed)
        return
    if args.target_chain_only:
        target_chain_only(args.seed)
        return
    if args.target_layer_only:
        target_layer_only(args.seed)
        return
    if args.target_verify_only:
        target_verify_only(args.seed)
        return
    if args.step_only:
        step_only(args)
        return
    r = bench_gpu(args)
    if args.round_only:
        print(json.dumps({"round_gpu_us": round(r["round_gpu_us"], 2), "steps": args.steps}), flush=True)
        return
    def frac(nbytes, us):
        return nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBS

    head_gbs = r["head_bytes"] / (r["head_us_cold"] * 1e-6) / 1e9  # cold: the weights come from HBM
    cpu = None if args.no_cpu_baseline else cpu_baseline(r, args.cpu_seconds)
    line = {
        "metric": "µs per spec round (draft step, verify+accept, KV compact) + % HBM roofline",
        "value": round(r["round_gpu_us"], 2),
        "unit": "µs",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["round_gpu_us"] / 1e3, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded random-init weights and inputs)",
        "config": {
            "workload": "greedy chain round, Qwen3-1.7B drafter shape, 16k trimmed head, drafter ctx 512: K=4 "
                        "draft steps, greedy verify + accept of the 5-row block against target logits "
                        "[5,151936] fp32 (a=2 accepted), the drafter update over the accepted rows; a chain "
                        "commit is contiguous, so the round has no KV compaction (the tree-path compaction "
                        "of a 28-layer target cache is timed on its own)",
            "k": K, "drafter_ctx": BASE_CTX, "head_rows": 16384, "vocab": 151936, "parallelism": "none (1 GPU)",
        },
        "breakdown": {
            "round_gpu_us": round(r["round_gpu_us"], 2),
            "round_wall_us_incl_sync": round(r["round_wall_us"], 2),
            "target_standin_us_excluded": round(r["target_standin_us"], 2),
            "draft_step_us": round(r["draft_step_us"], 2),
            "draft_step_us_cold": round(r["draft_step_us_cold"], 2),
            "draft_step_hbm_frac": round(frac(r["step_bytes"], r["draft_step_us_cold"]), 4),
            "draft_step_hbm_frac_warm": round(frac(r["step_bytes"], r["draft_step_us"]), 4),
            "verify_accept_us_k5": round(r["verify_accept_us"], 2),
            "kv_compact_us_28l_ctx2048_window6": round(r["kv_compact_us"], 2),
            "verify_stochastic_us_k5_vocab151936": round(r["stochastic_us"], 2),
            "draft_probs_us_k5_head16384": round(r["draft_probs_us"], 2),
            "target_layer_us_qwen3_1p7b_m60_ctx2048": round(r["target_layer_us"], 2),
            "target_layer_hbm_frac_m60": round(100_663_296 / (r["target_layer_us"] * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
            "verify_tree_greedy_us_n60": round(r["tree_verify_us"], 2),
            "target_forward_us_qwen3_1p7b_28l_m5_ctx512": round(r["target_chain_us"], 1),
            "target_forward_us_qwen3_1p7b_28l_m60_tree_ctx2048": round(r["target_tree_us"], 1),
            "tree_draft_us_qwen3_1p7b_depth6_width4_n60": round(r["tree_draft_us"], 1),
            "draft_step_us_qwen3_4b_ctx4096": round(r["draft_step_4b_us"], 2),
            "draft_step_us_cold_qwen3_4b_ctx4096": round(r["draft_step_4b_us_cold"], 2),
            "draft_step_hbm_frac_qwen3_4b": round(frac(STEP4_BYTES, r["draft_step_4b_us_cold"]), 4),
            "draft_step_hbm_frac_warm_qwen3_4b": round(frac(STEP4_BYTES, r["draft_step_4b_us"]), 4),
            "head_gemv_us": round(r["head_us"], 2),
            "head_gemv_us_cold": round(r["head_us_cold"], 2),
            "head_gemv_us_with_argmax_reduction": round(r["head_plain_us"], 2),
            "round_gpu_us_cold": round(r["round_gpu_us_cold"], 2),
            "config4_auto_k_qwen3_4b": {k: (round(v, 2) if isinstance(v, float) else v) for k, v in r["config4"].items()},
            "config5_tree_round_qwen3_1p7b": {k: (round(v, 2) if isinstance(v, float) else v)
                                              for k, v in r["config5"].items()},
        },
        "roofline": {
            "kernel": "draft head GEMV with argmax keys (16384 x 2048 bf16), cold: after a 1 GiB read that "
                      "evicts the Infinity Cache; one launch between events",
            "bound": "hbm",
            "achieved": round(head_gbs, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(head_gbs / PEAK_HBM_GBS, 4),
            "traffic": head_traffic(),
            "warm_achieved": round(r["head_bytes"] / (r["head_us"] * 1e-6) / 1e9, 1),
            "warm_frac": round(frac(r["head_bytes"], r["head_us"]), 4),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
