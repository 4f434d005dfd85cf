"""The one-launch draft step (wc_draft_step, csrc/step.hip) and the one-launch
layer wc_drafter_forward takes for one row, against the per-op launches of the
same computation (wc_set_one_launch_step(0)) (python/woodcock/spec.py:346-350;
drafter.py:164-215).  Both run the same products in the same summation order;
the QKV rows, the drafted token and head row, `out` and the appended cache row
are equal bit for bit, the attention output and what follows it within fp32
rounding (the compiler contracts a multiply and an add into one fma in
different places of the two kernels): 1e-5 relative, norm-wise.

Covered: the Qwen3-1.7B drafter (16k head, bf16 cache at context 512) over a
chain of steps and 64 graph replays of one step (the launch counter and the
argmax slot parity advance every launch); the Qwen3-4B drafter at context 4096
(several chunks per attention split); post_norm off (feedback = the pre-norm
hidden row); an fp32 cache with a sliding window; a two-layer drafter (the
layer without the token stream); and the bounded-wait give-up path forced from
the host with a zero spin limit: the launch still ends, the status word flags
it, ChainRound.finish raises, and the next launch is exact again.
"""
import ctypes as C

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _drafter(cuda, cfg, head_rows, seed, kv_dtype=torch.bfloat16):
    from woodcock_amd.drafter import Drafter
    from woodcock_amd.synthetic import draft_vocab, random_drafter

    d = Drafter(cfg, random_drafter(cfg, seed=seed, device=cuda), cuda, kv_dtype)
    d.restrict_vocab(draft_vocab(cfg.vocab_size, head_rows, seed=seed))
    return d


def _fill(cuda, cache, ctx, seed):
    g = torch.Generator(device=cuda).manual_seed(seed)
    for c in cache:
        c.keys[0, :, :ctx] = torch.randn(c.keys[0, :, :ctx].shape, generator=g, device=cuda).to(c.keys.dtype)
        c.values[0, :, :ctx] = torch.randn(c.values[0, :, :ctx].shape, generator=g, device=cuda).to(c.keys.dtype)


def _chain(d, cache, hid0, ctx, steps, one, feedback_out=1):
    """`steps` draft steps from hid0 at cache offset ctx: tokens, outs, hiddens."""
    from woodcock_amd import _lib
    from woodcock_amd.runtime import ptr, stream_ptr

    dm = d.cfg.hidden_size
    dev = hid0.device
    kp = (C.c_void_p * len(cache))(*[c.keys.data_ptr() for c in cache])
    vp = (C.c_void_p * len(cache))(*[c.values.data_ptr() for c in cache])
    kvdt = _lib.WC_BF16 if cache[0].keys.dtype == torch.bfloat16 else _lib.WC_F32
    off = torch.tensor([ctx], dtype=torch.int32, device=dev)
    hids = torch.zeros(steps + 1, dm, device=dev)
    outs = torch.zeros(steps, dm, device=dev)
    toks = torch.zeros(steps, dtype=torch.int32, device=dev)
    rows = torch.zeros(steps, dtype=torch.int32, device=dev)
    hids[0] = hid0
    _lib.call("wc_set_one_launch_step", int(one))
    try:
        for i in range(steps):
            _lib.call("wc_draft_step", C.byref(d.dims), C.byref(d.wstruct), ptr(hids[i:i + 1]), dm, None, 0,
                      ptr(outs[i:i + 1]), dm, ptr(toks[i:i + 1]), ptr(rows[i:i + 1]), kp, vp, kvdt,
                      cache[0].capacity, ptr(off), i, feedback_out, ptr(hids[i + 1:i + 2]), ptr(d.ws), stream_ptr())
        torch.cuda.synchronize()
    finally:
        _lib.call("wc_set_one_launch_step", 1)
    return toks.cpu(), rows.cpu(), outs.cpu(), hids.cpu()


def _clone(cache):
    from woodcock_amd.cache import KVCache

    out = []
    for c in cache:
        n = KVCache(c.kv_heads, c.head_dim, c.capacity, c.keys.dtype, c.keys.device)
        n.keys.copy_(c.keys)
        n.values.copy_(c.values)
        out.append(n)
    return out


def _status(d) -> int:
    torch.cuda.synchronize()
    return int(d.step_status().item())


def _same(cuda, d, ctx, cap, steps, seed, feedback_out=1, kv_dtype=torch.bfloat16):
    cache = d.make_cache(cap, dtype=kv_dtype)
    _fill(cuda, cache, ctx, seed)
    base = _clone(cache)
    hid0 = torch.randn(d.cfg.hidden_size, generator=torch.Generator(device=cuda).manual_seed(seed + 1), device=cuda)
    got = _chain(d, cache, hid0, ctx, steps, True, feedback_out)
    want = _chain(d, base, hid0, ctx, steps, False, feedback_out)
    assert _status(d) == 0
    assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])  # tokens, head rows
    assert torch.equal(got[2][0], want[2][0])  # `out` of the first step's input
    for name, g, w in (("out", got[2], want[2]), ("hidden", got[3], want[3])):
        assert _rel(g, w) < 1e-5, name
    for c, b in zip(cache, base):
        # the appended rows come from the QKV rows (bit-exact) on the first
        # step, then from hidden states equal within fp32 rounding
        assert _rel(c.keys.float(), b.keys.float()) < 1e-5 and _rel(c.values.float(), b.values.float()) < 1e-5
    return got


def _rel(a, b):
    a, b = (x.detach().float().cpu().numpy() if torch.is_tensor(x) else x for x in (a, b))
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def test_step_equals_per_op_launches_qwen3_1p7b(cuda):
    from woodcock_amd.config import qwen3_1p7b_drafter

    d = _drafter(cuda, qwen3_1p7b_drafter(), 16384, seed=101)
    _same(cuda, d, 512, 1024, 6, seed=102)


def test_step_qwen3_4b_long_context(cuda):
    from woodcock_amd.config import qwen3_4b_drafter

    d = _drafter(cuda, qwen3_4b_drafter(), 16384, seed=103)
    _same(cuda, d, 4096, 4096 + 16, 3, seed=104)


def test_step_prenorm_feedback(cuda):
    from woodcock_amd.config import qwen3_1p7b_drafter

    cfg = qwen3_1p7b_drafter()
    cfg.post_norm = False
    d = _drafter(cuda, cfg, 16384, seed=105)
    _same(cuda, d, 300, 512, 4, seed=106, feedback_out=0)


def test_step_fp32_cache_sliding_window(cuda):
    from woodcock_amd.config import qwen3_1p7b_drafter

    cfg = qwen3_1p7b_drafter()
    cfg.window = 24
    d = _drafter(cuda, cfg, 4096, seed=107, kv_dtype=torch.float32)
    _same(cuda, d, 70, 128, 4, seed=108, kv_dtype=torch.float32)


def test_two_layer_forward_one_row(cuda):
    """wc_drafter_forward at one row on a two-layer drafter: layer 0 (token
    stream) and layer 1 (without) each one launch, equal to the per-op path."""
    from woodcock_amd import _lib
    from woodcock_amd.config import qwen3_1p7b_drafter
    from woodcock_amd.runtime import ptr, stream_ptr

    cfg = qwen3_1p7b_drafter()
    cfg.num_layers = 2
    d = _drafter(cuda, cfg, 4096, seed=109)
    cache = d.make_cache(640)
    _fill(cuda, cache, 600, seed=110)
    base = _clone(cache)
    feat = torch.randn(1, 2048, generator=torch.Generator(device=cuda).manual_seed(111), device=cuda)
    tok = torch.tensor([1234], dtype=torch.int32, device=cuda)
    off = torch.tensor([600], dtype=torch.int32, device=cuda)

    def run(c, one):
        kp = (C.c_void_p * 2)(*[x.keys.data_ptr() for x in c])
        vp = (C.c_void_p * 2)(*[x.values.data_ptr() for x in c])
        h = torch.zeros(1, 2048, device=cuda)
        _lib.call("wc_set_one_launch_step", int(one))
        try:
            for _ in range(3):
                _lib.call("wc_drafter_forward", C.byref(d.dims), C.byref(d.wstruct), ptr(tok), ptr(feat), 2048, None,
                          0, 1, None, kp, vp, _lib.WC_BF16, 640, ptr(off), 0, None, None, 0, ptr(h), None, None,
                          ptr(d.ws), stream_ptr())
            torch.cuda.synchronize()
        finally:
            _lib.call("wc_set_one_launch_step", 1)
        return h.cpu()

    assert _rel(run(cache, True), run(base, False)) < 1e-5
    assert _status(d) == 0
    for c, b in zip(cache, base):
        assert _rel(c.keys.float(), b.keys.float()) < 1e-5 and _rel(c.values.float(), b.values.float()) < 1e-5


def test_step_graph_replays(cuda):
    """One step captured once and replayed 64 times (the launch index and the
    argmax slot set advance every replay): every replay returns the eager result."""
    from woodcock_amd import _lib
    from woodcock_amd.config import qwen3_1p7b_drafter
    from woodcock_amd.runtime import ptr, stream_ptr

    d = _drafter(cuda, qwen3_1p7b_drafter(), 16384, seed=112)
    cache = d.make_cache(1024)
    _fill(cuda, cache, 512, seed=113)
    dm = 2048
    kp = (C.c_void_p * 1)(cache[0].keys.data_ptr())
    vp = (C.c_void_p * 1)(cache[0].values.data_ptr())
    off = torch.tensor([512], dtype=torch.int32, device=cuda)
    hid = torch.randn(1, dm, generator=torch.Generator(device=cuda).manual_seed(114), device=cuda)
    out = torch.zeros(1, dm, device=cuda)
    nxt = torch.zeros(1, dm, device=cuda)
    tok = torch.zeros(1, dtype=torch.int32, device=cuda)

    def step():
        _lib.call("wc_draft_step", C.byref(d.dims), C.byref(d.wstruct), ptr(hid), dm, None, 0, ptr(out), dm, ptr(tok),
                  None, kp, vp, _lib.WC_BF16, 1024, ptr(off), 0, 1, ptr(nxt), ptr(d.ws), stream_ptr())

    step()
    torch.cuda.synchronize()
    want = (tok.clone(), out.clone(), nxt.clone())
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        step()
    torch.cuda.synchronize()
    for r in range(64):
        tok.zero_()
        nxt.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(tok, want[0]) and torch.equal(out, want[1]) and torch.equal(nxt, want[2]), f"replay {r}"
    assert _status(d) == 0


def test_step_give_up_is_reported_and_recovers(cuda):
    """A zero spin limit makes every wait that does not find its phase complete
    give up at once (forced from the host): the launch ends, the status word
    is set, ChainRound.finish raises; with the limit restored and the word
    cleared the next launch equals the per-op path again."""
    from woodcock_amd import _lib
    from woodcock_amd.config import qwen3_1p7b_drafter
    from woodcock_amd.spec import ChainRound
    from woodcock_amd.synthetic import SyntheticTarget

    d = _drafter(cuda, qwen3_1p7b_drafter(), 16384, seed=115)
    cache = d.make_cache(1024)
    _fill(cuda, cache, 512, seed=116)
    hid0 = torch.randn(2048, generator=torch.Generator(device=cuda).manual_seed(117), device=cuda)
    _lib.call("wc_set_spin_limit", 0)
    try:
        _chain(d, _clone(cache), hid0, 512, 4, True)
    finally:
        _lib.call("wc_set_spin_limit", -1)
    assert _status(d) != 0
    # the round loop reports it at its sync
    rnd = ChainRound(d, 4, 1024)
    target = SyntheticTarget(4, d.cfg.vocab_size, d.cfg.target_hidden_size, device=cuda, seed=118)
    rnd.set_root(512, hid0[None])
    rnd.enqueue_draft()
    target.plant(rnd.drafts, 2)
    rnd.enqueue_verify_commit(target.logits, target.taps)
    rnd.enqueue_readback()
    with pytest.raises(_lib.WoodcockHipError):
        rnd.finish()
    assert _status(d) == 0  # cleared by finish
    got = _chain(d, _clone(cache), hid0, 512, 4, True)
    want = _chain(d, _clone(cache), hid0, 512, 4, False)
    assert _status(d) == 0
    assert torch.equal(got[0], want[0]) and _rel(got[3], want[3]) < 1e-5


def _ws_buffers(d):
    """fp32 views of the drafter workspace's per-step buffers (qkv, attn, h1,
    act), at the offsets of the workspace layout (csrc/drafter_ws.h)."""
    from woodcock_amd import _lib

    cfg = d.cfg
    R = _lib.WC_MAX_STEP_ROWS
    nqkv = (cfg.num_heads + 2 * cfg.num_kv_heads) * cfg.head_dim

    def up(x):
        return (x + 255) // 256 * 256

    off = 0
    sizes = [4 * 32 * 65, 4 * 32 * 65, 4 * 32 * 64, 8 * R * 32 * 16]
    for s in sizes:
        off = up(off + s)
    out = {}
    for name, n in (("qkv", nqkv), ("attn", cfg.num_heads * cfg.head_dim), ("h1", cfg.hidden_size),
                    ("act", cfg.intermediate_size)):
        out[name] = d.ws[off:off + 4 * n].view(torch.float32)
        off = up(off + 4 * R * n)
    return out


def test_step_intermediates_equal_per_op(cuda):
    """One step from identical state: the QKV rows in the workspace equal the
    per-op launches' bit for bit; the attention output, h1 and the SwiGLU
    activations within fp32 rounding."""
    from woodcock_amd.config import qwen3_1p7b_drafter

    d = _drafter(cuda, qwen3_1p7b_drafter(), 16384, seed=119)
    cache = d.make_cache(1024)
    _fill(cuda, cache, 512, seed=120)
    hid0 = torch.randn(2048, generator=torch.Generator(device=cuda).manual_seed(121), device=cuda)
    bufs = _ws_buffers(d)
    got = _chain(d, _clone(cache), hid0, 512, 1, True)
    g = {k: v.clone().cpu() for k, v in bufs.items()}
    want = _chain(d, _clone(cache), hid0, 512, 1, False)
    w = {k: v.clone().cpu() for k, v in bufs.items()}
    assert torch.equal(got[0], want[0]) and torch.equal(got[2], want[2])
    assert torch.equal(g["qkv"], w["qkv"])
    for k in ("attn", "h1", "act"):
        assert _rel(g[k], w[k]) < 1e-5, k
