"""HIP drafter vs the reference C++ goldens and the oracle.

Tolerances (north_star): fp32 activations + fp32 KV within 1e-5 relative of the
reference's fp32 C++ drafter; bf16 KV within 1e-2 relative.  "Relative" is
norm-wise: max |got - ref| <= tol * max |ref| per output tensor.
"""
import ctypes as C

import numpy as np
import pytest
import torch

from conftest import load_golden
from drafter_replay import compare, fixture_config, fixture_weights, replay
from oracle import core

pytestmark = pytest.mark.gpu

FIXTURES = ["tiny", "tiny_prenorm", "tiny_window", "tiny_2layer", "mid"]


class CacheList(list):
    @property
    def offset(self):
        return self[0].offset

    @offset.setter
    def offset(self, v):
        for c in self:
            c.offset = v


class GpuAdapter:
    def __init__(self, cfg_dict, w_np, cuda, kv_dtype):
        from woodcock_amd.config import DrafterConfig
        from woodcock_amd.drafter import Drafter
        from woodcock_amd.synthetic import from_bits

        self.cuda = cuda
        self.d = Drafter(DrafterConfig.from_dict(cfg_dict), {k: from_bits(v, cuda) for k, v in w_np.items()}, cuda,
                         kv_dtype)

    def _t(self, a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(self.cuda)

    def fuse(self, taps):
        return self.d.fuse([self._t(t) for t in taps]).cpu().numpy()

    def make_cache(self, cap):
        return CacheList(self.d.make_cache(cap))

    def forward(self, tokens, feat, cache, positions=None, mask=None):
        hid, out = self.d(torch.from_numpy(np.asarray(tokens)), self._t(feat), cache, positions, mask)
        return hid.cpu().numpy(), out.cpu().numpy()

    def feedback(self, hidden, out):
        return out if self.d.cfg.post_norm else hidden

    def logits(self, out):
        return self.d.logits(self._t(out)).cpu().numpy()

    def cache_rows(self, cache, layer):
        n = cache.offset
        k = cache[layer].keys[0, :, :n].float().permute(1, 0, 2).reshape(n, -1).cpu().numpy()
        v = cache[layer].values[0, :, :n].float().permute(1, 0, 2).reshape(n, -1).cpu().numpy()
        return k, v


@pytest.mark.parametrize("name", FIXTURES)
def test_fp32_cache_matches_reference_cpp(cuda, name):
    z = load_golden(f"drafter_{name}.npz")
    res = replay(GpuAdapter(fixture_config(z), fixture_weights(z), cuda, torch.float32), z)
    compare(res, z, rtol=1e-5, what=f"hip-fp32/{name}")


@pytest.mark.parametrize("name", FIXTURES)
def test_bf16_cache_within_1e2_of_reference_cpp(cuda, name):
    z = load_golden(f"drafter_{name}.npz")
    res = replay(GpuAdapter(fixture_config(z), fixture_weights(z), cuda, torch.bfloat16), z)
    compare(res, z, rtol=1e-2, what=f"hip-bf16/{name}")


def _oracle_step_setup(cfg, seed, cuda, ctx, kv_dtype):
    """Random Qwen3-shaped drafter (16k restricted head), drafter KV prefilled to ctx."""
    from woodcock_amd.drafter import Drafter
    from woodcock_amd.synthetic import draft_vocab, random_drafter, to_bits

    ids = draft_vocab(cfg.vocab_size, 16384, seed=seed, always=(151643, 151645))
    w = random_drafter(cfg, seed=seed, device=cuda, head_rows=16384)
    d = Drafter(cfg, dict(w), cuda, kv_dtype)
    d._vocab_ids = torch.from_numpy(ids).to(cuda)
    d._build_structs(d._rope[0].shape[0])
    wn = {k: to_bits(v) for k, v in w.items()}
    od = core.Drafter(cfg.as_dict(), wn, d2t=None)
    od.d2t = ids
    cache = d.make_cache(ctx + 16)
    oc = od.make_cache(ctx + 16, kv_bf16=kv_dtype == torch.bfloat16)
    g = torch.Generator(device=cuda).manual_seed(seed + 1)
    for li, c in enumerate(cache):
        c.keys[0, :, :ctx] = torch.randn(c.keys[0, :, :ctx].shape, generator=g, device=cuda).to(kv_dtype)
        c.values[0, :, :ctx] = torch.randn(c.values[0, :, :ctx].shape, generator=g, device=cuda).to(kv_dtype)
        c.offset = ctx
        if kv_dtype == torch.bfloat16:
            oc.k[li][:] = to_bits(c.keys[0])
            oc.v[li][:] = to_bits(c.values[0])
        else:
            oc.k[li][:] = c.keys[0].cpu().numpy()
            oc.v[li][:] = c.values[0].cpu().numpy()
    oc.offset = ctx
    return d, od, cache, oc, ids


def _rel(a, b):
    return float(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64)).max() / np.abs(b).max())


@pytest.mark.parametrize("kv_dtype,tol,ctx", [(torch.float32, 1e-5, 512), (torch.bfloat16, 1e-4, 512),
                                              (torch.bfloat16, 1e-4, 2040)])
def test_qwen3_1p7b_draft_step_matches_oracle(cuda, kv_dtype, tol, ctx):
    """Qwen3-1.7B drafter step at full shape: one layer + the 16k head, GPU vs the
    oracle over identical bf16 weights and cache contents.  At context 2040
    (capacity 2056) with a bf16 cache the attention runs on the matrix cores
    (one 64-key chunk per wave), and the step's own key lands inside a wave's
    chunk (keys 56..58 of the chunk at 1984)."""
    from woodcock_amd.config import qwen3_1p7b_drafter

    cfg = qwen3_1p7b_drafter()
    d, od, cache, oc, ids = _oracle_step_setup(cfg, 3, cuda, ctx, kv_dtype)
    rng = np.random.default_rng(3)
    for step in range(3):
        tok = int(rng.integers(0, cfg.vocab_size))
        feat = rng.standard_normal((1, cfg.hidden_size)).astype(np.float32)
        hid, out = d(torch.tensor([tok]), torch.from_numpy(feat).to(cuda), cache)
        ohid, oout = od.forward([tok], feat, oc)
        assert _rel(hid.cpu().numpy(), ohid) <= tol, step
        assert _rel(out.cpu().numpy(), oout) <= tol, step
        z = d.logits(out).cpu().numpy()
        oz = od.logits(oout)
        assert _rel(z, oz) <= tol, step
        tok_dev = d.draft(out).cpu().numpy()
        # the fused final norm + head from the pre-norm hidden state
        out_n = torch.full_like(out, float("nan"))
        z_n = torch.full_like(z := torch.from_numpy(z).to(cuda), float("nan"))
        tok_n = d.draft_from_hidden(hid, out=out_n, logits=z_n).cpu().numpy()
        assert _rel(out_n.cpu().numpy(), oout) <= tol, step
        assert _rel(z_n.cpu().numpy(), oz) <= tol, step
        top2 = np.sort(oz[0])[-2:]
        if top2[1] - top2[0] > 1e-3 * np.abs(oz).max():
            assert int(tok_dev[0]) == int(ids[int(np.argmax(oz[0]))]), step
            assert int(tok_n[0]) == int(tok_dev[0]), step
        k_gpu = cache[0].keys[0, :, : oc.offset].float().cpu().numpy()
        assert _rel(k_gpu, oc.keys_f32(0)[:, : oc.offset]) <= max(tol, 1e-2 if kv_dtype == torch.bfloat16 else 0)


def test_update_rows_with_device_count(cuda):
    """M = a+1 rows (5) through fuse + forward with the row count read on device;
    rows beyond the count are not computed and the cache gets exactly count rows."""
    from woodcock_amd.config import qwen3_1p7b_drafter

    cfg = qwen3_1p7b_drafter()
    d, od, cache, oc, ids = _oracle_step_setup(cfg, 4, cuda, 100, torch.float32)
    rng = np.random.default_rng(4)
    taps = [rng.standard_normal((5, 2048)).astype(np.float32) for _ in range(3)]
    toks = rng.integers(0, cfg.vocab_size, 5).astype(np.int32)
    import ctypes as C

    from woodcock_amd import _lib
    from woodcock_amd.runtime import ptr, stream_ptr

    for n in (1, 3, 5):
        cache_off = cache[0].offset
        nrow = torch.tensor([n, cache_off], dtype=torch.int32, device=cuda)
        g = torch.full((5, 2048), float("nan"), device=cuda)
        tp = [torch.from_numpy(t).to(cuda) for t in taps]
        arr = (C.c_void_p * 3)(*[t.data_ptr() for t in tp])
        _lib.call("wc_drafter_fuse", C.byref(d.dims), C.byref(d.wstruct), arr, _lib.WC_F32, 2048, None, 0, 5,
                  ptr(nrow[0:1]), ptr(g), 2048, ptr(d.ws), stream_ptr())
        hid = torch.full((5, 2048), float("nan"), device=cuda)
        out = torch.full_like(hid, float("nan"))
        kp = (C.c_void_p * 1)(cache[0].keys.data_ptr())
        vp = (C.c_void_p * 1)(cache[0].values.data_ptr())
        adv = torch.zeros(1, dtype=torch.int32, device=cuda)
        tk = torch.from_numpy(toks).to(cuda)
        _lib.call("wc_drafter_forward", C.byref(d.dims), C.byref(d.wstruct), ptr(tk), ptr(g), 2048, None, 0, 5,
                  ptr(nrow[0:1]), kp, vp, _lib.WC_F32, cache[0].capacity, ptr(nrow[1:2]), 0, None, None, 0, ptr(hid),
                  ptr(out), ptr(adv), ptr(d.ws), stream_ptr())
        og = od.fuse([t[:n] for t in taps])
        ohid, oout = od.forward(toks[:n], og, oc)
        assert int(adv.item()) == cache_off + n
        assert _rel(g[:n].cpu().numpy(), og) <= 1e-5
        assert _rel(hid[:n].cpu().numpy(), ohid) <= 1e-5
        assert _rel(out[:n].cpu().numpy(), oout) <= 1e-5
        assert torch.isnan(hid[n:]).all() and torch.isnan(g[n:]).all()
        for c in cache:
            c.offset = cache_off + n


def test_qwen3_4b_step_and_update_match_oracle(cuda):
    """Qwen3-4B drafter width (hidden 2560, 32 q / 8 kv heads, SwiGLU 9728, fc
    7680 -> 2560, the 16k head) at drafter context 4096 with a bf16 cache: two
    draft steps (layer + fused final norm and head) and a 5-row update pass
    (fuse + forward), GPU vs the oracle over identical weights and cache."""
    import ctypes as C

    from woodcock_amd import _lib
    from woodcock_amd.config import qwen3_4b_drafter
    from woodcock_amd.runtime import ptr, stream_ptr

    cfg = qwen3_4b_drafter()
    dm = cfg.hidden_size
    d, od, cache, oc, ids = _oracle_step_setup(cfg, 6, cuda, 4096, torch.bfloat16)
    rng = np.random.default_rng(6)
    tol = 1e-4
    for step in range(2):
        tok = int(rng.integers(0, cfg.vocab_size))
        feat = rng.standard_normal((1, dm)).astype(np.float32)
        hid, out = d(torch.tensor([tok]), torch.from_numpy(feat).to(cuda), cache)
        ohid, oout = od.forward([tok], feat, oc)
        assert _rel(hid.cpu().numpy(), ohid) <= tol, step
        out_n = torch.full_like(out, float("nan"))
        z = torch.full((1, 16384), float("nan"), device=cuda)
        tk = d.draft_from_hidden(hid, out=out_n, logits=z).cpu().numpy()
        oz = od.logits(oout)
        assert _rel(out_n.cpu().numpy(), oout) <= tol, step
        assert _rel(z.cpu().numpy(), oz) <= tol, step
        top2 = np.sort(oz[0])[-2:]
        if top2[1] - top2[0] > 1e-3 * np.abs(oz).max():
            assert int(tk[0]) == int(ids[int(np.argmax(oz[0]))]), step
    # update pass over 5 accepted rows
    taps = [rng.standard_normal((5, dm)).astype(np.float32) for _ in range(3)]
    toks = rng.integers(0, cfg.vocab_size, 5).astype(np.int32)
    off = cache[0].offset
    nrow = torch.tensor([5, off], dtype=torch.int32, device=cuda)
    g = torch.empty(5, dm, device=cuda)
    tp = [torch.from_numpy(t).to(cuda) for t in taps]
    arr = (C.c_void_p * 3)(*[t.data_ptr() for t in tp])
    _lib.call("wc_drafter_fuse", C.byref(d.dims), C.byref(d.wstruct), arr, _lib.WC_F32, dm, None, 0, 5, ptr(nrow[0:1]),
              ptr(g), dm, ptr(d.ws), stream_ptr())
    hid = torch.empty(5, dm, device=cuda)
    kp = (C.c_void_p * 1)(cache[0].keys.data_ptr())
    vp = (C.c_void_p * 1)(cache[0].values.data_ptr())
    tk = torch.from_numpy(toks).to(cuda)
    _lib.call("wc_drafter_forward", C.byref(d.dims), C.byref(d.wstruct), ptr(tk), ptr(g), dm, None, 0, 5,
              ptr(nrow[0:1]), kp, vp, _lib.WC_BF16, cache[0].capacity, ptr(nrow[1:2]), 0, None, None, 0, ptr(hid),
              None, None, ptr(d.ws), stream_ptr())
    og = od.fuse(taps)
    ohid, _ = od.forward(toks, og, oc)
    assert _rel(g.cpu().numpy(), og) <= 1e-5
    assert _rel(hid.cpu().numpy(), ohid) <= tol


@pytest.mark.parametrize("tap_dtype", [torch.float32, torch.bfloat16])
def test_fuse_gathers_kept_tree_rows(cuda, tap_dtype):
    """Drafter.fuse at the accepted path of a tree (spec.py:327-328): the taps of
    a 60-row verify block gathered at keep = [0, 3, 17, 41] on the device
    (wc_drafter_fuse with tap_rows_dev and a device row count), with stale
    entries past n_keep -- one of them far outside the taps, as an earlier,
    larger tree could leave -- which must be neither read out of bounds nor
    written: rows past n_keep stay untouched."""
    from woodcock_amd import _lib
    from woodcock_amd.config import qwen3_1p7b_drafter
    from woodcock_amd.runtime import ptr, stream_ptr

    cfg = qwen3_1p7b_drafter()
    dm = cfg.hidden_size
    d, od, _, _, _ = _oracle_step_setup(cfg, 12, cuda, 16, torch.bfloat16)
    rng = np.random.default_rng(12)
    tp = [torch.from_numpy(rng.standard_normal((60, dm)).astype(np.float32)).to(cuda).to(tap_dtype)
          for _ in range(3)]
    taps = [t.float().cpu().numpy() for t in tp]
    keep = [0, 3, 17, 41]
    rows = 7
    kdev = torch.tensor(keep + [59, 1 << 20, -5], dtype=torch.int32, device=cuda)
    nk = torch.tensor([len(keep)], dtype=torch.int32, device=cuda)
    g = torch.full((rows, dm), float("nan"), device=cuda)
    arr = (C.c_void_p * 3)(*[t.data_ptr() for t in tp])
    _lib.call("wc_drafter_fuse", C.byref(d.dims), C.byref(d.wstruct), arr,
              _lib.WC_F32 if tap_dtype == torch.float32 else _lib.WC_BF16, dm, ptr(kdev), 60, rows, ptr(nk), ptr(g),
              dm, ptr(d.ws), stream_ptr())
    og = od.fuse([t[keep] for t in taps])
    got = g.cpu().numpy()
    assert _rel(got[:len(keep)], og) <= 1e-5
    assert np.isnan(got[len(keep):]).all()
    # the same gather with every row live equals the host-side gather
    nk.fill_(rows)
    kdev[len(keep):] = torch.tensor([50, 51, 59], dtype=torch.int32, device=cuda)
    _lib.call("wc_drafter_fuse", C.byref(d.dims), C.byref(d.wstruct), arr,
              _lib.WC_F32 if tap_dtype == torch.float32 else _lib.WC_BF16, dm, ptr(kdev), 60, rows, ptr(nk), ptr(g),
              dm, ptr(d.ws), stream_ptr())
    assert _rel(g.cpu().numpy(), od.fuse([t[keep + [50, 51, 59]] for t in taps])) <= 1e-5


def test_restricted_head_equals_gathered_full_head(cuda):
    """tests/test_vocab.py:37-47 on the GPU: bit-exact rows, token_ids maps rows."""
    from woodcock_amd.config import tiny_drafter
    from woodcock_amd.drafter import Drafter

    d = Drafter.from_synthetic(tiny_drafter(), seed=0, device=cuda)
    out = torch.randn(3, 32, device=cuda)
    full = d.logits(out)
    ids = [3, 7, 8, 21, 49]
    d.restrict_vocab(ids)
    assert torch.equal(d.logits(out), full[:, ids])
    tok = d.draft(out)
    rows = torch.argmax(full[:, ids], dim=-1)
    assert tok.tolist() == [ids[r] for r in rows.tolist()]
    assert d.token_ids(rows).tolist() == [ids[r] for r in rows.tolist()]
    with pytest.raises(ValueError):
        d.restrict_vocab(ids)
    with pytest.raises(ValueError):
        d.save("/tmp/never-written")


def test_gumbel_draws_follow_softmax(cuda):
    """Gumbel-max over the head rows with Philox uniforms == a draw from softmax(z/T):
    chi-square over 20000 rounds (round index read on device)."""
    from scipy.stats import chisquare

    from woodcock_amd.config import tiny_drafter
    from woodcock_amd.drafter import Drafter

    d = Drafter.from_synthetic(tiny_drafter(vocab_size=8), seed=1, device=cuda)
    out = torch.randn(1, 32, device=cuda) * 3
    z = d.logits(out)[0].double().cpu().numpy()
    T = 0.7
    p = np.exp((z - z.max()) / T)
    p /= p.sum()
    counts = np.zeros(8)
    rnd = torch.zeros(1, dtype=torch.int32, device=cuda)
    toks = []
    for r in range(20000):
        rnd.fill_(r)
        toks.append(d.draft(out, gumbel=(11, rnd, 5, T)))
    for t in torch.cat(toks).cpu().numpy():
        counts[t] += 1
    assert chisquare(counts, p * counts.sum()).pvalue > 1e-3
    # deterministic given (seed, round, purpose)
    rnd.fill_(7)
    a = d.draft(out, gumbel=(11, rnd, 5, T)).item()
    b = d.draft(out, gumbel=(11, rnd, 5, T)).item()
    assert a == b


@pytest.mark.parametrize("head_dim,heads,kv_heads", [(8, 4, 2), (32, 4, 1), (64, 4, 2), (128, 4, 4), (256, 2, 1)])
def test_head_dim_sweep_multi_row_forward(cuda, head_dim, heads, kv_heads):
    """Every instantiated head_dim / GQA grouping, 1-row and 3-row forwards with
    appends, against the oracle (fp32 cache, 1e-5)."""
    from woodcock_amd.config import DrafterConfig
    from woodcock_amd.drafter import Drafter
    from woodcock_amd.synthetic import random_drafter, to_bits

    cfg = DrafterConfig(hidden_size=128, num_layers=1, num_heads=heads, num_kv_heads=kv_heads, head_dim=head_dim,
                        intermediate_size=192, vocab_size=300, target_hidden_size=64, rope_theta=1e6)
    w = random_drafter(cfg, seed=head_dim, device=cuda)
    d = Drafter(cfg, dict(w), cuda, torch.float32)
    od = core.Drafter(cfg.as_dict(), {k: to_bits(v) for k, v in w.items()})
    cache, oc = d.make_cache(64), od.make_cache(64)
    rng = np.random.default_rng(head_dim)
    for L in (5, 1, 3, 1):
        toks = rng.integers(0, cfg.vocab_size, L)
        feat = rng.standard_normal((L, cfg.hidden_size)).astype(np.float32)
        hid, out = d(torch.from_numpy(toks), torch.from_numpy(feat).to(cuda), cache)
        ohid, oout = od.forward(toks, feat, oc)
        assert _rel(hid.cpu().numpy(), ohid) <= 1e-5, L
        assert _rel(out.cpu().numpy(), oout) <= 1e-5, L
        n = oc.offset
        assert _rel(cache[0].keys[0, :, :n].cpu().numpy(), oc.keys_f32(0)[:, :n]) <= 1e-5, L


def test_saved_drafter_reloads_and_computes_identically(cuda, tmp_path):
    """Drafter.save -> Drafter.load (config.json, model.safetensors, woodcock.json;
    python/woodcock/export.py:55-63 self-check): identical forward and head."""
    from woodcock_amd.config import DrafterConfig
    from woodcock_amd.drafter import Drafter

    cfg = DrafterConfig(hidden_size=256, num_layers=1, num_heads=4, num_kv_heads=2, head_dim=64,
                        intermediate_size=512, vocab_size=2048, target_hidden_size=192)
    d = Drafter.from_synthetic(cfg, seed=3, device=cuda, kv_dtype=torch.float32)
    d.save(tmp_path)
    e = Drafter.load(tmp_path, device=cuda, kv_dtype=torch.float32)
    g = torch.Generator(device=cuda).manual_seed(1)
    feat = torch.randn(3, cfg.hidden_size, generator=g, device=cuda)
    toks = torch.tensor([5, 77, 1000], dtype=torch.int32, device=cuda)
    outs = []
    for m in (d, e):
        cache = m.make_cache(16)
        hid, out = m(toks, feat, cache)
        outs.append((hid, out, m.draft(out)))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    assert torch.equal(outs[0][2], outs[1][2])


def test_head_logits_only_equals_argmax_head(cuda):
    """wc_draft_head / wc_draft_head_norm with no token output write the logits
    alone (the store epilogue; four rows on the few-row MFMA kernel, like the
    argmax head): the same logits as the argmax head, at one row (with and
    without the fused final norm) and at four rows, within 1e-6 of their
    magnitude (the same products in the same order, so equal in practice)."""
    import ctypes as C

    from woodcock_amd import _lib
    from woodcock_amd.config import QWEN3_EOS, qwen3_1p7b_drafter
    from woodcock_amd.drafter import Drafter
    from woodcock_amd.runtime import ptr, stream_ptr
    from woodcock_amd.synthetic import draft_vocab, random_drafter

    cfg = qwen3_1p7b_drafter()
    d = Drafter(cfg, random_drafter(cfg, seed=5, device=cuda), cuda, torch.bfloat16)
    d.restrict_vocab(draft_vocab(cfg.vocab_size, 16384, seed=5, always=QWEN3_EOS))
    dm, hr = cfg.hidden_size, 16384
    g = torch.Generator(device=cuda).manual_seed(5)
    x = torch.randn(4, dm, generator=g, device=cuda)
    dims, W, ws, s = C.byref(d.dims), C.byref(d.wstruct), ptr(d.ws), stream_ptr()
    for rows, norm in ((1, False), (1, True), (4, False)):
        outs = []
        for with_tok in (True, False):
            z = torch.full((rows, hr), float("nan"), device=cuda)
            tok = torch.empty(rows, dtype=torch.int32, device=cuda) if with_tok else None
            if norm:
                xn = torch.empty(1, dm, device=cuda)
                _lib.call("wc_draft_head_norm", dims, W, ptr(x), dm, None, 0, ptr(xn), dm, ptr(z), z.stride(0),
                          ptr(tok) if with_tok else None, None, None, ws, s)
            else:
                _lib.call("wc_draft_head", dims, W, ptr(x), dm, None, 0, rows, ptr(z), z.stride(0),
                          ptr(tok) if with_tok else None, None, None, ws, s)
            torch.cuda.synchronize()
            outs.append(z.cpu().numpy())
        assert np.isfinite(outs[1]).all(), (rows, norm)
        assert np.abs(outs[1] - outs[0]).max() <= 1e-6 * np.abs(outs[0]).max(), (rows, norm)
