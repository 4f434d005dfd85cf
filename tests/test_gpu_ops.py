"""The backend operations (wc_rmsnorm / wc_linear / wc_rope / wc_silu_mul /
wc_softmax / wc_attention, wc_kv_append / wc_kv_set_offset) against the
reference's own ops::* outputs (tests/golden/ops.npz, written by its
src/backends/cpu_ops.cpp; include/woodcock/ops.h:9-24), and the verify-width
target forward against the reference's Qwen3::forward (tests/golden/qwen3_small.npz;
src/core/qwen3.cpp:75-114).

Tolerances, max |got - want| / max |want| per tensor: rmsnorm 1e-6 (fp64 sum
of squares as the reference), RoPE bit-exact with the host cos / sin table and
2e-6 with device cos / sin, silu_mul and softmax 2e-6 (device exp), linear and
attention 1e-5 (fp32 sums in another order), the target forward 5e-5 with an
fp32 cache (bf16 hi + lo MFMA products).
"""
import numpy as np
import pytest
import torch

from conftest import load_golden
from golden import detgen

pytestmark = pytest.mark.gpu


def _nrel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


@pytest.fixture(scope="module")
def fx(cuda):
    return detgen.ops_inputs(), load_golden("ops.npz")


def _t(a, cuda):
    return torch.from_numpy(np.ascontiguousarray(a)).to(cuda)


@pytest.mark.parametrize("wdt", [torch.float32, torch.bfloat16])
def test_rmsnorm(cuda, fx, wdt):
    from woodcock_amd import ops

    x, y = fx
    for c in range(len(detgen.RMS)):
        xt = _t(x[f"rms{c}.x"], cuda)
        w = _t(x[f"rms{c}.w"], cuda).to(wdt)
        got = ops.rmsnorm(xt, w, float(x[f"rms{c}.eps"]))
        assert _nrel(got.cpu().numpy(), y[f"rms{c}.y"]) < 1e-6, c
        ops.rmsnorm(xt, w, float(x[f"rms{c}.eps"]), out=xt)  # in place
        assert torch.equal(xt, got), c


@pytest.mark.parametrize("wdt", [torch.float32, torch.bfloat16])
def test_linear(cuda, fx, wdt):
    from woodcock_amd import ops

    x, y = fx
    for c in range(len(detgen.LIN)):
        xt, W = _t(x[f"lin{c}.x"], cuda), _t(x[f"lin{c}.W"], cuda).to(wdt)
        assert _nrel(ops.linear(xt, W).cpu().numpy(), y[f"lin{c}.y"]) < 1e-5, c
        acc = _t(x[f"lin{c}.y0"], cuda)
        ops.linear(xt, W, acc, accumulate=True)
        assert _nrel(acc.cpu().numpy(), y[f"lin{c}.y_acc"]) < 1e-5, c


def test_rope(cuda, fx):
    import ctypes as C

    from woodcock_amd import _lib, ops

    x, y = fx
    for c, (L, heads, D, base) in enumerate(detgen.ROPE):
        pos = x[f"rope{c}.pos"]
        got = ops.rope(_t(x[f"rope{c}.x"], cuda), torch.from_numpy(pos), base)
        assert _nrel(got.cpu().numpy(), y[f"rope{c}.y"]) < 2e-6, c
        n = int(pos.max()) + 1
        cos = np.empty((n, D // 2), np.float32)
        sin = np.empty_like(cos)
        _lib.call("wc_rope_table", cos.ctypes.data_as(C.c_void_p), sin.ctypes.data_as(C.c_void_p), n, D, base)
        got = ops.rope(_t(x[f"rope{c}.x"], cuda), torch.from_numpy(pos), base, table=(_t(cos, cuda), _t(sin, cuda)))
        assert np.array_equal(got.cpu().numpy(), y[f"rope{c}.y"]), c


def test_silu_mul_and_softmax(cuda, fx):
    from woodcock_amd import ops

    x, y = fx
    g = ops.silu_mul(_t(x["silu.gate"], cuda), _t(x["silu.up"], cuda))
    assert _nrel(g.cpu().numpy(), y["silu.y"]) < 2e-6
    for c in range(len(detgen.SOFTMAX_N)):
        got = ops.softmax(_t(x[f"sm{c}.x"], cuda)).cpu().numpy()
        want = y[f"sm{c}.y"]
        assert _nrel(got, want) < 2e-6, c
        assert (got[x[f"sm{c}.x"] == -np.inf] == 0).all(), c
    # several rows at once equal one row at a time
    rows = torch.stack([_t(x["sm1.x"], cuda), _t(x["sm1.x"], cuda) * 0.5])
    both = ops.softmax(rows.clone())
    assert torch.equal(both[0], ops.softmax(_t(x["sm1.x"], cuda)))


def test_attention(cuda, fx):
    from woodcock_amd import ops

    x, y = fx
    for c in range(len(detgen.ATT)):
        m = x.get(f"att{c}.mask")
        got = ops.attention(_t(x[f"att{c}.q"], cuda), _t(x[f"att{c}.K"], cuda), _t(x[f"att{c}.V"], cuda),
                            None if m is None else torch.from_numpy(m), float(x[f"att{c}.scale"]))
        assert _nrel(got.cpu().numpy(), y[f"att{c}.out"]) < 1e-5, c


def test_kv_append_and_trim(cuda):
    """KVCache::append + commit, then trim_to (include/woodcock/cache.h:17-19;
    src/cache/kv_cache.cpp:8-19): rows land at the device offset, the offset
    advances by L (in place), and a trim rewinds it so the next append
    overwrites the discarded rows."""
    from woodcock_amd import _lib
    from woodcock_amd.runtime import ptr, stream_ptr

    row, cap = 2 * 16, 40
    kc = torch.zeros(cap, row, device=cuda)
    vc = torch.zeros(cap, row, device=cuda)
    off = torch.tensor([3], dtype=torch.int32, device=cuda)
    k1, v1 = torch.randn(5, row, device=cuda), torch.randn(5, row, device=cuda)
    _lib.call("wc_kv_append", ptr(kc), ptr(vc), cap, row, ptr(k1), ptr(v1), 5, ptr(off), ptr(off), stream_ptr())
    assert int(off.item()) == 8
    assert torch.equal(kc[3:8], k1) and torch.equal(vc[3:8], v1) and not kc[:3].any() and not kc[8:].any()
    _lib.call("wc_kv_set_offset", ptr(off), 5, stream_ptr())
    k2, v2 = torch.randn(2, row, device=cuda), torch.randn(2, row, device=cuda)
    _lib.call("wc_kv_append", ptr(kc), ptr(vc), cap, row, ptr(k2), ptr(v2), 2, ptr(off), ptr(off), stream_ptr())
    assert int(off.item()) == 7
    assert torch.equal(kc[3:5], k1[:2]) and torch.equal(kc[5:7], k2) and torch.equal(kc[7:8], k1[4:5])
    with pytest.raises(ValueError):
        _lib.call("wc_kv_set_offset", ptr(off), -1, stream_ptr())
    # overflow: rows at or past the capacity are dropped and the offset stops
    # at the capacity, so a later read of `offset` rows stays inside the cache
    _lib.call("wc_kv_set_offset", ptr(off), cap - 2, stream_ptr())
    k3, v3 = torch.randn(5, row, device=cuda), torch.randn(5, row, device=cuda)
    before = kc.clone()
    _lib.call("wc_kv_append", ptr(kc), ptr(vc), cap, row, ptr(k3), ptr(v3), 5, ptr(off), ptr(off), stream_ptr())
    assert int(off.item()) == cap
    assert torch.equal(kc[cap - 2:], k3[:2]) and torch.equal(vc[cap - 2:], v3[:2])
    assert torch.equal(kc[:cap - 2], before[:cap - 2])
    # a negative offset writes nothing before the cache and advances from 0
    off.fill_(-3)
    before = kc.clone()
    _lib.call("wc_kv_append", ptr(kc), ptr(vc), cap, row, ptr(k3), ptr(v3), 2, ptr(off), ptr(off), stream_ptr())
    assert torch.equal(kc, before) and int(off.item()) == 0


def test_target_forward_matches_reference_qwen3(cuda):
    """TargetModel (wc_target_embed + wc_target_layer x 2 + wc_target_head) against
    the reference's Qwen3::forward: causal prefill of 9 tokens, then a tree
    block with explicit positions and the tree mask; logits, feature taps and
    the K / V rows of both blocks."""
    from woodcock_amd.synthetic import from_bits
    from woodcock_amd.target import TargetConfig, TargetModel

    cfg = TargetConfig(**detgen.QWEN3)
    g = load_golden("qwen3_small.npz")
    x = detgen.qwen3_inputs()
    w = {k: from_bits(v, cuda) for k, v in detgen.qwen3_weights().items()}
    model = TargetModel(cfg, w, cuda, max_rows=16, feature_layers=detgen.QWEN3_TAPS)
    cache = model.make_cache(32, torch.float32)
    off = torch.zeros(1, dtype=torch.int32, device=cuda)
    logits, taps = model(torch.from_numpy(x["prefill.tokens"]).to(cuda), cache, off)
    assert _nrel(logits.cpu().numpy(), g["prefill.logits"]) < 5e-5
    assert _nrel(torch.stack(taps)[:, :9].cpu().numpy(), g["prefill.taps"]) < 5e-5
    off.fill_(9)
    logits, taps = model(torch.from_numpy(x["tree.tokens"]).to(cuda), cache, off,
                         positions=torch.from_numpy(x["tree.positions"]), mask=torch.from_numpy(g["tree.mask"]))
    assert _nrel(logits.cpu().numpy(), g["tree.logits"]) < 5e-5
    assert _nrel(torch.stack(taps)[:, :6].cpu().numpy(), g["tree.taps"]) < 5e-5
    for i, c in enumerate(cache):
        k = c.keys[0, :, :15].transpose(0, 1).reshape(15, -1).cpu().numpy()
        v = c.values[0, :, :15].transpose(0, 1).reshape(15, -1).cpu().numpy()
        assert _nrel(k, g[f"cache.k{i}"]) < 5e-5 and _nrel(v, g[f"cache.v{i}"]) < 5e-5, i
