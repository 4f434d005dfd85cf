"""Verify-width target forward (wc_target_embed + every wc_target_layer +
wc_target_head) against the oracle.

Target.__call__ (python/woodcock/target.py:82-116) is embedding rows, the
decoder layers (target.py:142-156; src/core/qwen3.cpp:75-114), the feature
taps at feature_layers (target.py:26-32,108-111) and the tied LM head over the
final norm (target.py:73-76,113-114).  The oracle runs the same stack as its
drafter forward with the layers' aux stream absent (a plain Qwen3 layer,
pinned by the reference C++ goldens of tests/test_oracle.py and by
tests/test_gpu_target_layer.py), the embedding rows as its residual input, the
target's final norm and the embedding matrix as its head.  Tolerances
(norm-wise relative): 2e-5 with an fp32 cache, 1e-4 with a bf16 cache (both
sides round the appended K/V to bf16; the GPU projections use fp32 = hi + lo
bf16 activations).  The greedy target tokens match wherever the top-2 margin
exceeds 1e-3 of the largest logit.
"""
import numpy as np
import pytest
import torch

from oracle import core
from oracle import sampling as S
from woodcock_amd.synthetic import to_bits
from woodcock_amd.target import TargetConfig, TargetModel, random_target

pytestmark = pytest.mark.gpu

SMALL = TargetConfig(hidden_size=512, num_heads=4, num_kv_heads=2, head_dim=128, intermediate_size=1024,
                     num_layers=6, vocab_size=1000)
# Qwen3-4B widths, two layers: one row runs the one-row kernels with x * gain
# staged per block (QKV, gate / up pair, the 151,936-row logits head)
QWEN3_4B_2L = TargetConfig(hidden_size=2560, num_heads=32, num_kv_heads=8, head_dim=128, intermediate_size=9728,
                           num_layers=2)


def oracle_target(cfg, w, layers, kv_bf16, cap):
    d = cfg.hidden_size
    weights = {}
    for i in range(layers):
        for n in ("input_layernorm.weight", "post_attention_layernorm.weight", "self_attn.q_proj.weight",
                  "self_attn.k_proj.weight", "self_attn.v_proj.weight", "self_attn.o_proj.weight",
                  "self_attn.q_norm.weight", "self_attn.k_norm.weight", "mlp.gate_proj.weight", "mlp.up_proj.weight",
                  "mlp.down_proj.weight"):
            weights[f"layers.{i}.{n}"] = to_bits(w[f"layers.{i}.{n}"])
    weights["embed_tokens.weight"] = np.zeros((1, d), np.uint16)
    weights["fc.weight"] = np.zeros((1, 8), np.uint16)
    weights["norm.weight"] = to_bits(w["norm.weight"])
    weights["lm_head.weight"] = to_bits(w["embed_tokens.weight"])
    od = core.Drafter(dict(hidden_size=d, num_layers=layers, num_heads=cfg.num_heads,
                           num_kv_heads=cfg.num_kv_heads, head_dim=cfg.head_dim,
                           intermediate_size=cfg.intermediate_size, target_hidden_size=d,
                           vocab_size=cfg.vocab_size, rms_norm_eps=cfg.rms_norm_eps, rope_theta=cfg.rope_theta,
                           feature_norm=False), weights)
    return od, od.make_cache(cap, kv_bf16=kv_bf16)


def rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(b))


def random_parents(n, rng):
    parents, dep = [-1], [0]
    for v in range(1, n):
        p = int(rng.integers(0, v))
        parents.append(p)
        dep.append(dep[p] + 1)
    return parents, dep


@pytest.mark.parametrize("cfg,rows,prefix,kv_bf16,tree", [
    (SMALL, 5, 40, False, False),
    (SMALL, 12, 100, False, True),
    (SMALL, 33, 200, True, True),
    (TargetConfig(num_layers=2), 5, 512, True, False),
    (TargetConfig(num_layers=2), 60, 300, True, True),
    (QWEN3_4B_2L, 1, 300, True, False),
    (QWEN3_4B_2L, 8, 2000, True, True),
])
def test_target_forward_matches_oracle(cuda, cfg, rows, prefix, kv_bf16, tree):
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(rows * 7 + prefix)
    w = random_target(cfg, seed=rows + prefix, device=dev)
    feats = (0, cfg.num_layers // 2, cfg.num_layers - 1)
    model = TargetModel(cfg, w, dev, max_rows=64, feature_layers=feats)
    cap = prefix + rows + 8
    dtype = torch.bfloat16 if kv_bf16 else torch.float32
    cache = model.make_cache(cap, dtype)
    g = torch.Generator(device=dev).manual_seed(int(rng.integers(1 << 30)))
    for c in cache:
        c.keys[0, :, :prefix] = torch.randn(c.keys[0, :, :prefix].shape, generator=g, device=dev).to(dtype)
        c.values[0, :, :prefix] = torch.randn(c.values[0, :, :prefix].shape, generator=g, device=dev).to(dtype)
    tokens = rng.integers(0, cfg.vocab_size, rows).astype(np.int32)
    if tree:
        parents, dep = random_parents(rows, rng)
        positions = np.array([prefix + dd for dd in dep], np.int32)
        mask = S.tree_attention_mask(S.DraftTree(list(tokens), parents, dep), prefix).astype(np.uint8)
    else:
        positions, mask = None, None
    # the oracle, one stack per tap depth (its forward returns the last residual only)
    emb = w["embed_tokens.weight"].float().cpu().numpy()[tokens]
    def run_oracle(layers):
        od, oc = oracle_target(cfg, w, layers, kv_bf16, cap)
        for i in range(layers):
            k0, v0 = cache[i].keys[0], cache[i].values[0]
            oc.k[i][:] = to_bits(k0) if kv_bf16 else k0.cpu().numpy()
            oc.v[i][:] = to_bits(v0) if kv_bf16 else v0.cpu().numpy()
        oc.offset = prefix
        hid, out = od.forward(np.zeros(rows, np.int32), emb, oc, positions=positions,
                              mask=None if mask is None else mask[:, : prefix + rows])
        return od, oc, hid, out
    wants = {}
    for f in feats:
        if f + 1 < cfg.num_layers:
            wants[f] = run_oracle(f + 1)[2]
    od, oc, ohid, oout = run_oracle(cfg.num_layers)
    wants[cfg.num_layers - 1] = ohid
    oz = od.logits(oout)

    off = torch.tensor([prefix], dtype=torch.int32, device=dev)
    logits, taps = model(torch.from_numpy(tokens).to(dev), cache, off,
                         positions=None if positions is None else torch.from_numpy(positions),
                         mask=None if mask is None else torch.from_numpy(mask))
    z = logits.cpu().numpy()
    tol = 1e-4 if kv_bf16 else 2e-5
    for f, t in zip(feats, taps):
        assert rel(t.cpu().numpy(), wants[f]) < tol, f
    assert rel(z, oz) < tol
    top2 = np.sort(oz, axis=-1)[:, -2:]
    clear = (top2[:, 1] - top2[:, 0]) > 1e-3 * np.abs(oz).max()
    assert (z.argmax(-1)[clear] == oz.argmax(-1)[clear]).all()
    # every layer's block K/V landed at the offset
    for i in range(cfg.num_layers):
        gk = cache[i].keys[0, :, prefix:prefix + rows].float().cpu().numpy()
        assert rel(gk, oc.keys_f32(i)[:, prefix:prefix + rows]) < max(tol, 1e-2 if kv_bf16 else 0)


def test_target_forward_rejects_bad_shapes(cuda):
    dev = torch.device("cuda", 0)
    model = TargetModel(SMALL, random_target(SMALL, device=dev), dev, max_rows=8)
    cache = model.make_cache(64)
    off = torch.zeros(1, dtype=torch.int32, device=dev)
    with pytest.raises(ValueError):
        model(torch.zeros(9, dtype=torch.int32, device=dev), cache, off)
    with pytest.raises(ValueError):
        model(torch.zeros(4, dtype=torch.int32, device=dev), cache[:3], off)


@pytest.mark.parametrize("cfg,rows,prefix", [(SMALL, 5, 40), (TargetConfig(num_layers=2), 5, 512),
                                             (TargetConfig(num_layers=2), 2, 300), (QWEN3_4B_2L, 1, 300)])
def test_few_row_path_equals_verify_width_path(cuda, cfg, rows, prefix):
    """A chain block that takes the few-row path (no mask, few query vectors)
    gives the logits, taps and appended K/V of the same block forced onto the
    verify-width path by an explicit causal mask, to the fp32 tolerance."""
    dev = torch.device("cuda", 0)
    w = random_target(cfg, seed=rows + prefix + 1, device=dev)
    model = TargetModel(cfg, w, dev, max_rows=64, feature_layers=(0, cfg.num_layers - 1))
    assert model._few_rows_fit(rows, prefix + rows)
    cap = prefix + rows + 8
    g = torch.Generator(device=dev).manual_seed(prefix)
    caches = [model.make_cache(cap), model.make_cache(cap)]
    for ca, cb in zip(*caches):
        ca.keys[0, :, :prefix] = torch.randn(ca.keys[0, :, :prefix].shape, generator=g, device=dev).bfloat16()
        ca.values[0, :, :prefix] = torch.randn(ca.values[0, :, :prefix].shape, generator=g, device=dev).bfloat16()
        cb.keys.copy_(ca.keys)
        cb.values.copy_(ca.values)
        ca.offset = cb.offset = prefix
    tokens = torch.from_numpy(np.random.default_rng(prefix).integers(0, cfg.vocab_size, rows).astype(np.int32))
    off = torch.tensor([prefix], dtype=torch.int32, device=dev)
    causal = np.tril(np.ones((rows, prefix + rows), np.uint8), k=prefix)
    za, ta = model(tokens.to(dev), caches[0], off)
    za, ta = za.clone(), [t.clone() for t in ta]
    zb, tb = model(tokens.to(dev), caches[1], off, mask=torch.from_numpy(causal))
    assert rel(za.cpu().numpy(), zb.cpu().numpy()) < 1e-4
    for x, y in zip(ta, tb):
        assert rel(x.cpu().numpy(), y.cpu().numpy()) < 1e-4
    for ca, cb in zip(*caches):
        kx = ca.keys[0, :, prefix:prefix + rows].float().cpu().numpy()
        ky = cb.keys[0, :, prefix:prefix + rows].float().cpu().numpy()
        assert rel(kx, ky) < 1e-2
