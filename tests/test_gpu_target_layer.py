"""Verify-width target layer (wc_target_layer) against the oracle.

A Qwen3 decoder layer (python/woodcock/target.py:142-156) is the drafter's
decoder layer without the token stream, so the oracle is its drafter forward
with one layer and no aux weights (oracle/wc_oracle.c, pinned by the reference
C++ goldens of tests/test_oracle.py).  Blocks of 1..60 rows with a random draft
tree: positions n + depth, the tree mask over the prefix and the ancestors
(python/woodcock/sampling.py:118-128), K/V appended at the cache offset.

Tolerances (norm-wise relative): 2e-5 with an fp32 cache -- the projections
run as bf16 MFMA on an fp32 = hi + lo bf16 split of the activations (~2^-17
relative per product); 1e-2 with a bf16 cache.
"""
import numpy as np
import pytest
import torch

from oracle import core
from oracle import sampling as S
from woodcock_amd.cache import KVCache
from woodcock_amd.synthetic import to_bits
from woodcock_amd.target import TargetConfig, TargetLayer, random_layer

pytestmark = pytest.mark.gpu

SMALL = TargetConfig(hidden_size=512, num_heads=4, num_kv_heads=2, head_dim=128, intermediate_size=1024)
FULL = TargetConfig()  # Qwen3-1.7B layer shape


def oracle_layer(cfg: TargetConfig, w: dict, x: np.ndarray, k0: np.ndarray, v0: np.ndarray, kv_bf16: bool,
                 offset: int, positions, mask):
    d = cfg.hidden_size
    weights = {f"layers.0.{n}": to_bits(t) for n, t in w.items()}
    weights["embed_tokens.weight"] = np.zeros((1, d), np.uint16)
    weights["fc.weight"] = np.zeros((1, 8), np.uint16)
    weights["norm.weight"] = np.full(d, 0x3F80, np.uint16)
    weights["lm_head.weight"] = np.zeros((1, d), np.uint16)
    od = core.Drafter(dict(hidden_size=d, num_layers=1, num_heads=cfg.num_heads, num_kv_heads=cfg.num_kv_heads,
                           head_dim=cfg.head_dim, intermediate_size=cfg.intermediate_size, target_hidden_size=d,
                           vocab_size=1, rms_norm_eps=cfg.rms_norm_eps, rope_theta=cfg.rope_theta,
                           feature_norm=False), weights)
    cache = od.make_cache(k0.shape[1], kv_bf16=kv_bf16)
    cache.k[0][:] = k0
    cache.v[0][:] = v0
    cache.offset = offset
    M = x.shape[0]
    hid, _ = od.forward(np.zeros(M, np.int32), x, cache, positions=positions,
                        mask=None if mask is None else mask[:, : offset + M])
    return hid, cache


def random_tree(M: int, rng) -> S.DraftTree:
    parents = [-1] + [int(rng.integers(0, v)) for v in range(1, M)]
    depth = [0] * M
    for v in range(1, M):
        depth[v] = depth[parents[v]] + 1
    return S.DraftTree([0] * M, parents, depth)


def norm_err(a, b):
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


@pytest.mark.parametrize("cfg,M,prefix,kv_bf16,tree", [
    (SMALL, 1, 40, False, False),
    (SMALL, 5, 64, False, False),
    (SMALL, 16, 100, False, True),
    (SMALL, 33, 100, False, True),
    (SMALL, 60, 300, False, True),
    (SMALL, 60, 300, True, True),
    (FULL, 16, 2048, True, True),
    (FULL, 60, 2048, False, True),
    (FULL, 60, 2048, True, True),
])
def test_target_layer_matches_oracle(cuda, cfg, M, prefix, kv_bf16, tree):
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(M * 1000 + prefix + int(kv_bf16))
    w = random_layer(cfg, seed=M + prefix, device=dev)
    layer = TargetLayer(cfg, w, dev)
    cap = prefix + M + 8
    dtype = torch.bfloat16 if kv_bf16 else torch.float32
    cache = KVCache(cfg.num_kv_heads, cfg.head_dim, cap, dtype, dev)
    g = torch.Generator(device=dev).manual_seed(int(rng.integers(1 << 30)))
    cache.keys[0, :, :prefix] = torch.randn(cache.keys[0, :, :prefix].shape, generator=g, device=dev).to(dtype)
    cache.values[0, :, :prefix] = torch.randn(cache.values[0, :, :prefix].shape, generator=g, device=dev).to(dtype)
    x = torch.randn(M, cfg.hidden_size, generator=g, device=dev)
    if tree:
        t = random_tree(M, rng)
        positions = np.array([prefix + dep for dep in t.depth], np.int32)
        mask = S.tree_attention_mask(t, prefix)
    else:
        positions, mask = None, None
    before_k = cache.keys[0, :, :prefix].clone()
    k0 = to_bits(cache.keys[0]) if kv_bf16 else cache.keys[0].cpu().numpy()
    v0 = to_bits(cache.values[0]) if kv_bf16 else cache.values[0].cpu().numpy()
    want, ocache = oracle_layer(cfg, w, x.cpu().numpy(), k0, v0, kv_bf16, prefix, positions,
                                None if mask is None else mask.astype(np.uint8))
    off = torch.tensor([prefix], dtype=torch.int32, device=dev)
    got = layer(x.clone(), cache, off,
                positions=None if positions is None else torch.from_numpy(positions),
                mask=None if mask is None else torch.from_numpy(mask.astype(np.uint8))).cpu().numpy()
    tol = 1e-2 if kv_bf16 else 2e-5
    assert norm_err(got, want) < tol, norm_err(got, want)
    # the block's K / V rows appended at the offset
    gk = cache.keys[0, :, prefix:prefix + M].float().cpu().numpy()
    gv = cache.values[0, :, prefix:prefix + M].float().cpu().numpy()
    wk = ocache.keys_f32(0)[:, prefix:prefix + M]
    wv = ocache.values_f32(0)[:, prefix:prefix + M]
    assert norm_err(gk, wk) < tol and norm_err(gv, wv) < tol
    # the prefix is untouched
    assert torch.equal(cache.keys[0, :, :prefix], before_k)


@pytest.mark.parametrize("cfg,M,prefix", [(SMALL, 7, 42), (SMALL, 60, 300), (FULL, 60, 2048)])
def test_target_layer_mask_row_stride(cuda, cfg, M, prefix):
    """The verify attention reads mask rows that are 16-byte aligned 16 bytes at
    a time and any other mask byte by byte: the same tree mask contiguous (row
    stride prefix + M), as a row view of a 16-byte-padded buffer, and as a view
    one byte into a buffer gives the same bits, within the bf16 tolerance of the
    oracle.  The cache slots past the block hold NaN: the last, partial key
    chunk of a split must not let them into the outputs."""
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(7 * M + prefix)
    w = random_layer(cfg, seed=M + prefix + 1, device=dev)
    layer = TargetLayer(cfg, w, dev)
    cap = prefix + M + 40
    cache = KVCache(cfg.num_kv_heads, cfg.head_dim, cap, torch.bfloat16, dev)
    g = torch.Generator(device=dev).manual_seed(int(rng.integers(1 << 30)))
    cache.keys[0, :, :prefix] = torch.randn(cache.keys[0, :, :prefix].shape, generator=g, device=dev).bfloat16()
    cache.values[0, :, :prefix] = torch.randn(cache.values[0, :, :prefix].shape, generator=g, device=dev).bfloat16()
    cache.keys[0, :, prefix + M:] = float("nan")
    cache.values[0, :, prefix + M:] = float("nan")
    k_init, v_init = cache.keys.clone(), cache.values.clone()
    x = torch.randn(M, cfg.hidden_size, generator=g, device=dev)
    t = random_tree(M, rng)
    positions = np.array([prefix + dep for dep in t.depth], np.int32)
    mask = S.tree_attention_mask(t, prefix).astype(np.uint8)
    assert mask.shape[1] % 16 != 0
    pad = torch.zeros(M, (mask.shape[1] + 15) // 16 * 16, dtype=torch.uint8, device=dev)
    pad[:, : mask.shape[1]] = torch.from_numpy(mask).to(dev)
    odd = torch.zeros(M, mask.shape[1] + 1, dtype=torch.uint8, device=dev)
    odd[:, 1:] = torch.from_numpy(mask).to(dev)
    assert odd[:, 1:].data_ptr() % 16 != 0
    off = torch.tensor([prefix], dtype=torch.int32, device=dev)
    pos = torch.from_numpy(positions)
    got = {}
    for name, m in (("contiguous", torch.from_numpy(mask)), ("padded rows", pad[:, : mask.shape[1]]),
                    ("unaligned base", odd[:, 1:])):
        cache.keys.copy_(k_init)
        cache.values.copy_(v_init)
        got[name] = layer(x.clone(), cache, off, positions=pos, mask=m).cpu().numpy()
        assert np.isfinite(got[name]).all(), name
    np.testing.assert_array_equal(got["padded rows"], got["contiguous"])
    np.testing.assert_array_equal(got["unaligned base"], got["contiguous"])
    k0 = to_bits(k_init[0])
    v0 = to_bits(v_init[0])
    want, _ = oracle_layer(cfg, w, x.cpu().numpy(), k0, v0, True, prefix, positions, mask)
    assert norm_err(got["padded rows"], want) < 1e-2, norm_err(got["padded rows"], want)


def test_target_layer_rejects_bad_shapes(cuda):
    dev = torch.device("cuda", 0)
    layer = TargetLayer(SMALL, random_layer(SMALL, device=dev), dev)
    cache = KVCache(SMALL.num_kv_heads, SMALL.head_dim, 128, torch.float32, dev)
    off = torch.zeros(1, dtype=torch.int32, device=dev)
    with pytest.raises(ValueError):
        layer(torch.zeros(65, SMALL.hidden_size, device=dev), cache, off)
    with pytest.raises(ValueError):
        layer(torch.zeros(4, SMALL.hidden_size + 1, device=dev), cache, off)


@pytest.mark.parametrize("rows,cols", [(16, 32), (48, 96), (4096, 2048), (2048, 6144)])
def test_fragment_major_weight_layout(cuda, rows, cols):
    """wc_weights_frag: tile T, step s, lane l holds w[16 T + l % 16][32 s + 8 (l / 16) .. + 8]
    (the A fragment of v_mfma_f32_16x16x32_bf16), the same bytes as the row-major matrix."""
    from woodcock_amd.target import frag_weights

    g = torch.Generator(device=cuda).manual_seed(rows + cols)
    w = torch.randn(rows, cols, generator=g, device=cuda).bfloat16()
    got = frag_weights(w).view(torch.int16).cpu().numpy().reshape(-1)
    a = w.view(torch.int16).cpu().numpy().reshape(rows // 16, 16, cols // 32, 4, 8)
    want = a.transpose(0, 2, 3, 1, 4).reshape(-1)  # [T][s][g][i][e]: lane l = 16 g + i
    np.testing.assert_array_equal(got, want)
