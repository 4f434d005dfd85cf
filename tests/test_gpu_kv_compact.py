"""KV compaction on the GPU vs the oracle and the reference goldens: byte for byte."""
import numpy as np
import pytest
import torch

from conftest import load_golden
from oracle import core

pytestmark = pytest.mark.gpu


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.cpu().contiguous().view(torch.uint8).numpy()


def test_reference_goldens(cuda):
    from woodcock_amd.cache import KVCache, compact_cache

    z = load_golden("kv_compact.npz")
    for c in range(12):
        start, keep = int(z[f"c{c}.start"]), z[f"c{c}.keep"].tolist()
        kin, vin = z[f"c{c}.k_in"], z[f"c{c}.v_in"]  # [layers][T][heads*dim]
        layers, T, row = kin.shape
        heads, dim = 2, row // 2
        caches = []
        for l in range(layers):
            kc = KVCache(heads, dim, T + 3, torch.float32, cuda)
            kc.keys[0, :, :T] = torch.from_numpy(kin[l].reshape(T, heads, dim).transpose(1, 0, 2).copy()).to(cuda)
            kc.values[0, :, :T] = torch.from_numpy(vin[l].reshape(T, heads, dim).transpose(1, 0, 2).copy()).to(cuda)
            kc.offset = T
            caches.append(kc)
        compact_cache(caches, start, keep)
        n = int(z[f"c{c}.size"])
        for l, kc in enumerate(caches):
            assert kc.offset == n
            k = kc.keys[0, :, :n].permute(1, 0, 2).reshape(n, row).cpu().numpy()
            v = kc.values[0, :, :n].permute(1, 0, 2).reshape(n, row).cpu().numpy()
            np.testing.assert_array_equal(k, z[f"c{c}.k_out"][l][:n])
            np.testing.assert_array_equal(v, z[f"c{c}.v_out"][l][:n])


def test_known_answer(cuda):
    """tests/cpp/test_main.cpp:42-50."""
    from woodcock_amd.cache import KVCache, compact_cache

    c = KVCache(1, 2, 5, torch.float32, cuda)
    c.keys[0, 0] = torch.arange(5, dtype=torch.float32, device=cuda)[:, None].expand(5, 2)
    c.values.copy_(c.keys)
    compact_cache([c], 1, [0, 2, 3])
    assert c.offset == 4
    assert c.keys[0, 0, :4, 0].tolist() == [0.0, 1.0, 3.0, 4.0]


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 128), (torch.float32, 128), (torch.bfloat16, 64),
                                     (torch.float32, 6)])
def test_28_layer_tree_rounds(cuda, dtype, D):
    """28 layers x 8 kv heads, context 2048 + a verify window of 6; 1000
    seeded rounds with a ~ U{0..5}; chain prefixes (identity: nothing moves) and
    tree paths (strictly increasing keep).  The verify window of every layer/head
    is compared byte for byte with the oracle; rows outside it must not change."""
    from woodcock_amd.cache import make_cache, compact_cache

    L, H, ctx, W = 28, 8, 2048, 6
    rounds = 1000 if (dtype, D) == (torch.bfloat16, 128) else 150
    caches = make_cache(L, H, D, ctx + W, dtype, cuda)
    g = torch.Generator(device=cuda).manual_seed(0)
    for c in caches:
        c.keys.copy_(torch.randn(c.keys.shape, generator=g, device=cuda).to(dtype))
        c.values.copy_(torch.randn(c.values.shape, generator=g, device=cuda).to(dtype))
    rng = np.random.default_rng(8)
    before_prefix = [(_bits(c.keys[0, :, :ctx]), _bits(c.values[0, :, :ctx])) for c in caches[:2]]
    for r in range(rounds):
        a = int(rng.integers(0, 6))
        if r % 2 == 0:
            keep = list(range(a + 1))  # chain: python/woodcock/spec.py:362
        else:
            keep = [0] + sorted(rng.choice(np.arange(1, W), a, replace=False).tolist())
        for c in caches:  # fresh verify-window contents each round
            c.keys[0, :, ctx:].copy_(torch.randn(c.keys[0, :, ctx:].shape, generator=g, device=cuda).to(dtype))
            c.values[0, :, ctx:].copy_(torch.randn(c.values[0, :, ctx:].shape, generator=g, device=cuda).to(dtype))
        host_k = [c.keys[0, :, ctx:].cpu().contiguous().view(torch.uint8).numpy().reshape(H, W, -1).copy()
                  for c in caches]
        host_v = [c.values[0, :, ctx:].cpu().contiguous().view(torch.uint8).numpy().reshape(H, W, -1).copy()
                  for c in caches]
        core.kv_compact(host_k, host_v, 0, keep)
        compact_cache(caches, ctx, keep)
        for li in (0, 13, 27) if r % 10 else range(L):
            got_k = _bits(caches[li].keys[0, :, ctx:]).reshape(H, W, -1)
            got_v = _bits(caches[li].values[0, :, ctx:]).reshape(H, W, -1)
            np.testing.assert_array_equal(got_k, host_k[li], err_msg=f"round {r} layer {li} keep {keep}")
            np.testing.assert_array_equal(got_v, host_v[li], err_msg=f"round {r} layer {li} keep {keep}")
        assert all(c.offset == ctx + a + 1 for c in caches)
    for (k0, v0), c in zip(before_prefix, caches[:2]):
        np.testing.assert_array_equal(_bits(c.keys[0, :, :ctx]), k0)
        np.testing.assert_array_equal(_bits(c.values[0, :, :ctx]), v0)


def test_compaction_from_device_verdict(cuda):
    """keep / n_keep / start straight from a tree verdict, no host round trip."""
    from woodcock_amd import sampling as S
    from woodcock_amd._lib import V_KEEP, V_N_KEEP, WC_MAX_NODES
    from woodcock_amd.cache import compact_cache_dev, make_cache

    tree = S.DraftTree(tokens=[0, 1, 2, 4], parents=[-1, 0, 0, 2], depth=[0, 1, 1, 2])
    lg = np.random.default_rng(0).standard_normal((4, 12)).astype(np.float32)
    lg[np.arange(4), [2, 9, 4, 3]] = 10.0
    verdict = S.verify_tree_greedy_dev(torch.from_numpy(lg).to(cuda), torch.tensor(tree.tokens, dtype=torch.int32,
                                       device=cuda), torch.tensor(tree.parents, dtype=torch.int32, device=cuda))
    caches = make_cache(3, 2, 8, 16, torch.bfloat16, cuda)
    for c in caches:
        c.keys.copy_(torch.randn_like(c.keys, dtype=torch.float32).to(torch.bfloat16))
        c.values.copy_(torch.randn_like(c.values, dtype=torch.float32).to(torch.bfloat16))
    before = [(c.keys.clone(), c.values.clone()) for c in caches]
    start = torch.tensor([5], dtype=torch.int32, device=cuda)
    offset = torch.zeros(1, dtype=torch.int32, device=cuda)
    compact_cache_dev(caches, start, verdict[V_KEEP:V_KEEP + WC_MAX_NODES + 1], verdict[V_N_KEEP:V_N_KEEP + 1],
                      WC_MAX_NODES + 1, offset)
    assert int(offset.item()) == 5 + 3  # keep = [0, 2, 3]
    for (k0, v0), c in zip(before, caches):
        for i, src in enumerate([0, 2, 3]):
            assert torch.equal(c.keys[0, :, 5 + i], k0[0, :, 5 + src])
            assert torch.equal(c.values[0, :, 5 + i], v0[0, :, 5 + src])
        assert torch.equal(c.keys[0, :, :5], k0[0, :, :5])


def test_invalid_keep_moves_nothing(cuda):
    """A non-increasing keep in device memory is caught by the kernel's own check:
    status set, cache untouched.  Host-side lists are validated before launch."""
    from woodcock_amd.cache import compact_cache, compact_cache_dev, make_cache

    caches = make_cache(2, 2, 8, 16, torch.float32, cuda)
    for c in caches:
        c.keys.normal_()
        c.values.normal_()
    before = [c.keys.clone() for c in caches]
    args = torch.tensor([4, 3, 0, 3, 2], dtype=torch.int32, device=cuda)  # start, n, keep
    status = torch.zeros(1, dtype=torch.int32, device=cuda)
    compact_cache_dev(caches, args[0:1], args[2:5], args[1:2], 3, None, status)
    assert int(status.item()) == 1
    for k0, c in zip(before, caches):
        assert torch.equal(c.keys, k0)
    with pytest.raises(ValueError):
        compact_cache(caches, 4, [0, 3, 2])
    with pytest.raises(ValueError):
        compact_cache(caches, 10, [0, 9])
