"""Greedy verification on the GPU vs the oracle: bit-exact accepted lengths,
next tokens, accepted paths and argmax indices (lowest index wins a tie)."""
import numpy as np
import pytest
import torch

from conftest import load_golden
from oracle import sampling as osamp

pytestmark = pytest.mark.gpu

V = 151936


def planted_chain_logits(rng, K, V, n_match, scale=3.0):
    """logits [K+1, V] ~ N(0, scale^2); draft d_i equals the row argmax for i < n_match
    and differs from it at row n_match (python/woodcock/spec.py:355-361 setting)."""
    lg = (scale * rng.standard_normal((K + 1, V))).astype(np.float32)
    am = lg.argmax(-1)
    drafts = []
    for i in range(K):
        if i < n_match:
            drafts.append(int(am[i]))
        else:
            d = int(rng.integers(0, V))
            if d == am[i]:
                d = (d + 1) % V
            drafts.append(d)
    return lg, drafts


def test_chain_round_k4_full_vocab(cuda):
    """Chain verify at K=4: [5, 151936] fp32 ~N(0, 3^2), argmax planted for the first 2 positions."""
    from woodcock_amd import sampling as S

    rng = np.random.default_rng(1)
    lg, drafts = planted_chain_logits(rng, 4, V, 2)
    want = osamp.verify_chain_greedy(lg, drafts)
    assert want[0] == 2
    got = S.verify_chain_greedy(torch.from_numpy(lg).to(cuda), drafts)
    assert got == want


@pytest.mark.parametrize("vocab", [1, 3, 5, 4095, 4096, 4097, 16384, 151936])
def test_chain_sweep_matches_oracle(cuda, vocab):
    from woodcock_amd import sampling as S

    rng = np.random.default_rng(vocab)
    for trial in range(12):
        K = int(rng.integers(0, 9))
        n_match = int(rng.integers(0, K + 1))
        lg, drafts = planted_chain_logits(rng, K, vocab, n_match)
        want = osamp.verify_chain_greedy(lg, drafts)
        got = S.verify_chain_greedy(torch.from_numpy(lg).to(cuda), drafts)
        assert got == want, (vocab, trial, K, n_match)


def test_chain_full_acceptance_and_k_max(cuda):
    from woodcock_amd import sampling as S

    rng = np.random.default_rng(3)
    for K in (1, 8, 63):
        lg, drafts = planted_chain_logits(rng, K, 1000, K)
        assert S.verify_chain_greedy(torch.from_numpy(lg).to(cuda), drafts) == (K, int(lg[K].argmax()))


def test_argmax_ties_take_lowest_index(cuda):
    from woodcock_amd import sampling as S

    lg = np.zeros((6, V), dtype=np.float32)
    lg[1, [7, 70000, 151935]] = 2.5
    lg[2, [151935, 40000]] = -0.0  # all zeros: index 0
    lg[3] = -1.0
    lg[3, [4096, 4095, 8191]] = 1.0  # straddles block chunks
    lg[4, :] = np.float32(-np.inf)
    lg[4, 99] = -1e30
    lg[5, 151935] = 1.0
    got = S.argmax_rows(torch.from_numpy(lg).to(cuda)).cpu().numpy()
    np.testing.assert_array_equal(got, np.argmax(lg, axis=-1))
    assert got.tolist() == [0, 7, 0, 4095, 99, 151935]


def test_strided_and_unaligned_rows(cuda):
    """Row stride larger than vocab (an odd stride takes the scalar-load path)."""
    from woodcock_amd import sampling as S

    rng = np.random.default_rng(4)
    for ld in (V + 4, V + 3):
        full = rng.standard_normal((5, ld)).astype(np.float32)
        t = torch.from_numpy(full).to(cuda)[:, :V]
        assert t.stride(0) == ld
        np.testing.assert_array_equal(S.argmax_rows(t).cpu().numpy(), np.argmax(full[:, :V], axis=-1))
        drafts = np.argmax(full[:4, :V], axis=-1).tolist()
        drafts[3] = (drafts[3] + 1) % V
        assert S.verify_chain_greedy(t, drafts) == osamp.verify_chain_greedy(full[:, :V], drafts)


def test_repeated_launches_reset_device_state(cuda):
    """The last block clears the argmax slots and the counter: 200 back-to-back
    verifications on one workspace stay exact."""
    from woodcock_amd import sampling as S

    rng = np.random.default_rng(5)
    cases, verdicts = [], []
    for _ in range(200):
        K = int(rng.integers(0, 6))
        lg, drafts = planted_chain_logits(rng, K, 20000, int(rng.integers(0, K + 1)))
        d = torch.tensor(drafts, dtype=torch.int32, device=cuda)
        verdicts.append(S.verify_chain_greedy_dev(torch.from_numpy(lg).to(cuda), d))
        cases.append((lg, drafts))
    torch.cuda.synchronize()
    from woodcock_amd.runtime import read_verdict

    for (lg, drafts), v in zip(cases, verdicts):
        r = read_verdict(v)
        n, nxt = osamp.verify_chain_greedy(lg, drafts)
        assert (r.n_accepted, r.next, r.n_keep) == (n, nxt, n + 1)
        assert list(r.tokens[: n + 1]) == drafts[:n] + [nxt]
        assert list(r.keep[: n + 1]) == list(range(n + 1))


def _tree_logits(am, vocab, rng):
    lg = rng.standard_normal((len(am), vocab)).astype(np.float32)
    lg[np.arange(len(am)), am] = 10.0
    return lg


def test_tree_matches_reference_goldens(cuda):
    from woodcock_amd import sampling as S

    z = load_golden("verify.npz")
    rng = np.random.default_rng(6)
    for c in range(40):
        tree = S.DraftTree(z[f"t{c}.tokens"].tolist(), z[f"t{c}.parents"].tolist(), z[f"t{c}.depth"].tolist())
        lg = _tree_logits(z[f"t{c}.am"], 6, rng)
        path, nxt = S.verify_tree_greedy(torch.from_numpy(lg).to(cuda), tree)
        assert path == z[f"t{c}.path"].tolist() and nxt == int(z[f"t{c}.next"]), c


def test_tree_known_answer(cuda):
    """tests/test_sampling.py:193-196: tokens [0,1,2,4], parents [-1,0,0,2], argmax [2,9,4,3]."""
    from woodcock_amd import sampling as S

    tree = S.DraftTree(tokens=[0, 1, 2, 4], parents=[-1, 0, 0, 2], depth=[0, 1, 1, 2])
    lg = _tree_logits(np.array([2, 9, 4, 3]), 12, np.random.default_rng(0))
    assert S.verify_tree_greedy(torch.from_numpy(lg).to(cuda), tree) == ([2, 3], 3)


def test_sixty_node_tree_full_vocab(cuda):
    """60-node tree, depth 6 / branching 4, over the full vocabulary; duplicate
    sibling tokens resolve to the first child in draw order."""
    from woodcock_amd import sampling as S

    rng = np.random.default_rng(7)
    for trial in range(20):
        parents, depth = [-1], [0]
        frontier = [0]
        while len(parents) < 60:
            nxt = []
            for p in frontier:
                for _ in range(4):
                    if len(parents) < 60 and depth[p] < 6:
                        parents.append(p)
                        depth.append(depth[p] + 1)
                        nxt.append(len(parents) - 1)
            frontier = nxt or frontier
        N = len(parents)
        tokens = rng.integers(0, 50, N).tolist()
        am = rng.integers(0, 50, N)
        # make a long accepted path likely
        v = 0
        for _ in range(6):
            kids = [c for c in range(N) if parents[c] == v]
            if not kids:
                break
            c = kids[int(rng.integers(0, len(kids)))]
            am[v] = tokens[c]
            v = c
        tree = S.DraftTree(tokens, parents, depth)
        lg = (3.0 * rng.standard_normal((N, V))).astype(np.float32)
        lg[np.arange(N), am] = 100.0
        want = osamp.verify_tree_greedy(am, osamp.DraftTree(tokens, parents, depth))
        assert S.verify_tree_greedy(torch.from_numpy(lg).to(cuda), tree) == want, trial


def test_invalid_arguments_raise(cuda):
    from woodcock_amd import sampling as S

    lg = torch.zeros(65, 10, device=cuda)
    with pytest.raises(ValueError):
        S.verify_chain_greedy(lg, list(range(64)))
    with pytest.raises(ValueError):
        S.verify_chain_greedy(torch.zeros(3, 10, device=cuda), [1])
    with pytest.raises(ValueError):
        S.verify_chain_greedy(torch.zeros(3, 10), [1, 2])  # host tensor: no CPU fallback
    with pytest.raises(ValueError):
        S.verify_chain_greedy(torch.zeros(3, 10, device=cuda, dtype=torch.float16), [1, 2])
    # a parent index outside the tree, seen only on the device: the kernel's own
    # check flags the verdict, which the host read turns into ValueError
    from woodcock_amd.runtime import read_verdict

    v = S.verify_tree_greedy_dev(torch.zeros(2, 10, device=cuda), torch.tensor([0, 1], dtype=torch.int32, device=cuda),
                                 torch.tensor([-1, 5], dtype=torch.int32, device=cuda))
    with pytest.raises(ValueError):
        read_verdict(v)
