"""End-to-end invariant of greedy speculative decoding on the GPU: whatever the
drafter proposes, the emitted stream equals plain autoregressive greedy
decoding of the same target (python/woodcock/spec.py:1-15;
tests/test_spec_model.py:51-56, 125-135, 193 of the reference).

The target is a random-init Qwen3-shaped ``TargetModel`` (full Qwen3-1.7B
width, three decoder layers, an 8192-token vocabulary, fp32 KV) run entirely
by the HIP library; the autoregressive stream comes from one-row forwards of
that model (``generate_autoregressive``).  The speculative side runs:

* chain rounds whose drafts are planted from the known continuation with
  random corruptions (every accept length 0..K occurs), K = 1, 3, 4 -- the
  partial accepts, the kept prefix of the target KV and the overwrite of the
  rejected entries, the drafter update;
* ``SpeculativeDecoder.generate`` with the real drafter: ``StaticPolicy(k)``
  chains eagerly and replayed from captured graphs, ``CostAwareChain``, a
  width-3 tree (mask, compaction along the branch), and a width-1 tree (the
  unfused tree path of a chain);

and after every round the target's and the drafter's offsets equal the
committed count.  A speculative token may differ from the autoregressive one
only where the autoregressive row's fp32 top-2 margin is below EPS: the verify
block's rows and the one-row forward sum in different orders
(scripts/diagnose_greedy_mismatch.py:1-52 of the reference); such steps are
counted, printed, and the comparison stops there.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

EPS = 1e-3  # fp32 logits; the row scale here is ~1
PROMPT = 12
NEW = 40


def _setup(cuda):
    from woodcock_amd.config import qwen3_1p7b_drafter
    from woodcock_amd.drafter import Drafter
    from woodcock_amd.synthetic import draft_vocab, random_drafter
    from woodcock_amd.target import TargetConfig, TargetModel, random_target

    tcfg = TargetConfig(num_layers=3, vocab_size=8192)
    model = TargetModel(tcfg, random_target(tcfg, seed=81, device=cuda), cuda, max_rows=64, feature_layers=(0, 1, 2))
    dcfg = qwen3_1p7b_drafter()
    dcfg.vocab_size = tcfg.vocab_size
    dcfg.feature_layers = [0, 1, 2]
    d = Drafter(dcfg, random_drafter(dcfg, seed=82, device=cuda), cuda, torch.bfloat16)
    d.restrict_vocab(draft_vocab(dcfg.vocab_size, 4096, seed=83))
    prompt = np.random.default_rng(84).integers(0, tcfg.vocab_size, PROMPT).tolist()
    return model, d, prompt


@pytest.fixture(scope="module")
def world(cuda):
    """(model, drafter, prompt, autoregressive stream, top-2 margins per step)."""
    from woodcock_amd.spec import generate_autoregressive

    model, d, prompt = _setup(cuda)
    margins = {}

    def on_logits(step, row):
        top = torch.topk(row.float(), 2).values.cpu().numpy()
        margins[step] = float(top[0] - top[1])

    cache = model.make_cache(PROMPT + NEW + 80, dtype=torch.float32)
    ref, st = generate_autoregressive(model, cache, prompt, NEW + 1, on_logits=on_logits)
    assert len(ref) == NEW + 1 and st.rounds == NEW
    assert int(cache[0].offset) == PROMPT + NEW
    m = np.array([margins[i] for i in range(NEW + 1)])
    print(f"autoregressive stream: {ref[:12]}...; {len(set(ref))} distinct tokens; min top-2 margin {m.min():.3g}")
    return model, d, prompt, ref, m


def _compare(out, ref, margins, what):
    """Token-for-token equality; a difference only at a step whose autoregressive
    margin is below EPS (then counted, and the streams are not compared beyond)."""
    n = min(len(out), len(ref))
    assert n > 1, what
    for i in range(n):
        if out[i] != ref[i]:
            assert margins[i] < EPS, f"{what}: token {i} is {out[i]}, autoregressive {ref[i]} (margin {margins[i]:.3g})"
            print(f"{what}: near-tie at token {i} (margin {margins[i]:.3g}); compared {i} tokens")
            return i
    return n


def _decoder(world, policy, cuda, k_max=4, depth=0, use_graphs=False):
    from woodcock_amd.spec import SpeculativeDecoder, TargetRunner, target_prefill

    model, d, prompt, ref, _ = world
    cache = model.make_cache(PROMPT + NEW + 80, dtype=torch.float32)
    runner = TargetRunner(model, cache)
    n, _ = target_prefill(model, cache, prompt)
    dec = SpeculativeDecoder(d, runner, policy, capacity=PROMPT + NEW + 80, k_max=k_max, max_tree_depth=depth,
                             use_graphs=use_graphs)
    root = torch.randn(1, d.cfg.hidden_size, generator=torch.Generator(device=cuda).manual_seed(85), device=cuda)
    dec.start(n, ref[0], root)
    return dec, runner


def _check_offsets(dec, runner):
    n = dec.rnd.committed()
    assert n == dec.n, (n, dec.n)
    assert all(c.offset == n for c in runner.cache)
    assert all(c.offset == n for c in dec.rnd.cache)


@pytest.mark.parametrize("k", [1, 3, 4])
def test_planted_chain_rounds_equal_autoregressive(world, cuda, k):
    """Chain rounds through ChainRound's device path with drafts planted from the
    autoregressive continuation (each position corrupted with probability 0.3),
    so every accept length from 0 to K occurs."""
    from woodcock_amd.policies import StaticPolicy

    model, d, prompt, ref, margins = world
    dec, runner = _decoder(world, StaticPolicy(k), cuda, k_max=k)
    r = dec.rnd
    rng = np.random.default_rng(86 + k)
    out = [ref[0]]
    accepts = []
    while len(out) < NEW:
        pos = len(out) - 1  # out[-1] == x_n
        fut = ref[pos + 1:pos + 1 + k] + [0] * k
        plant = [t if rng.random() > 0.3 else int(rng.integers(0, model.cfg.vocab_size)) for t in fut[:k]]
        r.enqueue_seq()
        r.drafts[:k].copy_(torch.tensor(plant, dtype=torch.int32))
        logits, taps = runner.verify_forward(r.seq, k + 1, r.n_dev())
        r.enqueue_verify_commit(logits, taps, k)
        r.enqueue_readback()
        res = r.finish()
        dec.n += res.n_accepted + 1
        dec.x_n = res.tokens[-1]
        out += res.tokens
        accepts.append(res.n_accepted)
        _check_offsets(dec, runner)
        if _compare(out, ref, margins, f"planted chain K={k}") < min(len(out), len(ref)):
            return
    assert set(accepts) >= {0, k}, accepts
    print(f"K={k}: accept lengths {accepts}")


@pytest.mark.parametrize("use_graphs", [False, True])
def test_static_chain_generate_equals_autoregressive(world, cuda, use_graphs):
    from woodcock_amd.policies import StaticPolicy

    _, _, _, ref, margins = world
    dec, runner = _decoder(world, StaticPolicy(4), cuda, use_graphs=use_graphs)
    out, st = dec.generate(NEW)
    _check_offsets(dec, runner)
    assert st.rounds == dec.rnd.syncs
    _compare(out, ref, margins, f"StaticPolicy(4) graphs={use_graphs}")


def test_cost_aware_chain_generate_equals_autoregressive(world, cuda):
    from woodcock_amd.policies import CostAwareChain

    _, _, _, ref, margins = world
    costs = dict(step_ms=0.1, head_ms=0.03, verify_ms={n: 2.0 + 0.25 * n for n in range(1, 10)})
    dec, runner = _decoder(world, CostAwareChain(**costs), cuda, k_max=8)
    out, st = dec.generate(NEW)
    _check_offsets(dec, runner)
    _compare(out, ref, margins, "CostAwareChain")


@pytest.mark.parametrize("width", [1, 3])
def test_tree_rounds_equal_autoregressive(world, cuda, width):
    """Trees go through drafting on the device, the verify forward with the tree
    mask, the greedy walk, compaction along the branch and the update; width 1
    is a chain taken down the tree path."""
    from woodcock_amd.policies import Plan, StaticPolicy

    _, _, _, ref, margins = world
    depth = 3
    policy = StaticPolicy(depth, width, 8 if width > 1 else depth)
    dec, runner = _decoder(world, policy, cuda, depth=depth)
    out = [ref[0]]
    while len(out) < NEW:
        res = dec.tree_round(Plan(depth, width, policy.budget))
        dec.n += len(res.tokens)
        dec.x_n = res.tokens[-1]
        out += res.tokens
        _check_offsets(dec, runner)
    _compare(out, ref, margins, f"tree width {width}")
