"""Write the golden fixtures in this directory from the reference's own C++ runtime.

Runs only where the reference checkout exists: ``oracle/Makefile`` compiles the
reference sources (src/core/drafter.cpp, src/cache/kv_cache.cpp,
src/sampling/sampling.cpp, ...) into oracle/_ref/libwcref.so and this script
drives it through oracle/refcpp.py.  The fixtures hold inputs and the
reference's outputs only (plus the seeded bf16 weights the outputs depend on).

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import refcpp  # noqa: E402
from woodcock_amd.config import DrafterConfig, tiny_drafter  # noqa: E402
from woodcock_amd.synthetic import random_drafter, to_bits  # noqa: E402

OUT = Path(__file__).resolve().parent
sys.path.insert(0, str(OUT))
import detgen  # noqa: E402


def mid_drafter() -> DrafterConfig:
    """head_dim 128 like Qwen3, target width != drafter width, rope theta 1e6."""
    return DrafterConfig(hidden_size=128, num_layers=1, num_heads=2, num_kv_heads=1, head_dim=128,
                         intermediate_size=256, vocab_size=300, target_hidden_size=96, rope_theta=1_000_000.0)


def drafter_case(name: str, cfg: DrafterConfig, seed: int, ctx: int, tree: bool) -> None:
    """fuse -> prefill forward over ctx tokens -> 3 chain steps (L=1, fed back) ->
    optional tree-drafting forward with explicit positions and mask -> update at L=3."""
    w = {k: to_bits(v) for k, v in random_drafter(cfg, seed=seed).items()}
    cd = cfg.as_dict()
    rd = refcpp.RefDrafter(cd, w)
    rng = np.random.default_rng(seed)
    Dt, d = cfg.target_hidden_size, cfg.hidden_size
    arrays: dict[str, np.ndarray] = {}
    taps = [rng.standard_normal((ctx, Dt)).astype(np.float32) for _ in range(cfg.num_features)]
    tokens = rng.integers(0, cfg.vocab_size, ctx).astype(np.int32)
    for i, t in enumerate(taps):
        arrays[f"in.taps{i}"] = t
    arrays["in.tokens"] = tokens
    g = rd.fuse(taps)
    arrays["out.fuse"] = g
    cache = rd.make_cache()
    hid, out = rd.forward(tokens, g, cache)
    arrays["out.prefill_hidden"], arrays["out.prefill_out"] = hid, out
    out = out[-1:]
    fb = out if cfg.post_norm else hid[-1:]
    steps = rng.integers(0, cfg.vocab_size, 3).astype(np.int32)
    arrays["in.step_tokens"] = steps
    for s in range(3):
        arrays[f"out.step{s}_logits_in"] = rd.logits(out)
        hid, out = rd.forward(steps[s : s + 1], fb, cache)
        arrays[f"out.step{s}_hidden"], arrays[f"out.step{s}_out"] = hid, out
        fb = out if cfg.post_norm else hid
    arrays["out.final_logits"] = rd.logits(out)
    base = ctx + 3
    if tree:
        # two frontier rows at depth 1 and 2 of a tree rooted at the last entry
        m = 2
        positions = np.array([base, base + 1], dtype=np.int32)
        mask = np.zeros((m, base + m), dtype=np.uint8)
        mask[:, :base] = 1
        mask[0, base] = 1
        mask[1, base] = 1
        mask[1, base + 1] = 1
        toks = rng.integers(0, cfg.vocab_size, m).astype(np.int32)
        feat = rng.standard_normal((m, d)).astype(np.float32)
        arrays["in.tree_tokens"], arrays["in.tree_feat"] = toks, feat
        arrays["in.tree_positions"], arrays["in.tree_mask"] = positions, mask
        hid, out = rd.forward(toks, feat, cache, positions=positions, mask=mask)
        arrays["out.tree_hidden"], arrays["out.tree_out"] = hid, out
        cache.trim_to(base)
    # update pass over a+1 = 3 accepted tokens with fused features (spec.py:366-374)
    utaps = [rng.standard_normal((3, Dt)).astype(np.float32) for _ in range(cfg.num_features)]
    utok = rng.integers(0, cfg.vocab_size, 3).astype(np.int32)
    for i, t in enumerate(utaps):
        arrays[f"in.update_taps{i}"] = t
    arrays["in.update_tokens"] = utok
    ug = rd.fuse(utaps)
    hid, out = rd.forward(utok, ug, cache)
    arrays["out.update_hidden"], arrays["out.update_out"] = hid, out
    n = cache.size
    for layer in range(cfg.num_layers):
        arrays[f"out.cache_k{layer}"] = cache.rows(layer, 0, n)
        arrays[f"out.cache_v{layer}"] = cache.rows(layer, 1, n)
    for k, v in w.items():
        arrays["w." + k] = v
    arrays["config"] = np.frombuffer(json.dumps(cd).encode(), dtype=np.uint8)
    rd.close()
    np.savez_compressed(OUT / f"drafter_{name}.npz", **arrays)


def kv_case() -> None:
    """KVCache::compact (src/cache/kv_cache.cpp:21-31) on random strictly increasing keeps."""
    rng = np.random.default_rng(7)
    layers, heads, dim = 3, 2, 4
    arrays = {}
    for c in range(12):
        start = int(rng.integers(0, 6))
        block = int(rng.integers(1, 9))
        n_keep = int(rng.integers(1, block + 1))
        keep = np.sort(rng.choice(block, n_keep, replace=False)).astype(np.int32)
        if c == 0:
            keep = np.arange(n_keep, dtype=np.int32)  # identity: nothing moves
        T = start + block
        cache = refcpp.RefCache.new(layers, heads, dim)
        ks = rng.standard_normal((layers, T, heads * dim)).astype(np.float32)
        vs = rng.standard_normal((layers, T, heads * dim)).astype(np.float32)
        for li in range(layers):
            cache.append(li, ks[li], vs[li], T)
        cache.commit(T)
        cache.compact(start, keep)
        arrays[f"c{c}.start"] = np.int32(start)
        arrays[f"c{c}.keep"] = keep
        arrays[f"c{c}.k_in"], arrays[f"c{c}.v_in"] = ks, vs
        arrays[f"c{c}.size"] = np.int32(cache.size)
        arrays[f"c{c}.k_out"] = np.stack([cache.rows(li, 0) for li in range(layers)])
        arrays[f"c{c}.v_out"] = np.stack([cache.rows(li, 1) for li in range(layers)])
    np.savez_compressed(OUT / "kv_compact.npz", **arrays)


def random_tree(rng, N: int):
    parents = [-1] + [int(rng.integers(0, v)) for v in range(1, N)]
    depth = [0] * N
    for v in range(1, N):
        depth[v] = depth[parents[v]] + 1
    tokens = rng.integers(0, 6, N).tolist()
    return tokens, parents, depth


def verify_case() -> None:
    """verify_tree_greedy and tree_mask (src/sampling/sampling.cpp:85-106), causal_mask
    (src/core/qwen3.cpp:44-53), probs_from_logits (sampling.cpp:9-45)."""
    rng = np.random.default_rng(11)
    arrays = {}
    for c in range(40):
        N = int(rng.integers(1, 24))
        tokens, parents, depth = random_tree(rng, N)
        am = rng.integers(0, 6, N).astype(np.int32)
        path, nxt = refcpp.verify_tree_greedy(am, tokens, parents, depth)
        prefix = int(rng.integers(0, 5))
        arrays[f"t{c}.tokens"] = np.array(tokens, np.int32)
        arrays[f"t{c}.parents"] = np.array(parents, np.int32)
        arrays[f"t{c}.depth"] = np.array(depth, np.int32)
        arrays[f"t{c}.am"] = am
        arrays[f"t{c}.path"] = np.array(path, np.int32)
        arrays[f"t{c}.next"] = np.int32(nxt)
        arrays[f"t{c}.prefix"] = np.int32(prefix)
        arrays[f"t{c}.mask"] = refcpp.tree_mask(tokens, parents, depth, prefix)
    for c, (prefix, L, window) in enumerate([(0, 1, 0), (5, 1, 0), (4, 3, 0), (6, 4, 3), (2, 5, 2), (0, 6, 0)]):
        arrays[f"m{c}.args"] = np.array([prefix, L, window], np.int32)
        arrays[f"m{c}.mask"] = refcpp.causal_mask(prefix, L, window)
    for c, (T, k, p) in enumerate([(1.0, 0, 1.0), (0.5, 0, 1.0), (1.0, 3, 1.0), (1.0, 0, 0.7), (0.7, 5, 0.9)]):
        z = (3.0 * rng.standard_normal(40)).astype(np.float32)
        arrays[f"p{c}.z"] = z
        arrays[f"p{c}.args"] = np.array([T, k, p], np.float32)
        arrays[f"p{c}.p"] = refcpp.probs_from_logits(z, T, k, p)
    np.savez_compressed(OUT / "verify.npz", **arrays)


def ops_case() -> None:
    """The backend operations ops::rmsnorm / linear / rope / silu_mul / softmax /
    attention (include/woodcock/ops.h:9-24; src/backends/cpu_ops.cpp:45-115) on
    the deterministic inputs of detgen.ops_inputs; the fixture holds the outputs."""
    x = detgen.ops_inputs()
    a: dict[str, np.ndarray] = {}
    for c in range(len(detgen.RMS)):
        a[f"rms{c}.y"] = refcpp.rmsnorm(x[f"rms{c}.x"], x[f"rms{c}.w"], float(x[f"rms{c}.eps"]))
    for c in range(len(detgen.LIN)):
        a[f"lin{c}.y"] = refcpp.linear(x[f"lin{c}.x"], x[f"lin{c}.W"])
        a[f"lin{c}.y_acc"] = refcpp.linear(x[f"lin{c}.x"], x[f"lin{c}.W"], x[f"lin{c}.y0"], accumulate=True)
    for c in range(len(detgen.ROPE)):
        a[f"rope{c}.y"] = refcpp.rope(x[f"rope{c}.x"], x[f"rope{c}.pos"], float(x[f"rope{c}.base"]))
    a["silu.y"] = refcpp.silu_mul(x["silu.gate"], x["silu.up"])
    for c in range(len(detgen.SOFTMAX_N)):
        a[f"sm{c}.y"] = refcpp.softmax(x[f"sm{c}.x"])
    for c in range(len(detgen.ATT)):
        a[f"att{c}.out"] = refcpp.attention(x[f"att{c}.q"], x[f"att{c}.K"], x[f"att{c}.V"], x.get(f"att{c}.mask"),
                                            float(x[f"att{c}.scale"]))
    np.savez_compressed(OUT / "ops.npz", **a)


def qwen3_case() -> None:
    """Qwen3::forward (src/core/qwen3.cpp:75-114) of the small two-layer target of
    detgen (hidden 256, 2 x 128 heads, one kv head, SwiGLU 256 -- a shape the
    GPU verify-width layer also runs): a causal prefill of 9 tokens, then a
    6-node tree block with explicit positions and the tree mask.  The fixture
    holds the logits, the feature taps (layers 0, 1, 1) and the KV cache rows."""
    from woodcock_amd.target import TargetConfig

    cfg = TargetConfig(**detgen.QWEN3)
    model = refcpp.RefQwen3(cfg, detgen.qwen3_weights(), detgen.QWEN3_TAPS)
    x = detgen.qwen3_inputs()
    cache = model.make_cache()
    a: dict[str, np.ndarray] = {}
    a["prefill.logits"], a["prefill.taps"] = model.forward(x["prefill.tokens"], cache)
    mask = refcpp.tree_mask(x["tree.tokens"], x["tree.parents"], x["tree.depth"], 9).astype(np.uint8)
    a["tree.mask"] = mask
    a["tree.logits"], a["tree.taps"] = model.forward(x["tree.tokens"], cache, positions=x["tree.positions"],
                                                     mask=mask)
    for li in range(cfg.num_layers):
        a[f"cache.k{li}"] = cache.rows(li, 0)
        a[f"cache.v{li}"] = cache.rows(li, 1)
    model.close()
    np.savez_compressed(OUT / "qwen3_small.npz", **a)


CASES = {
    "drafter": lambda: [drafter_case("tiny", tiny_drafter(), seed=1, ctx=9, tree=True),
                        drafter_case("tiny_prenorm", tiny_drafter(post_norm=False), seed=2, ctx=7, tree=False),
                        drafter_case("tiny_window", tiny_drafter(window=5), seed=3, ctx=9, tree=False),
                        drafter_case("tiny_2layer", tiny_drafter(num_layers=2), seed=4, ctx=6, tree=True),
                        drafter_case("mid", mid_drafter(), seed=5, ctx=40, tree=True)],
    "kv": kv_case,
    "verify": verify_case,
    "ops": ops_case,
    "qwen3": qwen3_case,
}


def main():
    """python tests/golden/make_golden.py [case ...]   (default: every case)"""
    if not refcpp.available():
        sys.exit("oracle/_ref/libwcref.so is missing: run `make -C oracle` where the reference exists")
    names = sys.argv[1:] or list(CASES)
    for n in names:
        CASES[n]()
    for f in sorted(OUT.glob("*.npz")):
        print(f.name, f.stat().st_size)


if __name__ == "__main__":
    main()
