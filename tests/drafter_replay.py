"""Replays the call sequence recorded in a drafter golden fixture on any drafter
implementation (the oracle, or the HIP drafter through an adapter) and returns
the outputs under the fixture's "out.*" keys."""
from __future__ import annotations

import json

import numpy as np


def fixture_config(z: dict) -> dict:
    return json.loads(bytes(z["config"]).decode())


def fixture_weights(z: dict) -> dict:
    return {k[2:]: v for k, v in z.items() if k.startswith("w.")}


def replay(d, z: dict) -> dict:
    """d provides fuse(taps), make_cache(cap), forward(tokens, feat, cache, positions=, mask=),
    feedback(hidden, out), logits(out), cache_rows(cache, layer) -> (K, V) [n][Hk*D],
    and caches with a settable .offset."""
    cfg = fixture_config(z)
    nf = cfg.get("num_features", 3)
    res = {}
    taps = [z[f"in.taps{i}"] for i in range(nf)]
    ctx = len(z["in.tokens"])
    g = d.fuse(taps)
    res["out.fuse"] = g
    cache = d.make_cache(ctx + 16)
    hid, out = d.forward(z["in.tokens"], g, cache)
    res["out.prefill_hidden"], res["out.prefill_out"] = hid, out
    out = out[-1:]
    fb = d.feedback(hid[-1:], out)
    for s in range(3):
        res[f"out.step{s}_logits_in"] = d.logits(out)
        hid, out = d.forward(z["in.step_tokens"][s : s + 1], fb, cache)
        res[f"out.step{s}_hidden"], res[f"out.step{s}_out"] = hid, out
        fb = d.feedback(hid, out)
    res["out.final_logits"] = d.logits(out)
    base = ctx + 3
    if "in.tree_tokens" in z:
        hid, out = d.forward(z["in.tree_tokens"], z["in.tree_feat"], cache, positions=z["in.tree_positions"],
                             mask=z["in.tree_mask"])
        res["out.tree_hidden"], res["out.tree_out"] = hid, out
        cache.offset = base
    utaps = [z[f"in.update_taps{i}"] for i in range(nf)]
    ug = d.fuse(utaps)
    hid, out = d.forward(z["in.update_tokens"], ug, cache)
    res["out.update_hidden"], res["out.update_out"] = hid, out
    for layer in range(cfg["num_layers"]):
        k, v = d.cache_rows(cache, layer)
        res[f"out.cache_k{layer}"], res[f"out.cache_v{layer}"] = k, v
    return res


def compare(res: dict, z: dict, rtol: float, what: str) -> None:
    """Every output within rtol of the fixture, scaled by the output's own magnitude
    (max |a - b| <= rtol * max |b|) -- a norm-wise relative bound that stays
    meaningful for entries near zero."""
    missing = [k for k in z if k.startswith("out.") and k not in res]
    assert not missing, f"{what}: replay produced no {missing}"
    for k, ref in z.items():
        if not k.startswith("out."):
            continue
        got = np.asarray(res[k], dtype=np.float64)
        ref = np.asarray(ref, dtype=np.float64)
        assert got.shape == ref.shape, f"{what} {k}: shape {got.shape} != {ref.shape}"
        scale = max(np.abs(ref).max(), 1e-30)
        err = np.abs(got - ref).max() / scale
        assert err <= rtol, f"{what} {k}: max error {err:.3e} relative to max |ref| exceeds {rtol:.1e}"
