"""Deterministic fixture inputs: the same bits on every platform and library version.

Values come from an integer hash (splitmix64 over uint64 counters, wraparound
arithmetic) turned into floats with exact operations only, so a fixture can
store the reference's outputs alone and the tests regenerate its inputs.
Used by make_golden.py (which writes the outputs) and by the tests that read
them.
"""
from __future__ import annotations

import numpy as np

_M = np.uint64(0xFFFFFFFFFFFFFFFF)


def _splitmix(x: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = x + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def det_uniform(seed: int, shape, scale: float = 1.0) -> np.ndarray:
    """float32 uniform on [-scale, scale): 24 hash bits per value."""
    n = int(np.prod(shape))
    with np.errstate(over="ignore"):
        ctr = np.arange(n, dtype=np.uint64) + np.uint64(seed) * np.uint64(0x100000001B3)
    h = _splitmix(ctr & _M) >> np.uint64(40)  # 24 bits
    u = h.astype(np.float32) * np.float32(2.0 ** -23) - np.float32(1.0)  # exact: [-1, 1)
    return (u * np.float32(scale)).astype(np.float32).reshape(shape)


def det_ints(seed: int, shape, hi: int) -> np.ndarray:
    n = int(np.prod(shape))
    with np.errstate(over="ignore"):
        ctr = np.arange(n, dtype=np.uint64) + np.uint64(seed) * np.uint64(0x100000001B3)
    return (_splitmix(ctr) % np.uint64(hi)).astype(np.int32).reshape(shape)


def bf16_exact(x: np.ndarray) -> np.ndarray:
    """x with the low 16 bits of every value cleared: a value bf16 holds exactly."""
    return (np.ascontiguousarray(x, np.float32).view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    return (bf16_exact(x).view(np.uint32) >> np.uint32(16)).astype(np.uint16)


# ------------------------------------------------------------------ backend operations

RMS = [(5, 48, 1e-6), (3, 2048, 1e-6), (64, 128, 1e-5)]
LIN = [(7, 96, 40), (1, 2048, 300), (13, 256, 64)]
ROPE = [(4, 3, 128, 1e6), (6, 2, 8, 1e4), (3, 16, 64, 5e5)]
SILU_N = 1000
SOFTMAX_N = [7, 1000, 20000]
ATT = [(5, 4, 2, 64, 37, True), (1, 16, 8, 128, 129, False), (6, 4, 1, 128, 300, True)]


def ops_inputs() -> dict[str, np.ndarray]:
    """Inputs of every backend-operation case, keyed like the fixture's outputs."""
    a: dict[str, np.ndarray] = {}
    s = 100
    for c, (rows, d, eps) in enumerate(RMS):
        a[f"rms{c}.x"] = det_uniform(s + c, (rows, d), 5.0)
        a[f"rms{c}.w"] = bf16_exact(1.0 + det_uniform(s + 10 + c, (d,), 0.2))
        a[f"rms{c}.eps"] = np.float32(eps)
    s = 200
    for c, (L, i, o) in enumerate(LIN):
        a[f"lin{c}.x"] = det_uniform(s + c, (L, i), 1.5)
        a[f"lin{c}.W"] = bf16_exact(det_uniform(s + 10 + c, (o, i), 0.08))
        a[f"lin{c}.y0"] = det_uniform(s + 20 + c, (L, o), 1.0)
    s = 300
    for c, (L, heads, D, base) in enumerate(ROPE):
        a[f"rope{c}.x"] = det_uniform(s + c, (L, heads, D), 2.0)
        pos = np.sort(det_ints(s + 10 + c, (L,), 70000))
        pos[0] = 0
        a[f"rope{c}.pos"] = pos.astype(np.int32)
        a[f"rope{c}.base"] = np.float32(base)
    a["silu.gate"] = det_uniform(400, (SILU_N,), 8.0)
    a["silu.up"] = det_uniform(401, (SILU_N,), 2.0)
    s = 500
    for c, n in enumerate(SOFTMAX_N):
        x = det_uniform(s + c, (n,), 6.0)
        if n > 7:
            x[det_ints(s + 10 + c, (n // 10,), n)] = -np.inf
        a[f"sm{c}.x"] = x
    s = 600
    for c, (L, H, Hk, D, T, masked) in enumerate(ATT):
        a[f"att{c}.q"] = det_uniform(s + c, (L, H, D), 1.5)
        a[f"att{c}.K"] = det_uniform(s + 10 + c, (T, Hk, D), 1.5)
        a[f"att{c}.V"] = det_uniform(s + 20 + c, (T, Hk, D), 1.0)
        if masked:
            m = (det_ints(s + 30 + c, (L, T), 10) < 7).astype(np.uint8)
            m[:, 0] = 1
            a[f"att{c}.mask"] = m
        a[f"att{c}.scale"] = np.float32(1.0 / np.sqrt(np.float32(D)))
    return a


# ------------------------------------------------------------------ small Qwen3 target

QWEN3 = dict(hidden_size=256, num_heads=2, num_kv_heads=1, head_dim=128, intermediate_size=256, num_layers=2,
             vocab_size=300, rope_theta=1e6)
QWEN3_TAPS = (0, 1, 1)
QWEN3_LAYER = {
    "input_layernorm.weight": lambda c: (c["hidden_size"],),
    "post_attention_layernorm.weight": lambda c: (c["hidden_size"],),
    "self_attn.q_proj.weight": lambda c: (c["num_heads"] * c["head_dim"], c["hidden_size"]),
    "self_attn.k_proj.weight": lambda c: (c["num_kv_heads"] * c["head_dim"], c["hidden_size"]),
    "self_attn.v_proj.weight": lambda c: (c["num_kv_heads"] * c["head_dim"], c["hidden_size"]),
    "self_attn.o_proj.weight": lambda c: (c["hidden_size"], c["num_heads"] * c["head_dim"]),
    "self_attn.q_norm.weight": lambda c: (c["head_dim"],),
    "self_attn.k_norm.weight": lambda c: (c["head_dim"],),
    "mlp.gate_proj.weight": lambda c: (c["intermediate_size"], c["hidden_size"]),
    "mlp.up_proj.weight": lambda c: (c["intermediate_size"], c["hidden_size"]),
    "mlp.down_proj.weight": lambda c: (c["hidden_size"], c["intermediate_size"]),
}


def qwen3_weights() -> dict[str, np.ndarray]:
    """bf16 bit patterns of the small target, our names (layers.{i}.*, embed_tokens, norm)."""
    c = QWEN3
    w: dict[str, np.ndarray] = {}
    seed = 700
    for i in range(c["num_layers"]):
        for n, shape in QWEN3_LAYER.items():
            sh = shape(c)
            seed += 1
            x = 1.0 + det_uniform(seed, sh, 0.17) if len(sh) == 1 else det_uniform(seed, sh, 0.087)
            w[f"layers.{i}.{n}"] = bf16_bits(x)
    w["embed_tokens.weight"] = bf16_bits(det_uniform(790, (c["vocab_size"], c["hidden_size"]), 0.87))
    w["norm.weight"] = bf16_bits(1.0 + det_uniform(791, (c["hidden_size"],), 0.17))
    return w


def qwen3_inputs() -> dict[str, np.ndarray]:
    """A causal prefill of 9 tokens, then a 6-node tree block at positions 9 + depth."""
    parents = np.array([-1, 0, 0, 1, 1, 3], np.int32)
    depth = np.array([0, 1, 1, 2, 2, 3], np.int32)
    return {"prefill.tokens": det_ints(800, (9,), QWEN3["vocab_size"]),
            "tree.tokens": det_ints(801, (6,), QWEN3["vocab_size"]),
            "tree.parents": parents, "tree.depth": depth, "tree.positions": (9 + depth).astype(np.int32)}
