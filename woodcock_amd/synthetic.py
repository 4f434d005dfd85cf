"""Seeded synthetic drafter weights and inputs (random init; no checkpoints offline).

Weights are N(0, std) in bf16; RMSNorm gains are 1 + N(0, gain_std) so a kernel
that ignored a gain would be caught.  Names are the reference's parameter names
(python/woodcock/drafter.py:66-142), so the same dict can be written as a
reference-format drafter directory.
"""
from __future__ import annotations

import numpy as np
import torch

from .config import DrafterConfig


def weight_shapes(cfg: DrafterConfig, head_rows: int | None = None) -> dict[str, tuple[int, ...]]:
    d, H, Hk, D = cfg.hidden_size, cfg.num_heads, cfg.num_kv_heads, cfg.head_dim
    F, Dt, nf = cfg.intermediate_size, cfg.target_hidden_size, cfg.num_features
    s: dict[str, tuple[int, ...]] = {
        "embed_tokens.weight": (cfg.vocab_size, d),
        "fc.weight": (d, nf * Dt),
        "norm.weight": (d,),
        "lm_head.weight": (head_rows or cfg.vocab_size, d),
    }
    if cfg.feature_norm:
        for i in range(nf):
            s[f"feature_norms.{i}.weight"] = (Dt,)
    for i in range(cfg.num_layers):
        p = f"layers.{i}."
        s[p + "input_layernorm.weight"] = (d,)
        s[p + "post_attention_layernorm.weight"] = (d,)
        s[p + "self_attn.q_proj.weight"] = (H * D, d)
        s[p + "self_attn.k_proj.weight"] = (Hk * D, d)
        s[p + "self_attn.v_proj.weight"] = (Hk * D, d)
        s[p + "self_attn.o_proj.weight"] = (d, H * D)
        s[p + "self_attn.q_norm.weight"] = (D,)
        s[p + "self_attn.k_norm.weight"] = (D,)
        s[p + "mlp.gate_proj.weight"] = (F, d)
        s[p + "mlp.up_proj.weight"] = (F, d)
        s[p + "mlp.down_proj.weight"] = (d, F)
        if i == 0:
            s[p + "aux_norm.weight"] = (d,)
            s[p + "self_attn.aux_q.weight"] = (H * D, d)
            s[p + "self_attn.aux_k.weight"] = (Hk * D, d)
            s[p + "self_attn.aux_v.weight"] = (Hk * D, d)
    return s


def random_drafter(cfg: DrafterConfig, seed: int = 0, device="cpu", std: float = 0.02, gain_std: float = 0.1,
                   head_rows: int | None = None) -> dict[str, torch.Tensor]:
    """bf16 tensors on `device`, deterministic for a given (seed, device type)."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    out = {}
    for name, shape in weight_shapes(cfg, head_rows).items():
        t = torch.randn(shape, generator=g, device=device, dtype=torch.float32)
        if len(shape) == 1:
            t = 1.0 + gain_std * t
        else:
            t = std * t
        out[name] = t.to(torch.bfloat16)
    return out


def to_bits(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor -> numpy uint16 bit patterns (host copy)."""
    return t.detach().to("cpu").contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits(a: np.ndarray, device="cpu") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint16).view(np.int16)).view(torch.bfloat16).to(device)


def draft_vocab(vocab: int, k: int, seed: int = 0, always=()) -> np.ndarray:
    """A seeded K-row draft vocabulary: random counts through top_ids semantics
    (python/woodcock/vocab.py:35-47) -- ascending ids, `always` forced in."""
    from .vocab import top_ids

    rng = np.random.default_rng(seed)
    counts = rng.zipf(1.2, size=vocab).astype(np.int64)
    return top_ids(counts, k, set(int(a) for a in always if a < vocab))
