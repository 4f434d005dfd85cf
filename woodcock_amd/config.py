"""Drafter hyper-parameters (python/woodcock/drafter.py:33-63; src/core/drafter.cpp:18-45).

Same field names, defaults and JSON format as the reference so an exported
drafter ``config.json`` loads unchanged; configs written by the reference's
earlier code base are accepted only when their legacy fields hold the values
this drafter can represent (drafter.py:57-63).
"""
from __future__ import annotations

import json
from dataclasses import asdict, dataclass, field
from pathlib import Path


@dataclass
class DrafterConfig:
    hidden_size: int
    num_layers: int
    num_heads: int
    num_kv_heads: int
    head_dim: int
    intermediate_size: int
    vocab_size: int
    target_hidden_size: int
    num_features: int = 3
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1_000_000.0
    post_norm: bool = True
    feature_norm: bool = True
    window: int | None = None
    feature_layers: list[int] = field(default_factory=list)

    def save(self, path) -> None:
        Path(path).write_text(json.dumps(asdict(self), indent=2))

    @classmethod
    def from_dict(cls, d: dict, where: str = "config") -> "DrafterConfig":
        d = dict(d)
        if d.pop("residual", "feature") != "feature" or d.pop("lowrank_rank", 0):
            raise ValueError(f"{where}: unsupported drafter configuration")
        d.pop("lowrank_k", None)
        return cls(**d)

    @classmethod
    def load(cls, path) -> "DrafterConfig":
        return cls.from_dict(json.loads(Path(path).read_text()), str(path))

    def as_dict(self) -> dict:
        return asdict(self)


def qwen3_1p7b_drafter() -> DrafterConfig:
    """One decoder layer at Qwen3-1.7B width (config_for_target, drafter.py:341-358)."""
    return DrafterConfig(hidden_size=2048, num_layers=1, num_heads=16, num_kv_heads=8, head_dim=128,
                         intermediate_size=6144, vocab_size=151936, target_hidden_size=2048,
                         rms_norm_eps=1e-6, rope_theta=1_000_000.0, feature_layers=[2, 14, 25])


def qwen3_4b_drafter() -> DrafterConfig:
    """One decoder layer at Qwen3-4B width."""
    return DrafterConfig(hidden_size=2560, num_layers=1, num_heads=32, num_kv_heads=8, head_dim=128,
                         intermediate_size=9728, vocab_size=151936, target_hidden_size=2560,
                         rms_norm_eps=1e-6, rope_theta=1_000_000.0, feature_layers=[2, 18, 33])


def tiny_drafter(**kw) -> DrafterConfig:
    """The reference's test configuration (tests/test_drafter.py:8-21)."""
    base = dict(hidden_size=32, num_layers=1, num_heads=4, num_kv_heads=2, head_dim=8, intermediate_size=48,
                vocab_size=50, target_hidden_size=24, rope_theta=10000.0)
    base.update(kw)
    return DrafterConfig(**base)


# Qwen3 end-of-sequence ids that every draft vocabulary keeps (docs/design-vocab-trim.md:71-78)
QWEN3_EOS = (151643, 151645)
