"""Verify-width target forward, one decoder layer at a time (python/woodcock/target.py).

``TargetLayer`` holds one Qwen3 decoder layer's device weights (the reference's
parameter names, python/woodcock/target.py:142-156 / mlx-lm Qwen3) and runs
``wc_target_layer`` over a verify block of up to 64 rows: the tree or chain
block at explicit positions with an explicit mask (target.py:82-116).  The
embedding, the final norm and the LM head of the target are the caller's.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from .cache import KVCache
from .runtime import device_of, ptr, stream_ptr

MAX_ROWS = 64

LAYER_NAMES = {
    "in_norm": "input_layernorm.weight",
    "post_norm": "post_attention_layernorm.weight",
    "q": "self_attn.q_proj.weight",
    "k": "self_attn.k_proj.weight",
    "v": "self_attn.v_proj.weight",
    "o": "self_attn.o_proj.weight",
    "q_norm": "self_attn.q_norm.weight",
    "k_norm": "self_attn.k_norm.weight",
    "gate": "mlp.gate_proj.weight",
    "up": "mlp.up_proj.weight",
    "down": "mlp.down_proj.weight",
}


@dataclass(frozen=True)
class TargetConfig:
    """The Qwen3 shape fields a decoder layer needs (Qwen3-1.7B by default)."""

    hidden_size: int = 2048
    num_heads: int = 16
    num_kv_heads: int = 8
    head_dim: int = 128
    intermediate_size: int = 6144
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6
    num_layers: int = 28


def layer_shapes(cfg: TargetConfig) -> dict[str, tuple[int, ...]]:
    d, H, Hk, D, F = cfg.hidden_size, cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.intermediate_size
    return {
        "input_layernorm.weight": (d,), "post_attention_layernorm.weight": (d,),
        "self_attn.q_proj.weight": (H * D, d), "self_attn.k_proj.weight": (Hk * D, d),
        "self_attn.v_proj.weight": (Hk * D, d), "self_attn.o_proj.weight": (d, H * D),
        "self_attn.q_norm.weight": (D,), "self_attn.k_norm.weight": (D,),
        "mlp.gate_proj.weight": (F, d), "mlp.up_proj.weight": (F, d), "mlp.down_proj.weight": (d, F),
    }


def random_layer(cfg: TargetConfig, seed: int = 0, device="cuda", std: float = 0.02, gain_std: float = 0.1):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    out = {}
    for name, shape in layer_shapes(cfg).items():
        t = torch.randn(shape, generator=g, device=device)
        out[name] = (1.0 + gain_std * t if len(shape) == 1 else std * t).to(torch.bfloat16)
    return out


class TargetLayer:
    def __init__(self, cfg: TargetConfig, weights: dict[str, torch.Tensor], device="cuda", max_rows: int = MAX_ROWS):
        self.cfg = cfg
        self.device = torch.device(device)
        shapes = layer_shapes(cfg)
        self.w = {}
        for name, shape in shapes.items():
            t = weights[name]
            if tuple(t.shape) != shape:
                raise ValueError(f"{name}: shape {tuple(t.shape)}, expected {shape}")
            self.w[name] = t.to(self.device, torch.bfloat16).contiguous()
        self.lw = _lib.LayerWeights()
        for f, name in LAYER_NAMES.items():
            setattr(self.lw, f, ptr(self.w[name]))
        self.dims = _lib.DrafterDims(cfg.hidden_size, 1, cfg.num_heads, cfg.num_kv_heads, cfg.head_dim,
                                     cfg.intermediate_size, cfg.hidden_size, 3, 1, 1, cfg.rms_norm_eps, 0)
        self.max_rows = max_rows
        n = _lib.lib().wc_target_workspace_bytes(C.byref(self.dims), max_rows)
        self.ws = torch.zeros(n, dtype=torch.uint8, device=self.device)  # split-K counters start at zero
        self._rope: tuple[torch.Tensor, torch.Tensor] | None = None

    def rope(self, positions: int) -> tuple[torch.Tensor, torch.Tensor]:
        if self._rope is None or self._rope[0].shape[0] < positions:
            n = max(positions, 64)
            half = self.cfg.head_dim // 2
            cos = np.empty((n, half), np.float32)
            sin = np.empty_like(cos)
            _lib.call("wc_rope_table", cos.ctypes.data_as(C.c_void_p), sin.ctypes.data_as(C.c_void_p), n,
                      self.cfg.head_dim, float(self.cfg.rope_theta))
            self._rope = (torch.from_numpy(cos).to(self.device), torch.from_numpy(sin).to(self.device))
        return self._rope

    def __call__(self, x: torch.Tensor, cache: KVCache, offset_dev: torch.Tensor,
                 positions: torch.Tensor | None = None, mask: torch.Tensor | None = None) -> torch.Tensor:
        """x [rows, hidden] fp32, updated in place and returned; the block's K/V
        land at cache slots *offset_dev .. + rows (the caller advances the offset)."""
        device_of(x)
        rows = x.shape[0]
        if x.dtype != torch.float32 or x.dim() != 2 or x.shape[1] != self.cfg.hidden_size or not x.is_contiguous():
            raise ValueError("x must be a contiguous float32 [rows, hidden] tensor")
        if not 1 <= rows <= self.max_rows:
            raise ValueError(f"rows must be in 1..{self.max_rows}")
        cos, sin = self.rope(cache.capacity + 64)
        pos = None if positions is None else positions.to(self.device, torch.int32).contiguous()
        if mask is not None:
            mask = mask.to(self.device, torch.uint8).contiguous()
            if mask.shape[0] != rows:
                raise ValueError("mask must have one row per input row")
        _lib.call("wc_target_layer", C.byref(self.dims), C.byref(self.lw), ptr(cos), ptr(sin), cos.shape[0], ptr(x),
                  rows, ptr(pos) if pos is not None else None, ptr(mask) if mask is not None else None,
                  mask.stride(0) if mask is not None else 0, ptr(cache.keys), ptr(cache.values),
                  _lib.WC_BF16 if cache.keys.dtype == torch.bfloat16 else _lib.WC_F32, cache.capacity,
                  ptr(offset_dev), ptr(self.ws), stream_ptr())
        return x
