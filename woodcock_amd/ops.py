"""The reference runtime's backend operations on the GPU
(include/woodcock/ops.h:9-24; src/backends/cpu_ops.cpp:45-115).

Each function enqueues one wc_* entry point of libwoodcock_hip.so on the
current stream over device tensors -- fp32 activations, bf16 or fp32 weights --
with the reference's argument meaning and layouts: activations [rows][cols],
attention K / V as KVCache rows [T][Hk][D] (include/woodcock/cache.h:9-28).
These are single operations for a backend under the reference's C++ runtime;
the drafter / target / verify entry points are the fused hot path.
"""
from __future__ import annotations

import torch

from . import _lib
from .runtime import device_of, ptr, stream_ptr


def _f32(t: torch.Tensor, name: str) -> torch.Tensor:
    device_of(t)
    if t.dtype != torch.float32 or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous float32 device tensor")
    return t


def _weight(w: torch.Tensor, name: str):
    device_of(w)
    if w.dtype not in (torch.float32, torch.bfloat16) or not w.is_contiguous():
        raise ValueError(f"{name} must be a contiguous float32 or bfloat16 device tensor")
    return _lib.WC_BF16 if w.dtype == torch.bfloat16 else _lib.WC_F32


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float, out: torch.Tensor | None = None) -> torch.Tensor:
    """Row-wise x * rsqrt(mean(x^2) + eps) * w over the last axis (ops.h:13); out may be x."""
    _f32(x, "x")
    d = x.shape[-1]
    if w.numel() != d:
        raise ValueError(f"weight has {w.numel()} entries for rows of {d}")
    out = torch.empty_like(x) if out is None else _f32(out, "out")
    _lib.call("wc_rmsnorm", ptr(x), ptr(out), x.numel() // d, d, ptr(w), _weight(w, "w"), float(eps), stream_ptr())
    return out


def linear(x: torch.Tensor, W: torch.Tensor, y: torch.Tensor | None = None, accumulate: bool = False) -> torch.Tensor:
    """y[L][out] (+)= x[L][in] . W[out][in]^T (ops.h:11)."""
    _f32(x, "x")
    out_f, in_f = W.shape
    if x.shape[-1] != in_f:
        raise ValueError(f"x rows of {x.shape[-1]} against a [{out_f}, {in_f}] weight")
    L = x.numel() // in_f
    if y is None:
        if accumulate:
            raise ValueError("accumulate needs y")
        y = torch.empty(*x.shape[:-1], out_f, dtype=torch.float32, device=x.device)
    else:
        _f32(y, "y")
        if y.numel() != L * out_f:
            raise ValueError("y has the wrong size")
    _lib.call("wc_linear", ptr(x), L, in_f, ptr(W), _weight(W, "W"), out_f, ptr(y), int(accumulate), stream_ptr())
    return y


def rope(x: torch.Tensor, positions: torch.Tensor, base: float, table: tuple[torch.Tensor, torch.Tensor] | None = None
         ) -> torch.Tensor:
    """Rotate-half RoPE in place on x [L, heads, D] at positions [L] (ops.h:15).
    table: the (cos, sin) [max_pos, D/2] of wc_rope_table, for cos / sin equal
    to the host recipe's bit for bit."""
    _f32(x, "x")
    if x.dim() != 3:
        raise ValueError("x must be [L, heads, head_dim]")
    L, heads, D = x.shape
    pos = positions.to(x.device, torch.int32).contiguous()
    if pos.numel() != L:
        raise ValueError("one position per row")
    cos = sin = None
    max_pos = 0
    if table is not None:
        cos, sin = (_f32(t, "table") for t in table)
        if cos.shape != sin.shape or cos.shape[-1] != D // 2:
            raise ValueError("rope tables must be [max_pos, head_dim / 2]")
        max_pos = cos.shape[0]
    _lib.call("wc_rope", ptr(x), L, heads, D, ptr(pos), float(base), ptr(cos), ptr(sin), max_pos, stream_ptr())
    return x


def silu_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """gate = silu(gate) * up, in place (ops.h:17)."""
    _f32(gate, "gate")
    _f32(up, "up")
    if gate.numel() != up.numel():
        raise ValueError("gate and up differ in size")
    _lib.call("wc_silu_mul", ptr(gate), ptr(up), gate.numel(), stream_ptr())
    return gate


def attention(q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, mask: torch.Tensor | None, scale: float
              ) -> torch.Tensor:
    """q [L, H, D]; K, V [T, Hk, D]; mask [L, T] (None = all visible) -> out [L, H, D] (ops.h:19-21)."""
    _f32(q, "q")
    _f32(K, "K")
    _f32(V, "V")
    L, H, D = q.shape
    T, Hk, Dk = K.shape
    if V.shape != K.shape or Dk != D:
        raise ValueError("K / V must be [T, Hk, head_dim] like q's head_dim")
    m = None
    if mask is not None:
        m = mask.to(q.device, torch.uint8).contiguous()
        if m.shape != (L, T):
            raise ValueError(f"mask must be [{L}, {T}]")
    out = torch.empty_like(q)
    _lib.call("wc_attention", ptr(q), L, H, Hk, D, ptr(K), ptr(V), T, ptr(m), ptr(out), float(scale), stream_ptr())
    return out


def softmax(x: torch.Tensor) -> torch.Tensor:
    """In-place softmax over the last axis of every row (ops.h:22)."""
    _f32(x, "x")
    n = x.shape[-1]
    _lib.call("wc_softmax", ptr(x), x.numel() // n, n, stream_ptr())
    return x
