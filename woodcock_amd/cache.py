"""Device KV caches and their in-place compaction.

``KVCache`` mirrors the mlx-lm cache object the reference drives
(python/woodcock/drafter.py:186-187,231-232; python/woodcock/target.py:152,159-175):
``keys`` / ``values`` are [1, kv_heads, capacity, head_dim] device tensors, and
``offset`` counts the valid entries (settable: a rollback just rewinds it,
python/woodcock/spec.py:275-276,351-352).  Capacity is allocated up front (HBM
is plentiful), so appends never reallocate.

``compact_cache`` keeps only entries ``start + keep[i]`` of the last block,
contiguously, for every layer in ONE kernel launch (wc_kv_compact).
"""
from __future__ import annotations

import ctypes as C

import torch

from . import _lib
from .runtime import device_of, ptr, stream_ptr


class KVCache:
    def __init__(self, kv_heads: int, head_dim: int, capacity: int, dtype=torch.bfloat16, device="cuda"):
        if dtype not in (torch.bfloat16, torch.float32):
            raise ValueError("KV cache dtype must be bfloat16 or float32")
        self.keys = torch.zeros(1, kv_heads, capacity, head_dim, dtype=dtype, device=device)
        self.values = torch.zeros_like(self.keys)
        self.offset = 0

    @property
    def capacity(self) -> int:
        return self.keys.shape[2]

    @property
    def kv_heads(self) -> int:
        return self.keys.shape[1]

    @property
    def head_dim(self) -> int:
        return self.keys.shape[3]

    @property
    def row_bytes(self) -> int:
        return self.head_dim * self.keys.element_size()


def make_cache(layers: int, kv_heads: int, head_dim: int, capacity: int, dtype=torch.bfloat16,
               device="cuda") -> list[KVCache]:
    return [KVCache(kv_heads, head_dim, capacity, dtype, device) for _ in range(layers)]


def _layer_ptrs(cache: list[KVCache]):
    if not cache:
        raise ValueError("empty cache list")
    if len(cache) > _lib.WC_MAX_LAYERS:
        raise ValueError(f"at most {_lib.WC_MAX_LAYERS} layers per compaction")
    c0 = cache[0]
    device_of(c0.keys)
    for c in cache:
        if c.keys.shape != c0.keys.shape or c.keys.dtype != c0.keys.dtype or c.values.shape != c0.keys.shape:
            raise ValueError("all layers of a compaction must share shape and dtype")
        if not (c.keys.is_contiguous() and c.values.is_contiguous()):
            raise ValueError("KV tensors must be contiguous")
    kp = (C.c_void_p * len(cache))(*[c.keys.data_ptr() for c in cache])
    vp = (C.c_void_p * len(cache))(*[c.values.data_ptr() for c in cache])
    return kp, vp


def compact_cache_dev(cache: list[KVCache], start_dev: torch.Tensor, keep_dev: torch.Tensor,
                      n_keep_dev: torch.Tensor, max_keep: int, offset_dev: torch.Tensor | None = None,
                      status_dev: torch.Tensor | None = None) -> None:
    """Enqueue the compaction with start / keep / n_keep read from device memory
    (e.g. views into a wc_verdict).  Host offsets are NOT updated."""
    kp, vp = _layer_ptrs(cache)
    c0 = cache[0]
    _lib.call("wc_kv_compact", kp, vp, len(cache), c0.kv_heads, c0.capacity, c0.row_bytes, ptr(start_dev),
              ptr(keep_dev), ptr(n_keep_dev), int(max_keep), ptr(offset_dev), ptr(status_dev), stream_ptr())


def compact_cache(cache: list[KVCache], start: int, keep: list[int]) -> None:
    """Keep only entries start + keep[i] of the last block, contiguously, then
    rewind every offset to start + len(keep) (python/woodcock/target.py:159-175)."""
    keep = [int(k) for k in keep]
    n = len(keep)
    if n > _lib.WC_MAX_NODES + 1:
        raise ValueError(f"at most {_lib.WC_MAX_NODES + 1} kept entries")
    if any(k < i for i, k in enumerate(keep)) or any(b <= a for a, b in zip(keep, keep[1:])):
        raise ValueError("keep must be strictly increasing")
    if n and start + keep[-1] >= cache[0].capacity:
        raise ValueError("keep index beyond the cache capacity")
    if start < 0:
        raise ValueError("start must be non-negative")
    if keep != list(range(n)):
        dev = cache[0].keys.device
        args = torch.tensor([start, n] + keep, dtype=torch.int32).to(dev)
        compact_cache_dev(cache, args[0:1], args[2:], args[1:2], max(n, 1))
    for c in cache:
        c.offset = start + n
