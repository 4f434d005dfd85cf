"""Speculative verification rules on the GPU (python/woodcock/sampling.py API).

Greedy rules run as one fused kernel (target argmax + acceptance) that writes a
device-side ``wc_verdict``; the host-facing functions read it back (one copy)
and return the reference's ``(n, next)`` / ``(path, next)`` tuples.  The
``*_dev`` variants leave the verdict on the device for a fused round.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

from . import _lib
from .runtime import device_of, i32, new_verdict, ptr, read_verdict, stream_ptr, workspace


@dataclass(frozen=True)
class SamplingParams:
    """python/woodcock/sampling.py:27-36."""

    temperature: float = 0.0  # 0 => greedy
    top_k: int = 0
    top_p: float = 1.0
    seed: int = 0

    @property
    def greedy(self) -> bool:
        return self.temperature <= 0.0


@dataclass
class DraftTree:
    """Flattened draft tree, node 0 the root; children[v] in draw (= node index)
    order (python/woodcock/sampling.py:87-115)."""

    tokens: list[int]
    parents: list[int]
    depth: list[int]
    children: list[list[int]] = field(default_factory=list)

    def __post_init__(self):
        if not self.children:
            self.children = [[] for _ in self.tokens]
            for v, par in enumerate(self.parents):
                if par >= 0:
                    self.children[par].append(v)

    def __len__(self):
        return len(self.tokens)

    def path_to(self, v: int) -> list[int]:
        out = []
        while v > 0:
            out.append(v)
            v = self.parents[v]
        return out[::-1]

    def is_chain(self) -> bool:
        return all(p == i - 1 for i, p in enumerate(self.parents))


def tree_attention_mask(tree: DraftTree, prefix_len: int) -> np.ndarray:
    """(N, prefix+N) bool: every node sees the prefix and its ancestors, itself
    included (python/woodcock/sampling.py:118-128)."""
    N = len(tree)
    m = np.zeros((N, prefix_len + N), dtype=bool)
    m[:, :prefix_len] = True
    anc = np.zeros((N, N), dtype=bool)
    for v in range(N):
        p = tree.parents[v]
        if p >= 0:
            anc[v] = anc[p]
        anc[v, v] = True
    m[:, prefix_len:] = anc
    return m


def _logits_2d(target_logits: torch.Tensor) -> torch.Tensor:
    if target_logits.dim() == 3:
        if target_logits.shape[0] != 1:
            raise ValueError("batch size 1 only")
        target_logits = target_logits[0]
    if target_logits.dim() != 2 or target_logits.dtype != torch.float32:
        raise ValueError("target logits must be a float32 (rows, vocab) tensor")
    device_of(target_logits)
    if target_logits.stride(1) != 1:
        target_logits = target_logits.contiguous()
    return target_logits


def argmax_rows(logits: torch.Tensor) -> torch.Tensor:
    """Row-wise argmax (lowest index wins a tie), int32 on the device."""
    lg = _logits_2d(logits)
    out = torch.empty(lg.shape[0], dtype=torch.int32, device=lg.device)
    _lib.call("wc_argmax_rows", ptr(lg), lg.shape[0], lg.shape[1], lg.stride(0), ptr(out),
              ptr(workspace(lg.device)), stream_ptr())
    return out


def verify_chain_greedy_dev(target_logits: torch.Tensor, draft_tokens: torch.Tensor,
                            verdict: torch.Tensor | None = None) -> torch.Tensor:
    """Enqueue the fused argmax + chain acceptance; returns the device verdict."""
    lg = _logits_2d(target_logits)
    rows = lg.shape[0]
    if draft_tokens.numel() != rows - 1:
        raise ValueError(f"{rows} logit rows need {rows - 1} draft tokens, got {draft_tokens.numel()}")
    verdict = new_verdict(lg.device) if verdict is None else verdict
    _lib.call("wc_verify_chain_greedy", ptr(lg), rows, lg.shape[1], lg.stride(0), ptr(draft_tokens), ptr(verdict),
              ptr(workspace(lg.device)), stream_ptr())
    return verdict


def verify_chain_greedy(target_logits: torch.Tensor, draft_tokens) -> tuple[int, int]:
    """target_logits (K+1, V) at [x_n, d_1..d_K] -> (n_accepted, next_token)
    (python/woodcock/sampling.py:60-66)."""
    lg = _logits_2d(target_logits)
    d = draft_tokens if isinstance(draft_tokens, torch.Tensor) else i32(list(draft_tokens), lg.device)
    v = read_verdict(verify_chain_greedy_dev(lg, d.to(lg.device, torch.int32)))
    return int(v.n_accepted), int(v.next)


def verify_tree_greedy_dev(target_logits: torch.Tensor, tree_tokens: torch.Tensor, tree_parents: torch.Tensor,
                           verdict: torch.Tensor | None = None) -> torch.Tensor:
    lg = _logits_2d(target_logits)
    N = lg.shape[0]
    if tree_tokens.numel() != N or tree_parents.numel() != N:
        raise ValueError("tree tokens / parents must have one entry per logit row")
    verdict = new_verdict(lg.device) if verdict is None else verdict
    _lib.call("wc_verify_tree_greedy", ptr(lg), N, lg.shape[1], lg.stride(0), ptr(tree_tokens), ptr(tree_parents),
              ptr(verdict), ptr(workspace(lg.device)), stream_ptr())
    return verdict


def verify_tree_greedy(target_logits: torch.Tensor, tree: DraftTree) -> tuple[list[int], int]:
    """Target logits at every tree node (N, V) -> (accepted node path, next token).
    Same walk as python/woodcock/sampling.py:131-140, with the target argmax fused."""
    lg = _logits_2d(target_logits)
    if len(tree) > _lib.WC_MAX_NODES:
        raise ValueError(f"at most {_lib.WC_MAX_NODES} tree nodes per round")
    v = read_verdict(verify_tree_greedy_dev(lg, i32(tree.tokens, lg.device), i32(tree.parents, lg.device)))
    return [int(v.keep[1 + i]) for i in range(v.n_accepted)], int(v.next)
