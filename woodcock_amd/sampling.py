"""Speculative verification rules on the GPU (python/woodcock/sampling.py API).

Greedy rules run as one fused kernel (target argmax + acceptance) that writes a
device-side ``wc_verdict``; the stochastic chain rule runs as two launches over
device probabilities.  The host-facing functions read the verdict back (one
copy) and return the reference's ``(n, next)`` / ``(path, next)`` tuples.  The
``*_dev`` variants leave the verdict on the device for a fused round.

Randomness: where the reference threads a numpy Generator through the rules,
these take a ``PhiloxStream`` -- (seed, round, purpose) of the counter-based
stream the kernels read; uniform j of a round is consumed in the reference's
order (sampling.py:79,165,193).
"""
from __future__ import annotations

import ctypes as C
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
    if target_logits.stride(1) != 1 or (target_logits.shape[0] == 1 and target_logits.stride(0) < target_logits.shape[1]):
        # (one row may carry any stride of its size-1 dimension; the kernels read rows at the stride)
        target_logits = target_logits.clone(memory_format=torch.contiguous_format)
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


# ------------------------------------------------------------------ stochastic rules

@dataclass
class PhiloxStream:
    """Uniform source of the stochastic kernels: round ``round`` of Philox4x64-10
    under ``seed``, sub-stream ``purpose``.  ``round_dev`` (int32 [1] on the
    device) is what the kernels read, so a captured graph advances by updating it."""

    seed: int
    round: int = 0
    purpose: int = 0
    round_dev: torch.Tensor | None = None

    def device_round(self, device) -> torch.Tensor:
        if self.round_dev is None or self.round_dev.device != device:
            self.round_dev = i32([self.round], device)
        else:
            self.round_dev.fill_(self.round)
        return self.round_dev

    def struct(self, round_dev: torch.Tensor) -> _lib.Uniforms:
        return _lib.Uniforms(self.seed, ptr(round_dev), self.purpose)


def probs_from_logits(logits: torch.Tensor, sp: SamplingParams | float, out: torch.Tensor | None = None
                      ) -> torch.Tensor:
    """Warped float32 distribution over the last axis (python/woodcock/sampling.py:39-55):
    softmax(logits / max(T, 1e-6)) after top-k (SamplingParams.top_k > 0: logits
    below the k-th largest drop out), then top-p (top_p < 1: the smallest
    descending-order prefix whose mass reaches top_p, renormalised)."""
    if isinstance(sp, (int, float)):
        t, top_k, top_p = float(sp), 0, 1.0
    else:
        t, top_k, top_p = float(sp.temperature), int(sp.top_k or 0), float(sp.top_p)
    lg = _logits_2d(logits)
    out = torch.empty_like(lg) if out is None else out
    if out.shape != lg.shape or out.dtype != torch.float32 or out.stride(1) != 1:
        raise ValueError("out must be a float32 tensor shaped like logits")
    _lib.call("wc_probs_from_logits", ptr(lg), lg.shape[0], lg.shape[1], lg.stride(0), t, top_k, top_p, ptr(out),
              out.stride(0), ptr(workspace(lg.device)), stream_ptr())
    return out


def verify_chain_stochastic_dev(p: torch.Tensor, q: torch.Tensor, draft_tokens: torch.Tensor,
                                rng: _lib.Uniforms, d2t: torch.Tensor | None = None,
                                draft_rows: torch.Tensor | None = None,
                                verdict: torch.Tensor | None = None) -> torch.Tensor:
    """Enqueue the stochastic chain rule; p (K+1, V) target probabilities, q (K, H)
    draft probabilities over the H head rows (d2t maps row -> token; None = identity)."""
    p2 = _logits_2d(p)
    rows, vocab = p2.shape
    K = rows - 1
    if draft_tokens.numel() != K:
        raise ValueError(f"{rows} probability rows need {K} draft tokens, got {draft_tokens.numel()}")
    if K > 0:
        q2 = _logits_2d(q)
        if q2.shape[0] < K:
            raise ValueError(f"q has {q2.shape[0]} rows, {K} needed")
        head_rows, ldq, qp = q2.shape[1], q2.stride(0), ptr(q2)
    else:
        head_rows, ldq, qp = 1, 1, None
    if d2t is not None and d2t.numel() != head_rows:
        raise ValueError(f"d2t has {d2t.numel()} entries for {head_rows} draft rows")
    verdict = new_verdict(p2.device) if verdict is None else verdict
    _lib.call("wc_verify_chain_stochastic", ptr(p2), rows, vocab, p2.stride(0), qp, head_rows, ldq,
              ptr(d2t) if d2t is not None else None, ptr(draft_tokens) if K > 0 else None,
              ptr(draft_rows) if draft_rows is not None else None, C.byref(rng), ptr(verdict),
              ptr(workspace(p2.device)), stream_ptr())
    return verdict


def verify_chain_stochastic_logits_dev(logits: torch.Tensor, temperature: float, q: torch.Tensor,
                                       draft_tokens: torch.Tensor, rng: _lib.Uniforms,
                                       d2t: torch.Tensor | None = None, draft_rows: torch.Tensor | None = None,
                                       verdict: torch.Tensor | None = None) -> torch.Tensor:
    """The stochastic chain rule straight from the target logits (K+1, V):
    p = softmax(logits / T) is formed inside the launch and never written
    (spec.py:316-324); otherwise as verify_chain_stochastic_dev.  Temperature
    only: a top-k / top-p target distribution is formed by probs_from_logits
    and verified by verify_chain_stochastic_dev."""
    lg = _logits_2d(logits)
    rows, vocab = lg.shape
    K = rows - 1
    if draft_tokens.numel() != K:
        raise ValueError(f"{rows} logit rows need {K} draft tokens, got {draft_tokens.numel()}")
    if K > 0:
        q2 = _logits_2d(q)
        if q2.shape[0] < K:
            raise ValueError(f"q has {q2.shape[0]} rows, {K} needed")
        head_rows, ldq, qp = q2.shape[1], q2.stride(0), ptr(q2)
    else:
        head_rows, ldq, qp = 1, 1, None
    if d2t is not None and d2t.numel() != head_rows:
        raise ValueError(f"d2t has {d2t.numel()} entries for {head_rows} draft rows")
    verdict = new_verdict(lg.device) if verdict is None else verdict
    _lib.call("wc_verify_chain_stochastic_logits", ptr(lg), rows, vocab, lg.stride(0), float(temperature), qp,
              head_rows, ldq, ptr(d2t) if d2t is not None else None, ptr(draft_tokens) if K > 0 else None,
              ptr(draft_rows) if draft_rows is not None else None, C.byref(rng), ptr(verdict),
              ptr(workspace(lg.device)), stream_ptr())
    return verdict


def verify_chain_stochastic(p: torch.Tensor, q: torch.Tensor, draft_tokens, rng: PhiloxStream,
                            d2t: torch.Tensor | None = None) -> tuple[int, int]:
    """p (K+1, V) target probabilities, q (K, H) draft probabilities the tokens were
    drawn from -> (n_accepted, next_token) (python/woodcock/sampling.py:69-82).
    Advances ``rng.round`` by one."""
    p2 = _logits_2d(p)
    dev = p2.device
    d = draft_tokens if isinstance(draft_tokens, torch.Tensor) else i32(list(draft_tokens), dev)
    rd = rng.device_round(dev)
    u = rng.struct(rd)
    v = read_verdict(verify_chain_stochastic_dev(p2, q, d.to(dev, torch.int32), u, d2t))
    rng.round += 1
    return int(v.n_accepted), int(v.next)


def verify_tree_stochastic_dev(p: torch.Tensor, q: torch.Tensor | None, tree_tokens: torch.Tensor,
                               tree_parents: torch.Tensor, rng: _lib.Uniforms, d2t: torch.Tensor | None = None,
                               verdict: torch.Tensor | None = None) -> torch.Tensor:
    """Enqueue the stochastic tree rule; p (N, V) target probabilities per node,
    q (N, H) the draft distribution each node's children were drawn from, over
    the H head rows (rows of leaves unused; d2t maps row -> token, None = identity)."""
    p2 = _logits_2d(p)
    N, vocab = p2.shape
    if tree_tokens.numel() != N or tree_parents.numel() != N:
        raise ValueError(f"{N} probability rows need {N} tree tokens and parents")
    if N > 1:
        if q is None:
            raise ValueError("q is required for a tree with children")
        q2 = _logits_2d(q)
        if q2.shape[0] < N:
            raise ValueError(f"q has {q2.shape[0]} rows, {N} needed")
        head_rows, ldq, qp = q2.shape[1], q2.stride(0), ptr(q2)
    else:
        head_rows, ldq, qp = 1, 1, None
    if d2t is not None and d2t.numel() != head_rows:
        raise ValueError(f"d2t has {d2t.numel()} entries for {head_rows} draft rows")
    verdict = new_verdict(p2.device) if verdict is None else verdict
    _lib.call("wc_verify_tree_stochastic", ptr(p2), N, vocab, p2.stride(0), qp, head_rows, ldq,
              ptr(d2t) if d2t is not None else None, ptr(tree_tokens), ptr(tree_parents), C.byref(rng),
              ptr(verdict), ptr(workspace(p2.device)), stream_ptr())
    return verdict


def verify_tree_stochastic(p: torch.Tensor, q: torch.Tensor | None, tree: DraftTree, rng: PhiloxStream,
                           d2t: torch.Tensor | None = None) -> tuple[list[int], int]:
    """Recursive rejection down the tree (python/woodcock/sampling.py:143-177):
    -> (accepted node path, next token).  Advances ``rng.round`` by one."""
    p2 = _logits_2d(p)
    dev = p2.device
    rd = rng.device_round(dev)
    v = read_verdict(verify_tree_stochastic_dev(p2, q, i32(tree.tokens, dev), i32(tree.parents, dev),
                                                rng.struct(rd), d2t))
    rng.round += 1
    if v.status != 0:
        raise ValueError("invalid tree, token or d2t")
    return [int(v.keep[1 + i]) for i in range(v.n_accepted)], int(v.next)


def tree_attention_mask_dev(parents: torch.Tensor, prefix_len: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """(N, prefix_len + N) uint8 mask on the device: the prefix plus each node's
    ancestors (python/woodcock/sampling.py:118-128)."""
    n = parents.numel()
    out = torch.empty(n, prefix_len + n, dtype=torch.uint8, device=parents.device) if out is None else out
    if out.dtype != torch.uint8 or out.shape[0] != n or out.shape[1] < prefix_len + n or out.stride(1) != 1:
        raise ValueError("out must be a uint8 (N, >= prefix_len + N) tensor")
    _lib.call("wc_tree_mask", ptr(parents), n, prefix_len, ptr(out), out.stride(0), stream_ptr())
    return out


def sample_without_replacement_dev(q: torch.Tensor, k: int | torch.Tensor, rng: _lib.Uniforms,
                                   d2t: torch.Tensor | None = None, uniform_base: int = 0
                                   ) -> tuple[torch.Tensor, torch.Tensor]:
    """Gumbel-top-k per row of q (rows, H) over the head rows
    (python/woodcock/sampling.py:196-203): -> (tokens (rows, k_max), counts (rows,)).
    Row r consumes one uniform per nonzero entry after those of rows < r."""
    q2 = _logits_2d(q)
    rows, H = q2.shape
    if isinstance(k, torch.Tensor):
        k_dev, k_max = k.to(q2.device, torch.int32).contiguous(), int(k.max())
    else:
        k_dev, k_max = None, int(k)
    if d2t is not None and d2t.numel() != H:
        raise ValueError(f"d2t has {d2t.numel()} entries for {H} draft rows")
    toks = torch.full((rows, k_max), -1, dtype=torch.int32, device=q2.device)
    counts = torch.zeros(rows, dtype=torch.int32, device=q2.device)
    _lib.call("wc_sample_without_replacement", ptr(q2), rows, H, q2.stride(0), ptr(d2t) if d2t is not None else None,
              ptr(k_dev) if k_dev is not None else None, k_max, C.byref(rng), int(uniform_base), ptr(toks),
              ptr(counts), stream_ptr())
    return toks, counts

