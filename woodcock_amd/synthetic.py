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


class SyntheticTarget:
    """Stand-in for the verify-width target forward: fixed target logits
    [K+1, V] fp32 ~ N(0, scale^2) and feature taps [K+1, Dt].

    ``plant(drafts_dev, n_agree)`` makes rows i < n_agree take the drafted token
    d_{i+1} as their argmax and keeps row n_agree away from d_{n_agree+1}, so a
    greedy verify accepts exactly n_agree drafts.  It runs as device ops on
    device-resident drafts (capturable in a graph) and restores the previous
    round's plant first; n_agree is a host int or a device int32 [1].

    As a decoder's target (``verify_forward``), the agreement of each round is
    drawn on the host before the round (``prepare``): with ``agree_p`` set,
    every draft position agrees independently with probability agree_p
    (seeded), so the round accepts the drafts before the first disagreeing one;
    the count goes to the device, where the plant reads it."""

    BIG, BLOCK = 1.0e4, -1.0e4

    def __init__(self, k: int, vocab: int, target_hidden: int, num_features: int = 3, device="cuda", seed: int = 0,
                 scale: float = 3.0, tap_dtype=torch.bfloat16, agree_p: float | None = None):
        g = torch.Generator(device=device)
        g.manual_seed(seed)
        self.logits = scale * torch.randn(k + 1, vocab, generator=g, device=device, dtype=torch.float32)
        self.taps = [torch.randn(k + 1, target_hidden, generator=g, device=device, dtype=torch.float32).to(tap_dtype)
                     for _ in range(num_features)]
        self.k = k
        self.vocab_size = vocab
        self.cache = None
        dev = self.logits.device
        self._rows = torch.arange(k, device=dev)
        self._prev_idx = torch.zeros(k, dtype=torch.long, device=dev)
        self._prev_val = self.logits[self._rows, self._prev_idx].clone()
        self._big = torch.full((k,), self.BIG, device=dev)
        self._block = torch.full((k,), self.BLOCK, device=dev)
        self.agree_p = agree_p
        self._rng = np.random.default_rng(seed + 0x5eed)
        self.n_agree_dev = torch.zeros(1, dtype=torch.int32, device=dev)
        self._n_agree_host = torch.zeros(1, dtype=torch.int32, pin_memory=dev.type == "cuda")
        self.agreements: list[int] = []

    def plant(self, drafts_dev: torch.Tensor, n_agree) -> None:
        rows = self._rows
        self.logits.index_put_((rows, self._prev_idx), self._prev_val)  # undo the previous plant
        self._prev_idx.copy_(drafts_dev[: self.k].long())
        self._prev_val.copy_(self.logits[rows, self._prev_idx])
        vals = torch.where(rows < n_agree, self._big, torch.where(rows == n_agree, self._block, self._prev_val))
        self.logits.index_put_((rows, self._prev_idx), vals)

    def set_agreement(self, n: int) -> None:
        """The next plant's agreeing row count (enqueued host -> device copy)."""
        self._n_agree_host[0] = int(n)
        self.n_agree_dev.copy_(self._n_agree_host, non_blocking=True)

    def prepare(self, rows: int) -> None:
        """Draw this round's agreement (chain of rows - 1 drafts), when agree_p is set."""
        if self.agree_p is None:
            return
        k = rows - 1
        hits = self._rng.random(k) < self.agree_p
        n = int(np.argmin(hits)) if not hits.all() else k
        self.agreements.append(n)
        self.set_agreement(n)

    def verify_forward(self, tokens: torch.Tensor, rows: int, offset_dev: torch.Tensor,
                       positions: torch.Tensor | None = None, mask: torch.Tensor | None = None):
        """Logits / taps of the verify block [x_n, d_1..d_K] (tokens [>= k + 1],
        device): the drafts planted with the device agreement count."""
        if rows > self.k + 1:
            raise ValueError(f"synthetic target holds {self.k + 1} rows, {rows} requested")
        self.plant(tokens[1:self.k + 1], self.n_agree_dev)
        return self.logits[:rows], [t[:rows] for t in self.taps]


def stochastic_workload(k: int, vocab: int, head_rows: int, seed: int = 0, zipf_s: float = 1.1,
                        noise: float = 0.5, always=()):
    """Accept/reject workload (host numpy): target logits [k+1, vocab] fp32 =
    log of a Zipf(s) law over a seeded permutation per row; a head_rows-entry
    ascending draft vocabulary d2t; draft logits [k, head_rows] fp32 =
    log p_i[d2t] + N(0, noise^2), so q_i = softmax of them is close to but not
    equal to p_i restricted to the draft vocabulary."""
    rng = np.random.default_rng(seed)
    ranks = np.arange(1, vocab + 1, dtype=np.float64)
    law = ranks ** -zipf_s
    law /= law.sum()
    logits = np.empty((k + 1, vocab), np.float32)
    for i in range(k + 1):
        logits[i, rng.permutation(vocab)] = np.log(law).astype(np.float32)
    # the draft vocabulary: row 0's likeliest half plus seeded draft_vocab ids
    top = np.argsort(-logits[0])[: head_rows // 2]
    rest = np.setdiff1d(draft_vocab(vocab, head_rows, seed=seed, always=always), top)
    d2t = np.sort(np.concatenate([top, rest[: head_rows - len(top)]])).astype(np.int32)
    draft_logits = (logits[:k][:, d2t] + noise * rng.standard_normal((k, len(d2t)))).astype(np.float32)
    return logits, draft_logits, d2t


def draw_rows(q_rows: np.ndarray, n: int, rng: np.random.Generator) -> np.ndarray:
    """n independent draws of a head row from each distribution q_rows[i] -> [n, K] int32."""
    c = np.cumsum(np.asarray(q_rows, np.float64), axis=-1)
    u = rng.random((n, q_rows.shape[0])) * c[:, -1]
    return np.stack([np.minimum(np.searchsorted(c[i], u[:, i], side="right"), c.shape[1] - 1)
                     for i in range(q_rows.shape[0])], axis=1).astype(np.int32)
