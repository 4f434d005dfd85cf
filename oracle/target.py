"""CPU restatement of the target's verify forward (test infrastructure only).

Target.__call__ with explicit positions and mask (python/woodcock/target.py:82-116):
the embedding rows, every decoder layer (target.py:142-156; the layer loop of
src/core/qwen3.cpp:86-111), the feature taps after the layers in
``feature_layers`` (target.py:26-32,108-111) and the tied LM head over the
final norm (target.py:73-76,113-114).

Each decoder layer is the oracle drafter's layer (``core.Drafter``, one layer,
its own KV cache) with the token stream absent: QKV = W . RMS_in(h) only, which
is a plain Qwen3 layer.  Chaining one such layer per target layer exposes the
residual stream after every layer, so the taps come from the same pass as the
logits.  The last layer's drafter output (RMSNorm with the target's final norm)
times the embedding matrix is the LM head.  Pinned by the reference C++
``Qwen3::forward`` goldens (tests/test_oracle.py).
"""
from __future__ import annotations

import numpy as np

from . import core

LAYER_KEYS = ("input_layernorm.weight", "post_attention_layernorm.weight", "self_attn.q_proj.weight",
              "self_attn.k_proj.weight", "self_attn.v_proj.weight", "self_attn.o_proj.weight",
              "self_attn.q_norm.weight", "self_attn.k_norm.weight", "mlp.gate_proj.weight",
              "mlp.up_proj.weight", "mlp.down_proj.weight")


class TargetStack:
    """cfg: a target.TargetConfig-like object; weights: reference names ->
    uint16 bf16 bits (``layers.{i}.*``, ``embed_tokens.weight``, ``norm.weight``)."""

    def __init__(self, cfg, weights: dict[str, np.ndarray], feature_layers, cap: int, kv_bf16: bool = True):
        self.cfg = cfg
        self.feature_layers = tuple(feature_layers)
        d = cfg.hidden_size
        self.embed = weights["embed_tokens.weight"]
        dummy_embed = np.zeros((1, d), np.uint16)
        dummy_fc = np.zeros((1, 8), np.uint16)
        self.layers, self.caches = [], []
        for i in range(cfg.num_layers):
            last = i == cfg.num_layers - 1
            w = {f"layers.0.{n}": weights[f"layers.{i}.{n}"] for n in LAYER_KEYS}
            w["embed_tokens.weight"] = dummy_embed
            w["fc.weight"] = dummy_fc
            w["norm.weight"] = weights["norm.weight"]
            w["lm_head.weight"] = self.embed if last else np.zeros((1, d), np.uint16)
            od = core.Drafter(dict(hidden_size=d, num_layers=1, num_heads=cfg.num_heads,
                                   num_kv_heads=cfg.num_kv_heads, head_dim=cfg.head_dim,
                                   intermediate_size=cfg.intermediate_size, target_hidden_size=d,
                                   vocab_size=cfg.vocab_size, rms_norm_eps=cfg.rms_norm_eps,
                                   rope_theta=cfg.rope_theta, feature_norm=False), w)
            self.layers.append(od)
            self.caches.append(od.make_cache(cap, kv_bf16=kv_bf16))

    @property
    def offset(self) -> int:
        return self.caches[0].offset

    @offset.setter
    def offset(self, n: int) -> None:
        for c in self.caches:
            c.offset = n

    def forward(self, tokens, positions=None, mask=None):
        """tokens [rows] at the current offset (positions / mask [rows, offset + rows]
        optional) -> (logits [rows, vocab], taps [rows, hidden] per feature layer);
        every layer's cache advances by rows."""
        tokens = np.asarray(tokens, np.int64).reshape(-1)
        h = core.bf16_to_f32(self.embed[tokens])
        taps = {}
        out = None
        for i, (od, c) in enumerate(zip(self.layers, self.caches)):
            h, out = od.forward(np.zeros(len(tokens), np.int32), h, c, positions=positions, mask=mask)
            if i in self.feature_layers:
                taps[i] = h.copy()
        logits = self.layers[-1].logits(out)
        return logits, [taps[f] for f in self.feature_layers]

    def compact(self, start: int, keep) -> None:
        """compact_cache (target.py:159-175) on every layer."""
        for c in self.caches:
            core.kv_compact(c.k, c.v, start, keep)
            c.offset = start + len(keep)
