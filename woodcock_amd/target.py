"""Verify-width target forward (python/woodcock/target.py).

``TargetLayer`` holds one Qwen3 decoder layer's device weights (the reference's
parameter names, python/woodcock/target.py:142-156 / mlx-lm Qwen3) and runs
``wc_target_layer`` over a verify block of up to 64 rows: the tree or chain
block at explicit positions with an explicit mask (target.py:82-116).
``TargetModel`` is the whole forward of ``Target.__call__`` (target.py:82-116):
embedding rows, every decoder layer, the feature taps at ``feature_layers``
(target.py:26-32,108-111) and the tied LM head over the final norm
(target.py:73-76,113-114) -- all device-side, one workspace and RoPE table
shared by the layers.
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
FEW_ROWS = 8  # chain verify blocks up to this many rows may run on the few-row path
FEW_ROWS_MAX_KEYS = 1024  # ... with more than 4 query vectors: contexts up to this many keys

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
    vocab_size: int = 151936
    tie_word_embeddings: bool = True


def frag_weights(w: torch.Tensor) -> torch.Tensor:
    """The fragment-major copy of a bf16 [rows, cols] matrix that the
    verify-width GEMMs stream (wc_weights_frag), rows padded with zeros to a
    multiple of 16."""
    device_of(w)
    rows = (w.shape[0] + 15) // 16 * 16
    if rows != w.shape[0]:
        w = torch.cat([w, w.new_zeros(rows - w.shape[0], w.shape[1])])
    out = torch.empty_like(w)
    _lib.call("wc_weights_frag", ptr(w), w.shape[0], w.shape[1], ptr(out), stream_ptr())
    return out


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
        # the matrices in the GEMMs' fragment-major order, the gains as they are
        self.wf = {name: frag_weights(t) if t.dim() == 2 else t for name, t in self.w.items()}
        self.lw = _lib.LayerWeights()
        for f, name in LAYER_NAMES.items():
            setattr(self.lw, f, ptr(self.wf[name]))
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
            mask = _mask_rows(mask, self.device, rows)
        _lib.call("wc_target_layer", C.byref(self.dims), C.byref(self.lw), ptr(cos), ptr(sin), cos.shape[0], ptr(x),
                  rows, ptr(pos) if pos is not None else None, ptr(mask) if mask is not None else None,
                  mask.stride(0) if mask is not None else 0, ptr(cache.keys), ptr(cache.values),
                  _lib.WC_BF16 if cache.keys.dtype == torch.bfloat16 else _lib.WC_F32, cache.capacity,
                  ptr(offset_dev), None, 0, ptr(self.ws), stream_ptr())
        return x


def _mask_rows(mask: torch.Tensor, device: torch.device, rows: int) -> torch.Tensor:
    """The [rows, >= offset + rows] uint8 mask as the layer reads it: rows may
    be strided (a row view of a wider buffer is used in place, and a row stride
    that is a multiple of 16 bytes lets the attention read 16 mask bytes at a
    time); anything else is copied."""
    mask = mask.to(device, torch.uint8)
    if mask.dim() != 2 or mask.shape[0] != rows:
        raise ValueError("mask must have one row per input row")
    if mask.stride(1) != 1 or mask.stride(0) < mask.shape[1]:
        mask = mask.contiguous()
    return mask


def default_feature_layers(num_layers: int) -> tuple[int, int, int]:
    """Low / mid / high taps (python/woodcock/target.py:26-32)."""
    return (2, num_layers // 2, num_layers - 3)


def random_target(cfg: TargetConfig, seed: int = 0, device="cuda", std: float = 0.02) -> dict[str, torch.Tensor]:
    """Random-init weights of the whole target under the reference's names."""
    out = {}
    for i in range(cfg.num_layers):
        for name, t in random_layer(cfg, seed=seed * 1000 + i, device=device, std=std).items():
            out[f"layers.{i}.{name}"] = t
    g = torch.Generator(device=device)
    g.manual_seed(seed + 17)
    out["embed_tokens.weight"] = (std * torch.randn(cfg.vocab_size, cfg.hidden_size, generator=g,
                                                    device=device)).to(torch.bfloat16)
    out["norm.weight"] = (1.0 + 0.1 * torch.randn(cfg.hidden_size, generator=g, device=device)).to(torch.bfloat16)
    if not cfg.tie_word_embeddings:
        out["lm_head.weight"] = (std * torch.randn(cfg.vocab_size, cfg.hidden_size, generator=g,
                                                   device=device)).to(torch.bfloat16)
    return out


class TargetModel:
    """The verify forward of the target over a block of up to 64 rows."""

    def __init__(self, cfg: TargetConfig, weights: dict[str, torch.Tensor], device="cuda", max_rows: int = MAX_ROWS,
                 feature_layers: tuple[int, ...] | None = None):
        self.cfg = cfg
        self.device = torch.device(device)
        self.feature_layers = tuple(feature_layers or default_feature_layers(cfg.num_layers))
        shapes = layer_shapes(cfg)
        self.w: dict[str, torch.Tensor] = {}
        self.wr: dict[str, torch.Tensor] = {}  # row-major matrices: the few-row path
        self.lw = []
        self.lwr = []
        for i in range(cfg.num_layers):
            lw, lwr = _lib.LayerWeights(), _lib.LayerWeights()
            for f, name in LAYER_NAMES.items():
                t = weights[f"layers.{i}.{name}"]
                if tuple(t.shape) != shapes[name]:
                    raise ValueError(f"layers.{i}.{name}: shape {tuple(t.shape)}, expected {shapes[name]}")
                t = t.to(self.device, torch.bfloat16).contiguous()
                setattr(lwr, f, ptr(t))
                if t.dim() == 2:  # the verify-width GEMMs stream the fragment-major copy
                    self.wr[f"layers.{i}.{name}"] = t
                    t = frag_weights(t)
                self.w[f"layers.{i}.{name}"] = t
                setattr(lw, f, ptr(t))
            # the few-row path's gate / up pair streams the fragment-major copies
            lwr.gate_frag = ptr(self.w[f"layers.{i}.mlp.gate_proj.weight"])
            lwr.up_frag = ptr(self.w[f"layers.{i}.mlp.up_proj.weight"])
            self.lw.append(lw)
            self.lwr.append(lwr)
        for name, shape in (("embed_tokens.weight", (cfg.vocab_size, cfg.hidden_size)),
                            ("norm.weight", (cfg.hidden_size,))):
            t = weights[name]
            if tuple(t.shape) != shape:
                raise ValueError(f"{name}: shape {tuple(t.shape)}, expected {shape}")
            self.w[name] = t.to(self.device, torch.bfloat16).contiguous()
        head = "embed_tokens.weight" if cfg.tie_word_embeddings else "lm_head.weight"
        if head not in self.w:
            self.w[head] = weights[head].to(self.device, torch.bfloat16).contiguous()
        self.head = frag_weights(self.w[head])  # the embedding gather keeps the row-major table
        self.dims = _lib.DrafterDims(cfg.hidden_size, 1, cfg.num_heads, cfg.num_kv_heads, cfg.head_dim,
                                     cfg.intermediate_size, cfg.hidden_size, 3, 1, 1, cfg.rms_norm_eps, 0)
        self.max_rows = max_rows
        n = _lib.lib().wc_target_workspace_bytes(C.byref(self.dims), max_rows)
        self.ws = torch.zeros(n, dtype=torch.uint8, device=self.device)  # split-K counters start at zero
        self._rope: tuple[torch.Tensor, torch.Tensor] | None = None
        self.x = torch.empty(max_rows, cfg.hidden_size, dtype=torch.float32, device=self.device)
        # few-row path: groups of up to WC_MAX_DRAFTER_LAYERS decoder layers per
        # wc_drafter_forward call (a drafter layer without the token stream is a
        # Qwen3 decoder layer), split after every feature layer
        self.fdims = _lib.DrafterDims(cfg.hidden_size, 1, cfg.num_heads, cfg.num_kv_heads, cfg.head_dim,
                                      cfg.intermediate_size, cfg.hidden_size, 1, 1, cfg.vocab_size,
                                      cfg.rms_norm_eps, 0)
        n = int(_lib.lib().wc_drafter_workspace_bytes(C.byref(self.fdims)))
        self.fws = torch.empty((n + 255) // 256 * 256, dtype=torch.uint8, device=self.device)
        _lib.call("wc_workspace_init", ptr(self.fws), self.fws.numel(), stream_ptr())
        self.x2 = torch.empty_like(self.x)
        self._groups = []
        g0 = 0
        for i in range(cfg.num_layers):
            if i - g0 + 1 == _lib.WC_MAX_DRAFTER_LAYERS or i in self.feature_layers or i == cfg.num_layers - 1:
                self._groups.append((g0, i + 1))
                g0 = i + 1
        self._fw_key = None
        self._fw: list[tuple[_lib.DrafterDims, _lib.DrafterWeights]] = []

    def make_cache(self, capacity: int, dtype=torch.bfloat16) -> list[KVCache]:
        return [KVCache(self.cfg.num_kv_heads, self.cfg.head_dim, capacity, dtype, self.device)
                for _ in range(self.cfg.num_layers)]

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

    def __call__(self, tokens: torch.Tensor, cache: list[KVCache], offset_dev: torch.Tensor,
                 positions: torch.Tensor | None = None, mask: torch.Tensor | None = None,
                 logits: torch.Tensor | None = None, taps: list[torch.Tensor] | None = None
                 ) -> tuple[torch.Tensor, list[torch.Tensor]]:
        """tokens [rows] int32 on the device -> (logits [rows, vocab] fp32, feature taps
        [rows, hidden] fp32 at feature_layers).  K/V of the block land at cache slots
        *offset_dev .. + rows of every layer (the caller advances the offsets);
        enqueue only, no host synchronisation."""
        cfg = self.cfg
        rows = tokens.numel()
        if not 1 <= rows <= self.max_rows:
            raise ValueError(f"rows must be in 1..{self.max_rows}")
        if len(cache) != cfg.num_layers:
            raise ValueError(f"{cfg.num_layers} cache layers needed, got {len(cache)}")
        cap = cache[0].capacity
        cos, sin = self.rope(cap + 64)
        pos = None if positions is None else positions.to(self.device, torch.int32).contiguous()
        if mask is not None:
            mask = _mask_rows(mask, self.device, rows)
        kvdt = _lib.WC_BF16 if cache[0].keys.dtype == torch.bfloat16 else _lib.WC_F32
        x = self.x[:rows]
        s = stream_ptr()
        tok = tokens.to(self.device, torch.int32).contiguous()
        _lib.call("wc_target_embed", ptr(self.w["embed_tokens.weight"]), cfg.vocab_size, cfg.hidden_size, ptr(tok),
                  rows, ptr(x), x.stride(0), s)
        if taps is None:
            taps = [torch.empty(rows, cfg.hidden_size, dtype=torch.float32, device=self.device)
                    for _ in self.feature_layers]
        final_norm = self.w["norm.weight"]
        if mask is None and self._few_rows_fit(rows, cache[0].offset + rows):
            return self._few_rows(tok, rows, cache, offset_dev, pos, kvdt, cos, sin, logits, taps)
        for i in range(cfg.num_layers):
            c = cache[i]
            # each layer leaves the next one's (or the head's) normed activations
            # in the workspace: one prep launch per forward instead of per layer
            nxt = self.w[f"layers.{i + 1}.input_layernorm.weight"] if i + 1 < cfg.num_layers else final_norm
            _lib.call("wc_target_layer", C.byref(self.dims), C.byref(self.lw[i]), ptr(cos), ptr(sin), cos.shape[0],
                      ptr(x), rows, ptr(pos) if pos is not None else None, ptr(mask) if mask is not None else None,
                      mask.stride(0) if mask is not None else 0, ptr(c.keys), ptr(c.values), kvdt, c.capacity,
                      ptr(offset_dev), ptr(nxt), int(i > 0), ptr(self.ws), s)
            for j, f in enumerate(self.feature_layers):
                if f == i:
                    taps[j][:rows].copy_(x)
        if logits is None:
            logits = torch.empty(rows, cfg.vocab_size, dtype=torch.float32, device=self.device)
        _lib.call("wc_target_head", C.byref(self.dims), ptr(self.head), ptr(final_norm), ptr(x), rows,
                  cfg.vocab_size, ptr(logits), logits.stride(0), 1, ptr(self.ws), s)
        return logits, taps

    def _few_rows_fit(self, rows: int, keys: int) -> bool:
        """Whether a mask-less block runs on the few-row path: its query vectors
        (rows x GQA group) fit one decode-attention block, and either the
        attention merges its splits in the same launch (<= 4 vectors) or every
        split holds one 32-key chunk (keys <= 1024; `keys` is the host's view of
        the cache offset plus the block -- the choice affects speed only).
        Measured: Qwen3-1.7B at 5 rows, context 512: 28 layers + head 2038 ->
        1738 us; Qwen3-4B at one row, context 4096: 3.74 -> 2.66 ms; Qwen3-4B at
        2..8 rows, context 4096 (several chunks per split for 8+ query vectors,
        or two row tiles that stream the weights twice): slower than the
        verify-width path."""
        qv = rows * (self.cfg.num_heads // self.cfg.num_kv_heads)
        return rows <= FEW_ROWS and qv <= 16 and (qv <= 4 or keys <= FEW_ROWS_MAX_KEYS)

    def _few_weights(self, cos: torch.Tensor, sin: torch.Tensor):
        """(dims, weights) of each layer group for wc_drafter_forward, rebuilt when
        the RoPE table moves."""
        key = (cos.data_ptr(), sin.data_ptr(), cos.shape[0])
        if key != self._fw_key:
            self._fw = []
            for g0, g1 in self._groups:
                dims = _lib.DrafterDims.from_buffer_copy(self.fdims)
                dims.num_layers = g1 - g0
                W = _lib.DrafterWeights()
                W.embed = ptr(self.w["embed_tokens.weight"])
                W.final_norm = ptr(self.w["norm.weight"])
                W.rope_cos, W.rope_sin, W.rope_max_pos = ptr(cos), ptr(sin), cos.shape[0]
                for j in range(g1 - g0):
                    W.layers[j] = self.lwr[g0 + j]
                self._fw.append((dims, W))
            self._fw_key = key
        return self._fw

    def _few_rows(self, tok, rows, cache, offset_dev, pos, kvdt, cos, sin, logits, taps):
        """A chain verify block of <= FEW_ROWS rows without a mask: the decoder
        layers on the drafter's one-/few-row GEMVs over the row-major weights
        (K split over the waves of a block, 1 KB weight rows per load) and the
        decode attention that normalises, rotates and appends on the fly -- six
        launches per layer against eleven on the verify-width path."""
        cfg = self.cfg
        s = stream_ptr()
        x, xo = self.x[:rows], self.x2[:rows]
        for (g0, g1), (dims, W) in zip(self._groups, self._few_weights(cos, sin)):
            kp = (C.c_void_p * (g1 - g0))(*[cache[i].keys.data_ptr() for i in range(g0, g1)])
            vp = (C.c_void_p * (g1 - g0))(*[cache[i].values.data_ptr() for i in range(g0, g1)])
            _lib.call("wc_drafter_forward", C.byref(dims), C.byref(W), ptr(tok), ptr(x), x.stride(0), None, 0, rows,
                      None, kp, vp, kvdt, cache[g0].capacity, ptr(offset_dev), 0,
                      ptr(pos) if pos is not None else None, None, 0, ptr(xo), None, None, ptr(self.fws), s)
            x, xo = xo, x
            for j, f in enumerate(self.feature_layers):
                if f == g1 - 1:
                    taps[j][:rows].copy_(x)
        if logits is None:
            logits = torch.empty(rows, cfg.vocab_size, dtype=torch.float32, device=self.device)
        _lib.call("wc_target_head", C.byref(self.dims), ptr(self.head), ptr(self.w["norm.weight"]), ptr(x), rows,
                  cfg.vocab_size, ptr(logits), logits.stride(0), 0, ptr(self.ws), s)
        return logits, taps

