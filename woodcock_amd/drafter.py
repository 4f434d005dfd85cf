"""The EAGLE-3 drafter on the GPU (python/woodcock/drafter.py:130-232 API).

    g_t = FC([RMS_1(f_low); RMS_2(f_mid); RMS_3(f_high)])
    QKV = W . RMS(h) + W_aux . RMS(e(x))        (layer 0; later layers single-stream)
    out = RMSNorm(h_L)                          (fed back as the next feature with post_norm)

Weights stay bf16 in HBM; activations are fp32; the KV cache is bf16 (or fp32
for the tight parity mode).  Every method enqueues HIP kernels through the C
ABI on the current stream; nothing falls back to the CPU.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import _lib
from .cache import KVCache
from .config import DrafterConfig
from .runtime import device_of, ptr, stream_ptr

_F32, _BF16 = _lib.WC_F32, _lib.WC_BF16


def _as_rows(x: torch.Tensor, width: int) -> torch.Tensor:
    """(B=1, L, width) or (L, width) -> contiguous-rows 2-D view."""
    if x.dim() == 3:
        if x.shape[0] != 1:
            raise ValueError("batch size 1 only")
        x = x[0]
    if x.dim() == 1:
        x = x[None]
    if x.dim() != 2 or x.shape[1] != width:
        raise ValueError(f"expected rows of width {width}, got shape {tuple(x.shape)}")
    if x.stride(1) != 1:
        x = x.contiguous()
    return x


class Drafter:
    def __init__(self, cfg: DrafterConfig, weights: dict[str, torch.Tensor], device=None, kv_dtype=torch.bfloat16):
        if cfg.num_layers > _lib.WC_MAX_DRAFTER_LAYERS:
            raise ValueError(f"at most {_lib.WC_MAX_DRAFTER_LAYERS} drafter layers")
        if cfg.num_features > _lib.WC_MAX_FEATURES:
            raise ValueError(f"at most {_lib.WC_MAX_FEATURES} target features")
        self.cfg = cfg
        dev = torch.device(device) if device is not None else next(iter(weights.values())).device
        self.device = dev
        self.kv_dtype = kv_dtype
        self.w = {}
        for k, v in weights.items():
            t = v.to(dev)
            if t.dtype != torch.bfloat16:
                t = t.to(torch.bfloat16)
            self.w[k] = t.contiguous()
        device_of(self.w["fc.weight"])
        self._vocab_ids: torch.Tensor | None = None
        self._head = self.w["lm_head.weight"]
        self._rope = None
        self._build_structs(8192)
        n = int(_lib.lib().wc_drafter_workspace_bytes(C.byref(self.dims)))
        self.ws = torch.empty((n + 255) // 256 * 256, dtype=torch.uint8, device=dev)
        _lib.call("wc_workspace_init", ptr(self.ws), self.ws.numel(), stream_ptr())

    # ------------------------------------------------------------------ setup

    def _build_structs(self, rope_positions: int) -> None:
        c = self.cfg
        self.dims = _lib.DrafterDims(c.hidden_size, c.num_layers, c.num_heads, c.num_kv_heads, c.head_dim,
                                     c.intermediate_size, c.target_hidden_size, c.num_features,
                                     self._head.shape[0], self.w["embed_tokens.weight"].shape[0],
                                     c.rms_norm_eps, int(c.window or 0))
        self._ensure_rope(rope_positions)
        W = _lib.DrafterWeights()
        W.embed = self.w["embed_tokens.weight"].data_ptr()
        W.fc = self.w["fc.weight"].data_ptr()
        for i in range(c.num_features):
            t = self.w.get(f"feature_norms.{i}.weight") if c.feature_norm else None
            W.feature_norm[i] = None if t is None else t.data_ptr()
        W.final_norm = self.w["norm.weight"].data_ptr()
        W.head = self._head.data_ptr()
        W.d2t = None if self._vocab_ids is None else self._vocab_ids.data_ptr()
        W.rope_cos = self._rope[0].data_ptr()
        W.rope_sin = self._rope[1].data_ptr()
        W.rope_max_pos = self._rope[0].shape[0]
        names = {"in_norm": "input_layernorm", "post_norm": "post_attention_layernorm", "aux_norm": "aux_norm",
                 "q": "self_attn.q_proj", "k": "self_attn.k_proj", "v": "self_attn.v_proj",
                 "o": "self_attn.o_proj", "aux_q": "self_attn.aux_q", "aux_k": "self_attn.aux_k",
                 "aux_v": "self_attn.aux_v", "q_norm": "self_attn.q_norm", "k_norm": "self_attn.k_norm",
                 "gate": "mlp.gate_proj", "up": "mlp.up_proj", "down": "mlp.down_proj"}
        for i in range(c.num_layers):
            L = W.layers[i]
            for field, name in names.items():
                t = self.w.get(f"layers.{i}.{name}.weight")
                if t is None and field not in ("aux_norm", "aux_q", "aux_k", "aux_v"):
                    raise ValueError(f"missing weight layers.{i}.{name}.weight")
                setattr(L, field, None if t is None else t.data_ptr())
        self.wstruct = W

    @property
    def pending_ok(self) -> bool:
        """The chain may leave each head's argmax pending for the next forward
        (wc_draft_head_norm_pending / wc_drafter_forward_pending): the first
        layer takes the token stream and hidden_size is a multiple of 512."""
        h = self.cfg.hidden_size
        return "layers.0.aux_norm.weight" in self.w and h % 512 == 0 and h <= 10240

    def _ensure_rope(self, positions: int) -> None:
        if self._rope is not None and self._rope[0].shape[0] >= positions:
            return
        n = 1 << max(13, int(positions - 1).bit_length())
        half = self.cfg.head_dim // 2
        cos = np.empty((n, half), dtype=np.float32)
        sin = np.empty_like(cos)
        _lib.call("wc_rope_table", cos.ctypes.data_as(C.c_void_p), sin.ctypes.data_as(C.c_void_p), n,
                  self.cfg.head_dim, self.cfg.rope_theta)
        self._rope = (torch.from_numpy(cos).to(self.device), torch.from_numpy(sin).to(self.device))
        if hasattr(self, "wstruct"):
            self.wstruct.rope_cos = self._rope[0].data_ptr()
            self.wstruct.rope_sin = self._rope[1].data_ptr()
            self.wstruct.rope_max_pos = n

    @classmethod
    def from_synthetic(cls, cfg: DrafterConfig, seed: int = 0, device="cuda", head_rows: int | None = None,
                       kv_dtype=torch.bfloat16) -> "Drafter":
        from .synthetic import random_drafter

        return cls(cfg, random_drafter(cfg, seed=seed, device=device, head_rows=head_rows), device, kv_dtype)

    @classmethod
    def load(cls, path, device="cuda", kv_dtype=torch.bfloat16, verify_sha: bool = True) -> "Drafter":
        """A local drafter directory in the reference format: config.json +
        model.safetensors, checked against woodcock.json when present
        (python/woodcock/drafter.py:321-330; python/woodcock/export.py:1-64)."""
        from .weights import read_drafter_dir

        cfg, weights, _ = read_drafter_dir(path, verify_sha)
        return cls(cfg, weights, device, kv_dtype)

    # ------------------------------------------------------------------ caches

    def make_cache(self, capacity: int = 4096, dtype=None) -> list[KVCache]:
        """One KV cache per layer, [1, kv_heads, capacity, head_dim] (drafter.py:231-232)."""
        self._ensure_rope(capacity + 64)
        return [KVCache(self.cfg.num_kv_heads, self.cfg.head_dim, capacity, dtype or self.kv_dtype, self.device)
                for _ in range(self.cfg.num_layers)]

    # ------------------------------------------------------------------ inference

    def fuse(self, feats: list[torch.Tensor]) -> torch.Tensor:
        """Target taps (each (B=1, L, target_hidden)) -> drafter-space feature g (L, hidden) fp32."""
        if len(feats) != self.cfg.num_features:
            raise ValueError(f"expected {self.cfg.num_features} feature taps, got {len(feats)}")
        rows = [_as_rows(f, self.cfg.target_hidden_size) for f in feats]
        dt = rows[0].dtype
        if dt not in (torch.float32, torch.bfloat16) or any(r.dtype != dt or r.shape != rows[0].shape for r in rows):
            raise ValueError("feature taps must share shape and dtype (float32 or bfloat16)")
        if any(r.stride(0) != rows[0].stride(0) for r in rows):
            rows = [r.contiguous() for r in rows]
        for r in rows:
            device_of(r)
        L = rows[0].shape[0]
        g = torch.empty(L, self.cfg.hidden_size, dtype=torch.float32, device=self.device)
        taps = (C.c_void_p * len(rows))(*[r.data_ptr() for r in rows])
        _lib.call("wc_drafter_fuse", C.byref(self.dims), C.byref(self.wstruct), taps,
                  _BF16 if dt == torch.bfloat16 else _F32, rows[0].stride(0), None, 0, L, None, ptr(g),
                  g.stride(0), ptr(self.ws), stream_ptr())
        return g

    def __call__(self, tokens, feat: torch.Tensor, cache: list[KVCache] | None = None, positions=None, mask=None):
        """One drafting forward (drafter.py:164-191).  tokens (B=1, L) ints; feat
        (B=1, L, hidden).  Returns (hidden, out) as (L, hidden) fp32; appends L
        entries to `cache` at cache[0].offset and advances every layer's offset.
        Without a cache a temporary one is used (attention over these L tokens)."""
        tok = torch.as_tensor(tokens).reshape(-1)
        L = tok.numel()
        f = _as_rows(feat, self.cfg.hidden_size)
        if f.shape[0] != L:
            raise ValueError(f"{L} tokens but {f.shape[0]} feature rows")
        if f.dtype != torch.float32:
            f = f.float()
        if cache is None:
            cache = self.make_cache(max(L, 1))
        offset = cache[0].offset
        cap = cache[0].capacity
        if offset + L > cap:
            raise ValueError(f"drafter cache capacity {cap} exceeded ({offset} + {L})")
        self._ensure_rope(cap + 64)
        dev = self.device
        tok = tok.to(dev, torch.int32)
        ints = torch.tensor([offset], dtype=torch.int32).to(dev)
        pos = None
        if positions is not None:
            pos = torch.as_tensor(positions).reshape(-1).to(dev, torch.int32)
            if pos.numel() != L:
                raise ValueError("one position per token")
            if int(pos.max()) >= self._rope[0].shape[0]:
                self._ensure_rope(int(pos.max()) + 1)
        m = None
        mask_ld = 0
        if mask is not None:
            mk = torch.as_tensor(np.asarray(mask) if not isinstance(mask, torch.Tensor) else mask)
            if mk.shape != (L, offset + L):
                raise ValueError(f"mask must be ({L}, {offset + L}), got {tuple(mk.shape)}")
            m = mk.to(dev, torch.uint8).contiguous()
            mask_ld = m.stride(0)
        hid = torch.empty(L, self.cfg.hidden_size, dtype=torch.float32, device=dev)
        out = torch.empty_like(hid)
        kp = (C.c_void_p * len(cache))(*[c.keys.data_ptr() for c in cache])
        vp = (C.c_void_p * len(cache))(*[c.values.data_ptr() for c in cache])
        kvdt = _BF16 if cache[0].keys.dtype == torch.bfloat16 else _F32
        _lib.call("wc_drafter_forward", C.byref(self.dims), C.byref(self.wstruct), ptr(tok), ptr(f), f.stride(0),
                  None, 0, L, None, kp, vp, kvdt, cap, ptr(ints), 0, ptr(pos), ptr(m), mask_ld, ptr(hid), ptr(out),
                  None, ptr(self.ws), stream_ptr())
        for c in cache:
            c.offset = offset + L
        return hid, out

    def feedback(self, hidden: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
        return out if self.cfg.post_norm else hidden

    def logits(self, out: torch.Tensor) -> torch.Tensor:
        """Draft logits over the head rows (full vocabulary or the restricted subset)."""
        o = _as_rows(out, self.cfg.hidden_size)
        if o.dtype != torch.float32:
            o = o.float()
        z = torch.empty(o.shape[0], self._head.shape[0], dtype=torch.float32, device=self.device)
        tok = torch.empty(o.shape[0], dtype=torch.int32, device=self.device)
        _lib.call("wc_draft_head", C.byref(self.dims), C.byref(self.wstruct), ptr(o), o.stride(0), None, 0,
                  o.shape[0], ptr(z), z.stride(0), ptr(tok), None, None, ptr(self.ws), stream_ptr())
        return z

    def draft(self, out: torch.Tensor, logits: torch.Tensor | None = None, rows: torch.Tensor | None = None,
              gumbel: tuple | None = None) -> torch.Tensor:
        """Fused head + argmax + d2t: the drafted token id per row of `out` (int32, device).
        gumbel = (seed, round_tensor, purpose, temperature) draws from softmax(z/T)."""
        o = _as_rows(out, self.cfg.hidden_size)
        if o.dtype != torch.float32:
            o = o.float()
        tok = torch.empty(o.shape[0], dtype=torch.int32, device=self.device)
        g = None
        if gumbel is not None:
            seed, rnd, purpose, temp = gumbel
            g = _lib.Gumbel(int(seed), rnd.data_ptr(), int(purpose), float(temp))
        _lib.call("wc_draft_head", C.byref(self.dims), C.byref(self.wstruct), ptr(o), o.stride(0), None, 0,
                  o.shape[0], ptr(logits), 0 if logits is None else logits.stride(0), ptr(tok), ptr(rows),
                  None if g is None else C.byref(g), ptr(self.ws), stream_ptr())
        return tok

    def draft_from_hidden(self, hidden: torch.Tensor, out: torch.Tensor | None = None,
                          logits: torch.Tensor | None = None) -> torch.Tensor:
        """Final RMSNorm + head + argmax + d2t in one launch chain, for one row of
        pre-norm hidden state (the drafter output is norm(hidden), python/woodcock/drafter.py:190);
        the normalised row is written to `out` when given."""
        h = _as_rows(hidden, self.cfg.hidden_size)
        if h.dtype != torch.float32 or h.shape[0] != 1:
            raise ValueError("hidden must be one float32 row")
        tok = torch.empty(1, dtype=torch.int32, device=self.device)
        _lib.call("wc_draft_head_norm", C.byref(self.dims), C.byref(self.wstruct), ptr(h), h.stride(0), None, 0,
                  ptr(out), 0 if out is None else out.stride(0), ptr(logits),
                  0 if logits is None else logits.stride(0), ptr(tok), None, None, ptr(self.ws), stream_ptr())
        return tok

    @property
    def vocab_ids(self) -> torch.Tensor | None:
        return self._vocab_ids

    def token_ids(self, rows: torch.Tensor) -> torch.Tensor:
        """Head row indices -> target token ids (drafter.py:213-215)."""
        return rows if self._vocab_ids is None else self._vocab_ids[rows.long()]

    def restrict_vocab(self, ids) -> None:
        """Keep only the head rows of `ids` (drafter.py:217-229): W[ids] gathered once,
        row r then drafts token ids[r]."""
        if self._vocab_ids is not None:
            raise ValueError("drafter vocabulary is already restricted")
        ids_t = torch.as_tensor(np.asarray(ids), dtype=torch.int64)
        if ids_t.dim() != 1 or ids_t.numel() == 0:
            raise ValueError("ids must be a non-empty 1-D list of token ids")
        if int(ids_t.min()) < 0 or int(ids_t.max()) >= self._head.shape[0]:
            raise ValueError("token id outside the head")
        self._head = self._head.index_select(0, ids_t.to(self.device)).contiguous()
        del self.w["lm_head.weight"]
        self._vocab_ids = ids_t.to(self.device, torch.int32)
        self._build_structs(self._rope[0].shape[0])

    def save(self, path, target_name: str | None = None) -> None:
        """config.json + model.safetensors + woodcock.json (drafter.py:310-319; export.py:27-53)."""
        if self._vocab_ids is not None:
            raise ValueError("a drafter with a restricted vocabulary cannot be saved")
        from .weights import write_drafter_dir

        write_drafter_dir(path, self.cfg, self.w, target_name)
