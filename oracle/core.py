"""ctypes wrapper of the C restatement ``oracle/wc_oracle.c`` (test infrastructure only).

The drafter restatement follows src/core/drafter.cpp:75-141 and
python/woodcock/drafter.py:149-229 with bf16 weights widened to fp32 and an
optional bf16 KV cache; see the header of wc_oracle.c for every citation.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_lib = None


def build(force: bool = False) -> None:
    """Compile liboracle.so (and _ref/libwcref.so where the reference exists)."""
    if force or not LIB_PATH.exists():
        subprocess.run(["make", "-s", "-C", str(HERE), "all"] + (["-B"] if force else []), check=True)


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = C.CDLL(str(LIB_PATH))
        _declare(_lib)
    return _lib


P = C.c_void_p


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _declare(L):
    L.or_philox4x64_10.argtypes = [P, P, P]
    L.or_uniforms.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint64, C.c_int64, P]
    L.or_rmsnorm.argtypes = [P, P, C.c_int, C.c_int, P, C.c_float]
    L.or_rope_table.argtypes = [P, P, C.c_int, C.c_int, C.c_float]
    L.or_linear.argtypes = [P, C.c_int, C.c_int, P, C.c_int, P, C.c_int]
    L.or_attention.argtypes = [P, C.c_int, C.c_int, C.c_int, C.c_int, P, P, C.c_int, C.c_int, C.c_int, P, P,
                               C.c_float]
    L.or_drafter_fuse.argtypes = [P, P, P, C.c_int, P]
    L.or_drafter_forward.argtypes = [P, P, P, C.c_int, P, P, P, C.c_int, C.c_int, C.c_int, P, P, P, P, P, P]
    L.or_drafter_forward.restype = C.c_int
    L.or_head_logits.argtypes = [P, P, P, C.c_int, P]
    L.or_argmax.argtypes = [P, C.c_int]
    L.or_argmax.restype = C.c_int
    L.or_kv_compact.argtypes = [P, P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, P, C.c_int]
    L.or_f32_to_bf16.argtypes = [P, P, C.c_int64]
    L.or_set_threads.argtypes = [C.c_int]
    L.or_get_threads.restype = C.c_int


def set_threads(n: int) -> None:
    lib().or_set_threads(int(n))


def get_threads() -> int:
    return int(lib().or_get_threads())


# ------------------------------------------------------------------ bf16 helpers

def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns (round to nearest even), as uint16."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().or_f32_to_bf16(_ptr(x), _ptr(out), x.size)
    return out


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ------------------------------------------------------------------ Philox4x64-10

def philox4x64_10(ctr, key) -> np.ndarray:
    c = np.ascontiguousarray(ctr, dtype=np.uint64)
    k = np.ascontiguousarray(key, dtype=np.uint64)
    out = np.empty(4, dtype=np.uint64)
    lib().or_philox4x64_10(_ptr(c), _ptr(k), _ptr(out))
    return out


def uniforms(seed: int, round_: int, purpose: int, start: int, n: int) -> np.ndarray:
    """Uniforms start..start+n-1 of stream (round, purpose) under seed, as float64 in [0, 1)."""
    out = np.empty(n, dtype=np.float64)
    lib().or_uniforms(seed, round_, purpose, start, n, _ptr(out))
    return out


class UniformStream:
    """np.random.Generator look-alike whose ``random()`` walks one Philox stream.

    Lets the numpy restatement of the verification rules consume uniforms in
    exactly the reference order (sampling.py:79,165,193,201) while the values
    come from the counter-based stream the HIP kernels use."""

    def __init__(self, seed: int, round_: int, purpose: int = 0, start: int = 0):
        self.seed, self.round, self.purpose, self.pos = seed, round_, purpose, start

    def random(self, size=None):
        n = 1 if size is None else int(np.prod(size))
        u = uniforms(self.seed, self.round, self.purpose, self.pos, n)
        self.pos += n
        return float(u[0]) if size is None else u.reshape(size)


# ------------------------------------------------------------------ basic ops

def rmsnorm(x: np.ndarray, w_bf16: np.ndarray | None, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    d = x.shape[-1]
    y = np.empty_like(x)
    w = None if w_bf16 is None else np.ascontiguousarray(w_bf16, dtype=np.uint16)
    lib().or_rmsnorm(_ptr(x), _ptr(y), x.size // d, d, _ptr(w), eps)
    return y


def rope_table(max_pos: int, head_dim: int, base: float) -> tuple[np.ndarray, np.ndarray]:
    c = np.empty((max_pos, head_dim // 2), dtype=np.float32)
    s = np.empty_like(c)
    lib().or_rope_table(_ptr(c), _ptr(s), max_pos, head_dim, base)
    return c, s


def linear(x: np.ndarray, w_bf16: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w_bf16, dtype=np.uint16)
    L, din = x.reshape(-1, x.shape[-1]).shape
    y = np.empty((L, w.shape[0]), dtype=np.float32)
    lib().or_linear(_ptr(x), L, din, _ptr(w), w.shape[0], _ptr(y), 0)
    return y


def argmax(z: np.ndarray) -> int:
    z = np.ascontiguousarray(z, dtype=np.float32)
    return int(lib().or_argmax(_ptr(z), z.size))


# ------------------------------------------------------------------ drafter

class _Dims(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("hidden", "num_layers", "heads", "kv_heads", "head_dim", "inter",
                                        "target_hidden", "num_features", "head_rows", "vocab")] + \
               [("eps", C.c_float), ("rope_theta", C.c_float)] + \
               [(n, C.c_int) for n in ("post_norm", "feature_norm", "window")]


_LAYER_FIELDS = ("in_norm", "aux_norm", "post_norm", "q", "k", "v", "o", "aux_q", "aux_k", "aux_v", "q_norm",
                 "k_norm", "gate", "up", "down")


class _LayerW(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in _LAYER_FIELDS]


class _Weights(C.Structure):
    _fields_ = [("embed", C.c_void_p), ("fc", C.c_void_p), ("fnorm", C.c_void_p * 8), ("final_norm", C.c_void_p),
                ("head", C.c_void_p), ("layers", C.POINTER(_LayerW))]


# reference parameter names (python/woodcock/drafter.py:66-142; src/core/drafter.cpp:47-73)
LAYER_NAMES = {
    "in_norm": "input_layernorm.weight",
    "aux_norm": "aux_norm.weight",
    "post_norm": "post_attention_layernorm.weight",
    "q": "self_attn.q_proj.weight",
    "k": "self_attn.k_proj.weight",
    "v": "self_attn.v_proj.weight",
    "o": "self_attn.o_proj.weight",
    "aux_q": "self_attn.aux_q.weight",
    "aux_k": "self_attn.aux_k.weight",
    "aux_v": "self_attn.aux_v.weight",
    "q_norm": "self_attn.q_norm.weight",
    "k_norm": "self_attn.k_norm.weight",
    "gate": "mlp.gate_proj.weight",
    "up": "mlp.up_proj.weight",
    "down": "mlp.down_proj.weight",
}


class Drafter:
    """fp32 drafter oracle over bf16 weights.

    cfg: DrafterConfig fields as a dict (drafter.py:33-49).
    weights: reference parameter name -> uint16 bf16 bit array.
    head: rows of lm_head to use (the restricted head, drafter.py:217-229);
    d2t: head row -> token id (None = identity).
    """

    def __init__(self, cfg: dict, weights: dict[str, np.ndarray], d2t: np.ndarray | None = None):
        self.cfg = dict(cfg)
        self.w = {k: np.ascontiguousarray(v, dtype=np.uint16) for k, v in weights.items()}
        self.d2t = None if d2t is None else np.ascontiguousarray(d2t, dtype=np.int32)
        head = self.w["lm_head.weight"]
        if self.d2t is not None and head.shape[0] != len(self.d2t):
            head = np.ascontiguousarray(head[self.d2t])
        self.head = head
        c = self.cfg
        self.dims = _Dims(c["hidden_size"], c["num_layers"], c["num_heads"], c["num_kv_heads"], c["head_dim"],
                          c["intermediate_size"], c["target_hidden_size"], c.get("num_features", 3),
                          head.shape[0], c["vocab_size"], c.get("rms_norm_eps", 1e-6),
                          c.get("rope_theta", 1e6), int(c.get("post_norm", True)),
                          int(c.get("feature_norm", True)), int(c.get("window") or 0))
        nl = c["num_layers"]
        self._layers = (_LayerW * nl)()
        for i in range(nl):
            for f in _LAYER_FIELDS:
                a = self.w.get(f"layers.{i}.{LAYER_NAMES[f]}")
                setattr(self._layers[i], f, None if a is None else a.ctypes.data)
        self._wt = _Weights()
        self._wt.embed = self.w["embed_tokens.weight"].ctypes.data
        self._wt.fc = self.w["fc.weight"].ctypes.data
        for i in range(self.dims.num_features):
            a = self.w.get(f"feature_norms.{i}.weight")
            self._wt.fnorm[i] = None if a is None else a.ctypes.data
        self._wt.final_norm = self.w["norm.weight"].ctypes.data
        self._wt.head = self.head.ctypes.data
        self._wt.layers = self._layers
        self._rope = None

    def rope_table(self, max_pos: int):
        if self._rope is None or self._rope[0].shape[0] < max_pos:
            self._rope = rope_table(max_pos, self.cfg["head_dim"], self.cfg.get("rope_theta", 1e6))
        return self._rope

    def fuse(self, taps: list[np.ndarray]) -> np.ndarray:
        """taps: num_features arrays [L][target_hidden] -> g [L][hidden] (drafter.cpp:75-89)."""
        ts = [np.ascontiguousarray(t, dtype=np.float32).reshape(-1, self.dims.target_hidden) for t in taps]
        L = ts[0].shape[0]
        arr = (C.c_void_p * len(ts))(*[t.ctypes.data for t in ts])
        g = np.empty((L, self.dims.hidden), dtype=np.float32)
        lib().or_drafter_fuse(C.byref(self.dims), C.byref(self._wt), arr, L, _ptr(g))
        return g

    def make_cache(self, cap: int, kv_bf16: bool = False) -> "Cache":
        return Cache(self.dims.num_layers, self.dims.kv_heads, cap, self.dims.head_dim, kv_bf16)

    def forward(self, tokens, feat, cache: "Cache", positions=None, mask=None):
        """One drafting forward at cache.offset; returns (hidden, out) [L][hidden]
        and advances cache.offset by L (drafter.cpp:91-136)."""
        tok = np.ascontiguousarray(tokens, dtype=np.int32).reshape(-1)
        L = tok.size
        f = np.ascontiguousarray(feat, dtype=np.float32).reshape(L, self.dims.hidden)
        pos = None if positions is None else np.ascontiguousarray(positions, dtype=np.int32).reshape(-1)
        m = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint8).reshape(L, cache.offset + L)
        max_pos = int(max(cache.offset + L, 0 if pos is None else pos.max() + 1)) + 1
        rc, rs = self.rope_table(max(max_pos, cache.cap + 1))
        hid = np.empty((L, self.dims.hidden), dtype=np.float32)
        out = np.empty_like(hid)
        kp = (C.c_void_p * self.dims.num_layers)(*[a.ctypes.data for a in cache.k])
        vp = (C.c_void_p * self.dims.num_layers)(*[a.ctypes.data for a in cache.v])
        rc_ = lib().or_drafter_forward(C.byref(self.dims), C.byref(self._wt), _ptr(tok), L, _ptr(f), kp, vp,
                                       int(cache.bf16), cache.cap, cache.offset, _ptr(pos), _ptr(m), _ptr(rc),
                                       _ptr(rs), _ptr(hid), _ptr(out))
        if rc_ != 0:
            raise ValueError("drafter cache capacity exceeded")
        cache.offset += L
        return hid, out

    def feedback(self, hidden, out):
        return out if self.cfg.get("post_norm", True) else hidden

    def logits(self, out) -> np.ndarray:
        o = np.ascontiguousarray(out, dtype=np.float32).reshape(-1, self.dims.hidden)
        z = np.empty((o.shape[0], self.dims.head_rows), dtype=np.float32)
        lib().or_head_logits(C.byref(self.dims), C.byref(self._wt), _ptr(o), o.shape[0], _ptr(z))
        return z

    def token_ids(self, rows):
        rows = np.asarray(rows)
        return rows if self.d2t is None else self.d2t[rows]


class Cache:
    """Per-layer K/V, layout [kv_heads][cap][head_dim], fp32 or bf16 bits."""

    def __init__(self, layers: int, kv_heads: int, cap: int, head_dim: int, bf16: bool):
        dt = np.uint16 if bf16 else np.float32
        self.k = [np.zeros((kv_heads, cap, head_dim), dtype=dt) for _ in range(layers)]
        self.v = [np.zeros((kv_heads, cap, head_dim), dtype=dt) for _ in range(layers)]
        self.cap, self.bf16, self.offset = cap, bf16, 0

    def keys_f32(self, layer: int) -> np.ndarray:
        return bf16_to_f32(self.k[layer]) if self.bf16 else self.k[layer]

    def values_f32(self, layer: int) -> np.ndarray:
        return bf16_to_f32(self.v[layer]) if self.bf16 else self.v[layer]


# ------------------------------------------------------------------ KV compaction

def kv_compact(k_layers: list[np.ndarray], v_layers: list[np.ndarray], start: int, keep) -> None:
    """In-place compaction of [kv_heads][cap][...] caches (target.py:159-175)."""
    keep = np.ascontiguousarray(keep, dtype=np.int32)
    kv_heads, cap = k_layers[0].shape[:2]
    row_bytes = k_layers[0][0, 0].nbytes
    kp = (C.c_void_p * len(k_layers))(*[a.ctypes.data for a in k_layers])
    vp = (C.c_void_p * len(v_layers))(*[a.ctypes.data for a in v_layers])
    lib().or_kv_compact(kp, vp, len(k_layers), kv_heads, cap, row_bytes, start, _ptr(keep), keep.size)


def default_threads() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1
