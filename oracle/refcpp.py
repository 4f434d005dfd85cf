"""ctypes wrapper of ``oracle/_ref/libwcref.so`` -- the reference's own C++ runtime.

TEST INFRASTRUCTURE ONLY.  The library is compiled by oracle/Makefile from the
reference's sources where they lie (never copied into this repository) plus
``ref_driver.cpp``.  It is built only where the reference checkout exists; tests
that need it skip when it is absent.  It is fp32 throughout and loads bf16
safetensors by widening them (src/core/weights.cpp:100-122).
"""
from __future__ import annotations

import ctypes as C
import json
import tempfile
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_ref" / "libwcref.so"
# the same runtime with woodcock_amd/backends/hip_ops.cpp in its backend slot
HIP_LIB_PATH = HERE / "_ref" / "libwcref_hip.so"

_libs: dict[str, C.CDLL] = {}
P = C.c_void_p


def available(path: Path = LIB_PATH) -> bool:
    return Path(path).exists()


def lib(path: Path | None = None):
    key = str(LIB_PATH if path is None else path)
    if key not in _libs:
        L = C.CDLL(key)
        L.wcref_last_error.restype = C.c_char_p
        L.wcref_drafter_open.argtypes = [C.c_char_p, C.POINTER(C.c_void_p)]
        L.wcref_drafter_close.argtypes = [P]
        L.wcref_drafter_cache_new.argtypes = [P, C.POINTER(C.c_void_p)]
        L.wcref_drafter_fuse.argtypes = [P, P, C.c_int, C.c_int, P]
        L.wcref_drafter_forward.argtypes = [P, P, C.c_int, P, P, P, P, P, P]
        L.wcref_drafter_logits.argtypes = [P, P, P]
        L.wcref_cache_new.argtypes = [C.c_int, C.c_int, C.c_int, C.POINTER(C.c_void_p)]
        L.wcref_cache_free.argtypes = [P]
        L.wcref_cache_size.argtypes = [P]
        L.wcref_cache_append.argtypes = [P, C.c_int, P, P, C.c_int]
        L.wcref_cache_commit.argtypes = [P, C.c_int]
        L.wcref_cache_trim_to.argtypes = [P, C.c_int]
        L.wcref_cache_compact.argtypes = [P, C.c_int, P, C.c_int]
        L.wcref_cache_rows.argtypes = [P, C.c_int, C.c_int, C.c_int, P]
        L.wcref_argmax.argtypes = [P, C.c_int]
        L.wcref_probs_from_logits.argtypes = [P, C.c_int, C.c_float, C.c_int, C.c_float, P]
        L.wcref_verify_tree_greedy.argtypes = [P, P, P, P, C.c_int, P, P, P]
        L.wcref_tree_mask.argtypes = [P, P, P, C.c_int, C.c_int, P]
        L.wcref_causal_mask.argtypes = [C.c_int, C.c_int, C.c_int, P]
        L.wcref_rmsnorm.argtypes = [P, P, C.c_int, C.c_int, P, C.c_float]
        L.wcref_rope.argtypes = [P, C.c_int, C.c_int, C.c_int, P, C.c_float]
        L.wcref_softmax.argtypes = [P, C.c_int]
        L.wcref_attention.argtypes = [P, C.c_int, C.c_int, C.c_int, C.c_int, P, P, C.c_int, P, P, C.c_float]
        L.wcref_linear.argtypes = [P, C.c_int, C.c_int, P, C.c_int, P, C.c_int]
        L.wcref_silu_mul.argtypes = [P, P, C.c_int64]
        L.wcref_qwen3_open.argtypes = [C.c_char_p, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_void_p)]
        L.wcref_qwen3_close.argtypes = [P]
        L.wcref_qwen3_cache_new.argtypes = [P, C.POINTER(C.c_void_p)]
        L.wcref_qwen3_forward.argtypes = [P, P, C.c_int, P, P, P, P, P]
        _libs[key] = L
    return _libs[key]


def _check(rc: int, L=None) -> None:
    if rc != 0:
        raise RuntimeError((L or lib()).wcref_last_error().decode())


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _i32(a):
    return np.ascontiguousarray(a, dtype=np.int32)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ------------------------------------------------------------------ drafter files

def write_drafter_dir(path: Path, cfg: dict, weights: dict[str, np.ndarray]) -> None:
    """config.json + bf16 model.safetensors in the reference's drafter format
    (python/woodcock/drafter.py:310-319; src/core/drafter.cpp:18-73)."""
    import torch
    from safetensors.torch import save_file

    path.mkdir(parents=True, exist_ok=True)
    (path / "config.json").write_text(json.dumps(cfg, indent=2))
    tensors = {k: torch.from_numpy(np.ascontiguousarray(v, dtype=np.uint16).view(np.int16)).view(torch.bfloat16)
               for k, v in weights.items()}
    save_file(tensors, str(path / "model.safetensors"), metadata={"format": "woodcock-drafter-v1"})


class RefDrafter:
    """The reference C++ Drafter (include/woodcock/drafter.h:48-58) over a temp dir."""

    def __init__(self, cfg: dict, weights: dict[str, np.ndarray], lib_path: Path | None = None):
        self.cfg = cfg
        self.L = lib(lib_path)
        self._tmp = tempfile.TemporaryDirectory()
        write_drafter_dir(Path(self._tmp.name), cfg, weights)
        h = C.c_void_p()
        _check(self.L.wcref_drafter_open(self._tmp.name.encode(), C.byref(h)), self.L)
        self.h = h
        self.head_rows = weights["lm_head.weight"].shape[0]

    def close(self):
        if self.h:
            self.L.wcref_drafter_close(self.h)
            self.h = None
        self._tmp.cleanup()

    def __del__(self):  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass

    def make_cache(self) -> "RefCache":
        h = C.c_void_p()
        _check(self.L.wcref_drafter_cache_new(self.h, C.byref(h)), self.L)
        return RefCache(h, self.cfg["num_layers"], self.cfg["num_kv_heads"] * self.cfg["head_dim"], self.L)

    def fuse(self, taps) -> np.ndarray:
        ts = [_f32(t).reshape(-1, self.cfg["target_hidden_size"]) for t in taps]
        L = ts[0].shape[0]
        arr = (C.c_void_p * len(ts))(*[t.ctypes.data for t in ts])
        g = np.empty((L, self.cfg["hidden_size"]), dtype=np.float32)
        _check(self.L.wcref_drafter_fuse(self.h, arr, len(ts), L, _p(g)), self.L)
        return g

    def forward(self, tokens, feat, cache: "RefCache", positions=None, mask=None):
        tok = _i32(tokens).reshape(-1)
        L = tok.size
        f = _f32(feat).reshape(L, self.cfg["hidden_size"])
        pos = None if positions is None else _i32(positions).reshape(-1)
        m = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint8)
        hid = np.empty_like(f)
        out = np.empty_like(f)
        _check(self.L.wcref_drafter_forward(self.h, _p(tok), L, _p(f), cache.h, _p(pos), _p(m), _p(hid), _p(out)), self.L)
        return hid, out

    def logits(self, out) -> np.ndarray:
        o = _f32(out).reshape(-1, self.cfg["hidden_size"])
        z = np.empty((o.shape[0], self.cfg["vocab_size"]), dtype=np.float32)
        for r in range(o.shape[0]):
            row = np.ascontiguousarray(o[r])
            _check(self.L.wcref_drafter_logits(self.h, _p(row), _p(z[r])), self.L)
        return z[:, : self.head_rows]


class RefCache:
    """The reference KVCache (include/woodcock/cache.h:9-28): [T][kv_heads*head_dim] fp32 per layer."""

    def __init__(self, h, layers: int, row: int, L=None):
        self.h, self.layers, self.row = h, layers, row
        self.L = L or lib()

    @classmethod
    def new(cls, layers: int, kv_heads: int, head_dim: int, lib_path: Path | None = None) -> "RefCache":
        L = lib(lib_path)
        h = C.c_void_p()
        _check(L.wcref_cache_new(layers, kv_heads, head_dim, C.byref(h)), L)
        return cls(h, layers, kv_heads * head_dim, L)

    def __del__(self):  # pragma: no cover
        try:
            if self.h:
                self.L.wcref_cache_free(self.h)
        except Exception:
            pass

    @property
    def size(self) -> int:
        return int(self.L.wcref_cache_size(self.h))

    @property
    def offset(self) -> int:
        return self.size

    @offset.setter
    def offset(self, n: int) -> None:
        self.trim_to(n)

    def append(self, layer: int, k, v, L: int):
        _check(self.L.wcref_cache_append(self.h, layer, _p(_f32(k)), _p(_f32(v)), L), self.L)

    def commit(self, L: int):
        self.L.wcref_cache_commit(self.h, L)

    def trim_to(self, n: int):
        self.L.wcref_cache_trim_to(self.h, n)

    def compact(self, start: int, keep):
        k = _i32(keep)
        _check(self.L.wcref_cache_compact(self.h, start, _p(k), k.size), self.L)

    def rows(self, layer: int, which: int, n: int | None = None) -> np.ndarray:
        n = self.size if n is None else n
        out = np.empty((n, self.row), dtype=np.float32)
        _check(self.L.wcref_cache_rows(self.h, layer, which, n, _p(out)), self.L)
        return out


class RefQwen3:
    """The reference C++ Qwen3 target (include/woodcock/model.h:19-48) over a temp
    dir holding config.json + model.safetensors under the Hugging Face names
    (src/core/qwen3.cpp:22-83).  cfg: target.TargetConfig-like; weights: our
    names (``layers.{i}.*``, ``embed_tokens.weight``, ``norm.weight``) -> bf16 bits."""

    def __init__(self, cfg, weights: dict[str, np.ndarray], taps=(-1, -1, -1)):
        import torch
        from safetensors.torch import save_file

        self.cfg = cfg
        self._tmp = tempfile.TemporaryDirectory()
        path = Path(self._tmp.name)
        (path / "config.json").write_text(json.dumps({
            "hidden_size": cfg.hidden_size, "num_hidden_layers": cfg.num_layers,
            "num_attention_heads": cfg.num_heads, "num_key_value_heads": cfg.num_kv_heads,
            "head_dim": cfg.head_dim, "intermediate_size": cfg.intermediate_size, "vocab_size": cfg.vocab_size,
            "rms_norm_eps": cfg.rms_norm_eps, "rope_theta": cfg.rope_theta,
            "tie_word_embeddings": cfg.tie_word_embeddings}))
        tensors = {"model." + k: torch.from_numpy(np.ascontiguousarray(v, dtype=np.uint16).view(np.int16))
                   .view(torch.bfloat16) for k, v in weights.items()}
        save_file(tensors, str(path / "model.safetensors"))
        h = C.c_void_p()
        _check(lib().wcref_qwen3_open(str(path).encode(), *[int(t) for t in taps], C.byref(h)))
        self.h = h
        self.n_taps = 3

    def close(self):
        if self.h:
            lib().wcref_qwen3_close(self.h)
            self.h = None
        self._tmp.cleanup()

    def __del__(self):  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass

    def make_cache(self) -> RefCache:
        h = C.c_void_p()
        _check(lib().wcref_qwen3_cache_new(self.h, C.byref(h)))
        return RefCache(h, self.cfg.num_layers, self.cfg.num_kv_heads * self.cfg.head_dim)

    def forward(self, tokens, cache: RefCache, positions=None, mask=None):
        """-> (logits [L, vocab], taps [3, L, hidden]); the cache grows by L."""
        tok = _i32(tokens).reshape(-1)
        L = tok.size
        pos = None if positions is None else _i32(positions).reshape(-1)
        m = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint8)
        logits = np.empty((L, self.cfg.vocab_size), np.float32)
        taps = np.empty((3, L, self.cfg.hidden_size), np.float32)
        _check(lib().wcref_qwen3_forward(self.h, _p(tok), L, cache.h, _p(pos), _p(m), _p(logits), _p(taps)))
        return logits, taps


def linear(x, W, y=None, accumulate: bool = False) -> np.ndarray:
    x, W = _f32(x), _f32(W)
    L = x.size // W.shape[1]
    y = np.zeros((L, W.shape[0]), np.float32) if y is None else _f32(y).copy()
    _check(lib().wcref_linear(_p(x), L, W.shape[1], _p(W), W.shape[0], _p(y), int(accumulate)))
    return y


def silu_mul(gate, up) -> np.ndarray:
    g = _f32(gate).copy()
    _check(lib().wcref_silu_mul(_p(g), _p(_f32(up)), g.size))
    return g


def rmsnorm(x, w, eps: float) -> np.ndarray:
    x = _f32(x)
    d = x.shape[-1]
    y = np.empty_like(x)
    _check(lib().wcref_rmsnorm(_p(x), _p(y), x.size // d, d, _p(_f32(w)), eps))
    return y


def rope(x, positions, base: float) -> np.ndarray:
    """x [L, heads, D] -> rotated copy."""
    y = _f32(x).copy()
    L, heads, D = y.shape
    _check(lib().wcref_rope(_p(y), L, heads, D, _p(_i32(positions)), base))
    return y


def softmax(x) -> np.ndarray:
    y = _f32(x).copy()
    _check(lib().wcref_softmax(_p(y), y.size))
    return y


def attention(q, K, V, mask, scale: float) -> np.ndarray:
    """q [L, H, D]; K, V [T, Hk, D]; mask [L, T] or None."""
    q, K, V = _f32(q), _f32(K), _f32(V)
    L, H, D = q.shape
    T, Hk, _ = K.shape
    m = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint8)
    out = np.empty_like(q)
    _check(lib().wcref_attention(_p(q), L, H, Hk, D, _p(K), _p(V), T, _p(m), _p(out), scale))
    return out


# ------------------------------------------------------------------ sampling / masks

def argmax(z) -> int:
    z = _f32(z)
    return int(lib().wcref_argmax(_p(z), z.size))


def probs_from_logits(z, temperature: float, top_k: int = 0, top_p: float = 1.0) -> np.ndarray:
    z = _f32(z)
    p = np.empty_like(z)
    _check(lib().wcref_probs_from_logits(_p(z), z.size, temperature, top_k, top_p, _p(p)))
    return p


def verify_tree_greedy(am, tokens, parents, depth):
    N = len(tokens)
    path = np.zeros(max(N, 1), dtype=np.int32)
    n_path, nxt = C.c_int(), C.c_int()
    _check(lib().wcref_verify_tree_greedy(_p(_i32(am)), _p(_i32(tokens)), _p(_i32(parents)), _p(_i32(depth)), N,
                                          _p(path), C.byref(n_path), C.byref(nxt)))
    return path[: n_path.value].tolist(), nxt.value


def tree_mask(tokens, parents, depth, prefix: int) -> np.ndarray:
    N = len(tokens)
    m = np.zeros((N, prefix + N), dtype=np.uint8)
    _check(lib().wcref_tree_mask(_p(_i32(tokens)), _p(_i32(parents)), _p(_i32(depth)), N, prefix, _p(m)))
    return m.astype(bool)


def causal_mask(prefix: int, L: int, window: int = 0) -> np.ndarray:
    m = np.zeros((L, prefix + L), dtype=np.uint8)
    _check(lib().wcref_causal_mask(prefix, L, window, _p(m)))
    return m.astype(bool)
