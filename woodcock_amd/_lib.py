"""ctypes binding of libwoodcock_hip.so (the C ABI in include/woodcock_hip.h).

Loading fails loudly: there is no CPU fallback anywhere in this package.
Status codes become exceptions: WC_E_INVALID -> ValueError (the reference
raises ValueError for bad arguments, python/woodcock/drafter.py:60-61,221-222),
anything else -> RuntimeError.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libwoodcock_hip.so"

WC_OK, WC_E_INVALID, WC_E_HIP, WC_E_UNSUPPORTED = 0, 1, 2, 3
WC_F32, WC_BF16 = 0, 1
WC_MAX_NODES = 64
WC_MAX_LAYERS = 64
ABI_VERSION = 2


class Verdict(C.Structure):
    """Mirror of wc_verdict (include/woodcock_hip.h)."""

    _fields_ = [
        ("n_accepted", C.c_int32),
        ("next", C.c_int32),
        ("n_keep", C.c_int32),
        ("n_uniforms", C.c_int32),
        ("status", C.c_int32),
        ("reserved", C.c_int32 * 3),
        ("tokens", C.c_int32 * (WC_MAX_NODES + 1)),
        ("keep", C.c_int32 * (WC_MAX_NODES + 1)),
    ]


VERDICT_BYTES = C.sizeof(Verdict)
VERDICT_INTS = VERDICT_BYTES // 4
# int32 offsets of the verdict fields, for device-side views
V_N_ACCEPTED, V_NEXT, V_N_KEEP, V_N_UNIFORMS, V_STATUS = 0, 1, 2, 3, 4
V_TOKENS = Verdict.tokens.offset // 4
V_KEEP = Verdict.keep.offset // 4

P = C.c_void_p
I32 = C.c_int32
I64 = C.c_int64

WC_MAX_DRAFTER_LAYERS = 4
WC_MAX_FEATURES = 3
WC_MAX_STEP_ROWS = 16


class DrafterDims(C.Structure):
    """Mirror of wc_drafter_dims."""

    _fields_ = [(n, C.c_int32) for n in ("hidden", "num_layers", "heads", "kv_heads", "head_dim", "inter",
                                          "target_hidden", "num_features", "head_rows", "vocab")] + \
               [("eps", C.c_float), ("window", C.c_int32)]


class LayerWeights(C.Structure):
    """Mirror of wc_layer_weights (device pointers)."""

    _fields_ = [(n, C.c_void_p) for n in ("in_norm", "post_norm", "aux_norm", "q", "k", "v", "o", "aux_q", "aux_k",
                                          "aux_v", "q_norm", "k_norm", "gate", "up", "down", "gate_frag", "up_frag")]


class DrafterWeights(C.Structure):
    """Mirror of wc_drafter_weights (device pointers)."""

    _fields_ = [("embed", C.c_void_p), ("fc", C.c_void_p), ("feature_norm", C.c_void_p * WC_MAX_FEATURES),
                ("final_norm", C.c_void_p), ("head", C.c_void_p), ("d2t", C.c_void_p), ("rope_cos", C.c_void_p),
                ("rope_sin", C.c_void_p), ("rope_max_pos", C.c_int32),
                ("layers", LayerWeights * WC_MAX_DRAFTER_LAYERS)]


class Gumbel(C.Structure):
    """Mirror of wc_gumbel."""

    _fields_ = [("seed", C.c_uint64), ("round_dev", C.c_void_p), ("purpose", C.c_int32), ("temperature", C.c_float)]

class Uniforms(C.Structure):
    """Mirror of wc_uniforms."""

    _fields_ = [("seed", C.c_uint64), ("round_dev", C.c_void_p), ("purpose", C.c_int32)]


_SIGS = {
    "wc_version": ([], C.c_int),
    "wc_last_error": ([], C.c_char_p),
    "wc_workspace_bytes": ([], C.c_size_t),
    "wc_workspace_init": ([P, C.c_size_t, P], C.c_int),
    "wc_set_spin_limit": ([C.c_int], C.c_int),
    "wc_argmax_rows": ([P, C.c_int, C.c_int, I64, P, P, P], C.c_int),
    "wc_verify_chain_greedy": ([P, C.c_int, C.c_int, I64, P, P, P, P], C.c_int),
    "wc_verify_chain_greedy_fuse": ([P, C.c_int, C.c_int, I64, P, P, P, P, P, P, C.c_int, I64, P, I64, P, P],
                                    C.c_int),
    "wc_verify_chain_greedy_static": ([P, C.c_int, C.c_int, I64, P, P, P], C.c_int),
    "wc_verify_tree_greedy": ([P, C.c_int, C.c_int, I64, P, P, P, P, P], C.c_int),
    "wc_kv_compact": ([P, P, C.c_int, C.c_int, C.c_int, C.c_int, P, P, P, C.c_int, P, P, P], C.c_int),
    "wc_rope_table": ([P, P, C.c_int, C.c_int, C.c_float], C.c_int),
    "wc_drafter_workspace_bytes": ([P], C.c_size_t),
    "wc_drafter_fuse": ([P, P, P, C.c_int, I64, P, C.c_int, C.c_int, P, P, I64, P, P], C.c_int),
    "wc_drafter_forward": ([P, P, P, P, I64, P, C.c_int, C.c_int, P, P, P, C.c_int, C.c_int, P, C.c_int, P, P, I64,
                            P, P, P, P, P], C.c_int),
    "wc_draft_head": ([P, P, P, I64, P, C.c_int, C.c_int, P, I64, P, P, P, P, P], C.c_int),
    "wc_probs_from_logits": ([P, C.c_int, C.c_int, I64, C.c_float, C.c_int, C.c_float, P, I64, P, P], C.c_int),
    "wc_verify_chain_stochastic": ([P, C.c_int, C.c_int, I64, P, C.c_int, I64, P, P, P, P, P, P, P], C.c_int),
    "wc_verify_chain_stochastic_logits": ([P, C.c_int, C.c_int, I64, C.c_float, P, C.c_int, I64, P, P, P, P, P, P,
                                           P], C.c_int),
    "wc_verify_tree_stochastic": ([P, C.c_int, C.c_int, I64, P, C.c_int, I64, P, P, P, P, P, P, P], C.c_int),
    "wc_verify_tree_stochastic_indexed": ([P, C.c_int, C.c_int, I64, P, C.c_int, P, C.c_int, I64, P, P, P, P, P, P,
                                           P, P], C.c_int),
    "wc_tree_mask": ([P, C.c_int, C.c_int, P, I64, P], C.c_int),
    "wc_sample_without_replacement": ([P, C.c_int, C.c_int, I64, P, P, C.c_int, P, I64, P, P, P], C.c_int),
    "wc_draft_head_norm": ([P, P, P, I64, P, C.c_int, P, I64, P, I64, P, P, P, P, P], C.c_int),
    "wc_draft_head_norm_pending": ([P, P, P, I64, P, C.c_int, P, I64, P, I64, P, P, P], C.c_int),
    "wc_drafter_forward_pending": ([P, P, P, P, P, I64, P, C.c_int, P, P, C.c_int, C.c_int, P, C.c_int, P, P, P, P,
                                    P, P], C.c_int),
    "wc_target_workspace_bytes": ([P, C.c_int], C.c_size_t),
    "wc_tree_draft_state_bytes": ([], C.c_size_t),
    "wc_tree_draft_begin": ([P, P, P], C.c_int),
    "wc_tree_draft_expand": ([P, P, C.c_int, C.c_int, I64, P, C.c_int, C.c_int, P], C.c_int),
    "wc_tree_draft_expand_logits": ([P, P, C.c_int, C.c_int, I64, P, C.c_int, C.c_int, P], C.c_int),
    "wc_tree_draft_frontier": ([P, C.c_int, C.c_int, C.c_int, P, C.c_int, C.c_int, C.c_int, P, P, P, P, I64, P],
                               C.c_int),
    "wc_tree_draft_select": ([P, C.c_int, C.c_int, P, P, P, P, P], C.c_int),
    "wc_tree_draft_expand_sample": ([P, P, C.c_int, C.c_int, I64, P, C.c_int, C.c_int, P, P], C.c_int),
    "wc_tree_draft_select_all": ([P, C.c_int, P, P, P, P, P, P], C.c_int),
    "wc_weights_frag": ([P, C.c_int, C.c_int, P, P], C.c_int),
    "wc_target_embed": ([P, C.c_int, C.c_int, P, C.c_int, P, I64, P], C.c_int),
    "wc_target_head": ([P, P, P, P, C.c_int, C.c_int, P, I64, C.c_int, P, P], C.c_int),
    "wc_target_layer": ([P, P, P, P, C.c_int, P, C.c_int, P, P, I64, P, P, C.c_int, C.c_int, P, P, C.c_int, P, P],
                        C.c_int),
    "wc_rmsnorm": ([P, P, C.c_int, C.c_int, P, C.c_int, C.c_float, P], C.c_int),
    "wc_linear": ([P, C.c_int, C.c_int, P, C.c_int, C.c_int, P, C.c_int, P], C.c_int),
    "wc_rope": ([P, C.c_int, C.c_int, C.c_int, P, C.c_float, P, P, C.c_int, P], C.c_int),
    "wc_silu_mul": ([P, P, I64, P], C.c_int),
    "wc_attention": ([P, C.c_int, C.c_int, C.c_int, C.c_int, P, P, C.c_int, P, P, C.c_float, P], C.c_int),
    "wc_softmax": ([P, C.c_int, C.c_int, P], C.c_int),
    "wc_kv_append": ([P, P, C.c_int, C.c_int, P, P, C.c_int, P, P, P], C.c_int),
    "wc_kv_set_offset": ([P, C.c_int, P], C.c_int),
}

_lib = None


class WoodcockHipError(RuntimeError):
    pass


def lib() -> C.CDLL:
    """The loaded library; raises if it is missing or was built for another ABI."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise WoodcockHipError(
                f"{LIB_PATH} is missing: build it with `python -m woodcock_amd.build` (hipcc, gfx950)")
        handle = C.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | os.RTLD_LOCAL)
        for name, (args, res) in _SIGS.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = res
        v = handle.wc_version()
        if v != ABI_VERSION:
            raise WoodcockHipError(f"{LIB_PATH} has ABI {v}, expected {ABI_VERSION}: rebuild it")
        _lib = handle
    return _lib


def exported_symbols() -> list[str]:
    return list(_SIGS)


def check(status: int) -> None:
    if status == WC_OK:
        return
    msg = lib().wc_last_error().decode(errors="replace")
    if status == WC_E_INVALID:
        raise ValueError(msg)
    raise WoodcockHipError(f"status {status}: {msg}")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))


def stream_handle(stream=None) -> int | None:
    """hipStream_t of a torch stream (default: the current stream of the current device)."""
    import torch

    s = torch.cuda.current_stream() if stream is None else stream
    return s.cuda_stream or None
