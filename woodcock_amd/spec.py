"""The fused greedy chain round with ONE host synchronisation
(python/woodcock/spec.py:331-374, _fused_chain_round + _update).

Everything between two host reads stays on the device:

    head(RMSNorm(root)) -> d_1                          (final norm + draft head + argmax + d2t)
    for k in 1..K-1: drafter layer(d_k, fb) -> head(RMSNorm(h)) -> d_{k+1}
    target logits at [x_n, d_1..d_K]                    (supplied by the target; out of scope here)
    fused target argmax + greedy accept -> verdict      (a, accepted tokens + next, keep)
    compact the target KV with keep (identity for a chain: offset only)
    update: fuse(taps[keep]) and one drafter pass over the a+1 accepted tokens,
            which appends them to the drafter cache and yields the next root
    copy the verdict to pinned host memory              <- the round's single sync

Round-varying integers -- the committed count n (drafter base == target
start), the accepted count, the gathered rows -- are read from device memory,
so the same kernel sequence (or one captured HIP graph) serves every round.

State invariants follow python/woodcock/spec.py:1-15: before a round the
drafter cache holds real entries 0..n-1 and the root is the drafter's hidden
state of entry n-1 (row n_keep-1 of the previous update); its output, the final
RMSNorm of it, is formed by the head launch that consumes it, so no drafter
pass of the round runs a norm of its own on the critical path.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import torch

from . import _lib
from .cache import KVCache, compact_cache_dev
from .drafter import Drafter
from .runtime import new_verdict, ptr, read_verdict, stream_ptr

# state vector slots (device int32)
S_N, S_ROUND, S_TARGET_OFFSET = 0, 1, 2


@dataclass
class RoundResult:
    n_accepted: int
    tokens: list[int]  # accepted drafts + the target's next token


class ChainRound:
    """Device state and buffers of a greedy chain of length K (<= 15).

    target: object with ``logits`` [K+1, V] fp32 and ``taps`` (num_features
    tensors [K+1, target_hidden]) device tensors at [x_n, d_1..d_K] -- the
    verify-width target forward, which this module does not implement."""

    def __init__(self, drafter: Drafter, k: int, capacity: int, target_cache: list[KVCache] | None = None):
        if not 1 <= k <= _lib.WC_MAX_STEP_ROWS - 1:
            raise ValueError(f"chain length must be in 1..{_lib.WC_MAX_STEP_ROWS - 1}")
        self.d = drafter
        self.K = k
        dev = drafter.device
        dm = drafter.cfg.hidden_size
        self.cache = drafter.make_cache(capacity)
        self.target_cache = target_cache
        self.state = torch.zeros(8, dtype=torch.int32, device=dev)
        self.verdict = new_verdict(dev)
        self.drafts = torch.zeros(k, dtype=torch.int32, device=dev)
        self.step_hid = torch.zeros(max(k - 1, 1), dm, dtype=torch.float32, device=dev)
        self.step_out = torch.zeros_like(self.step_hid)
        self.upd_hid = torch.zeros(k + 1, dm, dtype=torch.float32, device=dev)
        self.upd_out = torch.zeros_like(self.upd_hid)
        self.g = torch.zeros_like(self.upd_hid)
        self.host_verdict = torch.zeros(_lib.VERDICT_INTS, dtype=torch.int32, pin_memory=True)
        n = int(_lib.lib().wc_workspace_bytes())
        self.vws = torch.empty((n + 255) // 256 * 256, dtype=torch.uint8, device=dev)
        _lib.call("wc_workspace_init", ptr(self.vws), self.vws.numel(), stream_ptr())
        self.syncs = 0
        self._kp = (C.c_void_p * len(self.cache))(*[c.keys.data_ptr() for c in self.cache])
        self._vp = (C.c_void_p * len(self.cache))(*[c.values.data_ptr() for c in self.cache])
        self._kvdt = _lib.WC_BF16 if self.cache[0].keys.dtype == torch.bfloat16 else _lib.WC_F32

    # ------------------------------------------------------------------ state

    def set_root(self, n: int, root_hidden: torch.Tensor) -> None:
        """Start state: n committed entries in the drafter cache and the root --
        the drafter's pre-norm hidden state of entry n-1 (its output, the final
        RMSNorm of it, is formed by the first head launch of the round)."""
        self.upd_hid[0].copy_(root_hidden.reshape(-1))
        self.verdict.zero_()
        self.verdict[_lib.V_N_KEEP] = 1
        self.state.zero_()
        self.state[S_N] = n
        self.state[S_TARGET_OFFSET] = n
        for c in self.cache:
            c.offset = n

    def _fb_rows(self, hid: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
        return out if self.d.cfg.post_norm else hid

    # ------------------------------------------------------------------ enqueue

    def enqueue_draft(self) -> None:
        """K head launches and K-1 drafter layers from the root; drafts -> self.drafts."""
        d = self.d
        dims, W, ws, s = C.byref(d.dims), C.byref(d.wstruct), ptr(d.ws), stream_ptr()
        n_keep = ptr(self.verdict[_lib.V_N_KEEP:_lib.V_N_KEEP + 1])
        dm = d.cfg.hidden_size
        cap = self.cache[0].capacity
        # d_1 from the root = update row n_keep - 1; the head applies the final
        # RMSNorm and leaves the root's output in upd_out (same row)
        _lib.call("wc_draft_head_norm", dims, W, ptr(self.upd_hid), dm, n_keep, -1, ptr(self.upd_out), dm, None, 0,
                  ptr(self.drafts[0:1]), None, None, ws, s)
        root_fb = self._fb_rows(self.upd_hid, self.upd_out)
        for k in range(1, self.K):
            if k == 1:
                feat, frow, fadd = root_fb, n_keep, -1
            else:
                feat, frow, fadd = self._fb_rows(self.step_hid, self.step_out)[k - 2:k - 1], None, 0
            # the chain appends at n + k - 1 (contiguous positions, causal, python/woodcock/spec.py:349);
            # the layer's final RMSNorm is left to the next head (out_out = NULL)
            _lib.call("wc_drafter_forward", dims, W, ptr(self.drafts[k - 1:k]), ptr(feat), dm, frow, fadd, 1, None,
                      self._kp, self._vp, self._kvdt, cap, ptr(self.state[S_N:S_N + 1]), k - 1, None, None, 0,
                      ptr(self.step_hid[k - 1:k]), None, None, ws, s)
            _lib.call("wc_draft_head_norm", dims, W, ptr(self.step_hid[k - 1:k]), dm, None, 0,
                      ptr(self.step_out[k - 1:k]), dm, None, 0, ptr(self.drafts[k:k + 1]), None, None, ws, s)
        # the speculative entries n..n+K-2 are simply overwritten later: the
        # drafter's committed count n is never advanced by the chain (spec.py:351-352)

    def enqueue_verify(self, target_logits: torch.Tensor) -> None:
        """Fused target argmax + greedy acceptance (spec.py:355-361) -> verdict."""
        _lib.call("wc_verify_chain_greedy", ptr(target_logits), target_logits.shape[0], target_logits.shape[1],
                  target_logits.stride(0), ptr(self.drafts), ptr(self.verdict), ptr(self.vws), stream_ptr())

    def enqueue_commit(self, taps: list[torch.Tensor]) -> None:
        """Compaction of the target KV (spec.py:362) and the drafter update over
        the a+1 accepted tokens (spec.py:363-374), all keyed off the verdict."""
        d = self.d
        V = _lib
        keep = self.verdict[V.V_KEEP:V.V_KEEP + V.WC_MAX_NODES + 1]
        n_keep = self.verdict[V.V_N_KEEP:V.V_N_KEEP + 1]
        if self.target_cache is not None:
            compact_cache_dev(self.target_cache, self.state[S_N:S_N + 1], keep, n_keep, self.K + 1,
                              self.state[S_TARGET_OFFSET:S_TARGET_OFFSET + 1], self.verdict[V.V_STATUS:V.V_STATUS + 1])
        dims, W, ws, s = C.byref(d.dims), C.byref(d.wstruct), ptr(d.ws), stream_ptr()
        dm = d.cfg.hidden_size
        tp = (C.c_void_p * len(taps))(*[t.data_ptr() for t in taps])
        tdt = V.WC_BF16 if taps[0].dtype == torch.bfloat16 else V.WC_F32
        V.call("wc_drafter_fuse", dims, W, tp, tdt, taps[0].stride(0), ptr(keep), self.K + 1, ptr(n_keep), ptr(self.g),
               dm, ws, s)
        # appends the accepted entries at n and advances n in place (last kernel of the pass)
        V.call("wc_drafter_forward", dims, W, ptr(self.verdict[V.V_TOKENS:V.V_TOKENS + self.K + 1]), ptr(self.g), dm,
               None, 0, self.K + 1, ptr(n_keep), self._kp, self._vp, self._kvdt, self.cache[0].capacity,
               ptr(self.state[S_N:S_N + 1]), 0, None, None, 0, ptr(self.upd_hid), None,
               ptr(self.state[S_N:S_N + 1]), ws, s)

    def enqueue_readback(self) -> None:
        self.host_verdict.copy_(self.verdict, non_blocking=True)

    def enqueue_round(self, target) -> None:
        self.enqueue_draft()
        self.enqueue_verify(target.logits)
        self.enqueue_commit(target.taps)
        self.enqueue_readback()

    # ------------------------------------------------------------------ host side

    def finish(self) -> RoundResult:
        """The round's single host synchronisation: wait for the verdict copy."""
        torch.cuda.current_stream().synchronize()
        self.syncs += 1
        v = _lib.Verdict.from_buffer_copy(self.host_verdict.numpy().tobytes())
        if v.status != 0:
            raise ValueError(f"device-side verification rejected its inputs (status {v.status})")
        a = int(v.n_accepted)
        for c in self.cache:
            c.offset += a + 1
        return RoundResult(a, [int(t) for t in v.tokens[: a + 1]])

    def run(self, target) -> RoundResult:
        self.enqueue_round(target)
        return self.finish()

    def committed(self) -> int:
        """Device committed count (reads device memory: a sync, for tests only)."""
        return int(self.state[S_N].item())


def verdict_of(t: torch.Tensor):
    return read_verdict(t)
