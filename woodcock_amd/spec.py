"""Speculative-decoding rounds with ONE host synchronisation each
(python/woodcock/spec.py:104-374).

``ChainRound`` holds the device side of a round and enqueues its launches:

    head(RMSNorm(root)) -> d_1                          (final norm + draft head + argmax + d2t)
    for k in 1..K-1: drafter layer(d_k, fb) -> head(RMSNorm(h)) -> d_{k+1}
    target logits at [x_n, d_1..d_K]                    (the target's verify forward)
    fused target argmax + greedy accept -> verdict      (a, accepted tokens + next, keep)
    update: fuse(taps[keep]) and one drafter pass over the a+1 accepted tokens,
            which appends them to the drafter cache and yields the next root
    copy the verdict to pinned host memory              <- the round's single sync

A chain keeps the verify block's prefix, so the target's KV needs no move: its
committed length is the device count n that the update advances
(python/woodcock/target.py:170, compact_cache with keep == range(n)).  A tree
round (``enqueue_tree_*``) keeps ``[0] + path``: the target KV is gathered along
the accepted branch (wc_kv_compact) and the taps at the same rows feed the
update (spec.py:325-328).

Round-varying integers -- the committed count n (drafter base == target
start), the accepted count, the kept rows, x_n -- are read from device memory,
so the same kernel sequence (or one captured HIP graph per chain length)
serves every round.

``SpeculativeDecoder`` is the round loop of SpeculativeDecoder.generate
(spec.py:151-212): before each round the policy plans the draft shape
(``CostAwareChain`` re-chooses the chain length every round), after it the
policy observes the outcome; greedy chains run the fused single-sync round
(spec.py:331-364), trees the drafting / verify / compact / update sequence of
spec.py:187-201 -- also with one host synchronisation, since tree drafting and
the tree verification stay on the device.  At T > 0 every round (a chain is a
width-1 tree) takes that sequence with the stochastic branches: sampled
drafting (spec.py:238-249), the warped target distribution and recursive
rejection down the tree (spec.py:320-324).

State invariants follow python/woodcock/spec.py:1-15: before a round the
drafter cache holds real entries 0..n-1 and the root is the drafter's hidden
state of entry n-1 (row n_keep-1 of the previous update); its output, the final
RMSNorm of it, is formed by the head launch that consumes it, so no drafter
pass of the round runs a norm of its own on the critical path.
"""
from __future__ import annotations

import ctypes as C
import time
from dataclasses import dataclass, field

import numpy as np
import torch

from . import _lib
from .cache import KVCache, compact_cache_dev
from .drafter import Drafter
from .policies import Plan, Policy
from .runtime import check_verdict, new_verdict, ptr, read_verdict, stream_ptr
from .sampling import SamplingParams, probs_from_logits

# state vector slots (device int32)
S_N, S_ROUND = 0, 1
# sub-streams of a sampled round's uniforms (Philox under the sampling seed, keyed by the round counter)
PURPOSE_VERIFY, PURPOSE_DRAFT = 0, 1


@dataclass
class RoundResult:
    n_accepted: int
    tokens: list[int]  # accepted drafts + the target's next token
    k: int = 0         # drafts verified this round (chain length, or tree nodes besides the root)
    depth: int = 0     # chain length, or the tree's depth


class ChainRound:
    """Device state and buffers of greedy rounds with chains of up to ``k``
    drafts (<= 15) and kept blocks of up to ``max_keep`` rows (>= k + 1; a tree
    round keeps its depth + 1 rows at most).

    The chain methods take the round's chain length (default ``k``): every
    buffer is sized for the longest, so rounds of different lengths share the
    drafter cache, the verdict and the device state."""

    def __init__(self, drafter: Drafter, k: int, capacity: int, target_cache: list[KVCache] | None = None,
                 max_keep: int | None = None):
        if not 1 <= k <= _lib.WC_MAX_STEP_ROWS - 1:
            raise ValueError(f"chain length must be in 1..{_lib.WC_MAX_STEP_ROWS - 1}")
        max_keep = max(k + 1, max_keep or 0)
        if max_keep > _lib.WC_MAX_STEP_ROWS:
            raise ValueError(f"at most {_lib.WC_MAX_STEP_ROWS} kept rows per round")
        self.d = drafter
        self.K = k
        self.pending = True  # chain heads hand their argmax to the next forward (Drafter.pending_ok)
        self.max_keep = max_keep
        dev = drafter.device
        dm = drafter.cfg.hidden_size
        self.cache = drafter.make_cache(capacity)
        self.target_cache = target_cache
        self.state = torch.zeros(8, dtype=torch.int32, device=dev)
        self.verdict = new_verdict(dev)
        # the verify block's tokens [x_n, d_1..d_K]; the drafts are written in place
        self.seq = torch.zeros(k + 1, dtype=torch.int32, device=dev)
        self.drafts = self.seq[1:]
        self.step_hid = torch.zeros(max(k - 1, 1), dm, dtype=torch.float32, device=dev)
        self.step_out = torch.zeros_like(self.step_hid)
        self.upd_hid = torch.zeros(max_keep, dm, dtype=torch.float32, device=dev)
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

    def set_root(self, n: int, root_hidden: torch.Tensor, x_n: int = 0) -> None:
        """Start state: n committed entries in the drafter cache, x_n the newest
        committed token (not yet in either cache) and the root -- the drafter's
        pre-norm hidden state of entry n-1 (its output, the final RMSNorm of it,
        is formed by the first head launch of the round)."""
        self.upd_hid[0].copy_(root_hidden.reshape(-1))
        self.verdict.zero_()
        self.verdict[_lib.V_N_KEEP] = 1
        self.verdict[_lib.V_NEXT] = int(x_n)
        self.verdict[_lib.V_TOKENS] = int(x_n)
        self.state.zero_()
        self.state[S_N] = n
        for c in self.cache:
            c.offset = n

    def _fb_rows(self, hid: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
        return out if self.d.cfg.post_norm else hid

    def n_dev(self) -> torch.Tensor:
        """The committed count n on the device: the drafter's base and the target's offset."""
        return self.state[S_N:S_N + 1]

    def x_n_dev(self) -> torch.Tensor:
        """x_n on the device: the last round's next token."""
        return self.verdict[_lib.V_NEXT:_lib.V_NEXT + 1]

    def _k(self, k: int | None) -> int:
        k = self.K if k is None else int(k)
        if not 1 <= k <= self.K:
            raise ValueError(f"chain length {k} outside 1..{self.K}")
        return k

    # ------------------------------------------------------------------ chain rounds

    def enqueue_draft(self, k: int | None = None) -> None:
        """k head launches and k-1 drafter layers from the root; drafts -> self.drafts[:k]."""
        k = self._k(k)
        d = self.d
        dims, W, ws, s = C.byref(d.dims), C.byref(d.wstruct), ptr(d.ws), stream_ptr()
        n_keep = ptr(self.verdict[_lib.V_N_KEEP:_lib.V_N_KEEP + 1])
        dm = d.cfg.hidden_size
        cap = self.cache[0].capacity
        # d_1 from the root = update row n_keep - 1; the head applies the final
        # RMSNorm and leaves the root's output in upd_out (same row)
        # every head but the last leaves its argmax pending in the workspace: the
        # next forward resolves it as its token (and writes drafts[i - 1]), so no
        # head launch ends in a last-block reduction on the critical path
        pend = self.pending and d.pending_ok
        head = "wc_draft_head_norm_pending" if pend and k > 1 else "wc_draft_head_norm"
        tok0 = () if head == "wc_draft_head_norm_pending" else (ptr(self.drafts[0:1]), None)
        _lib.call(head, dims, W, ptr(self.upd_hid), dm, n_keep, -1, ptr(self.upd_out), dm, None, 0, *tok0, None, ws, s)
        root_fb = self._fb_rows(self.upd_hid, self.upd_out)
        for i in range(1, k):
            if i == 1:
                feat, frow, fadd = root_fb, n_keep, -1
            else:
                feat, frow, fadd = self._fb_rows(self.step_hid, self.step_out)[i - 2:i - 1], None, 0
            # the chain appends at n + i - 1 (contiguous positions, causal, python/woodcock/spec.py:349);
            # the layer's final RMSNorm is left to the next head (out_out = NULL)
            if pend:
                _lib.call("wc_drafter_forward_pending", dims, W, ptr(self.drafts[i - 1:i]), None, ptr(feat), dm, frow,
                          fadd, self._kp, self._vp, self._kvdt, cap, ptr(self.n_dev()), i - 1, None,
                          ptr(self.step_hid[i - 1:i]), None, None, ws, s)
            else:
                _lib.call("wc_drafter_forward", dims, W, ptr(self.drafts[i - 1:i]), ptr(feat), dm, frow, fadd, 1,
                          None, self._kp, self._vp, self._kvdt, cap, ptr(self.n_dev()), i - 1, None, None, 0,
                          ptr(self.step_hid[i - 1:i]), None, None, ws, s)
            if pend and i < k - 1:
                _lib.call("wc_draft_head_norm_pending", dims, W, ptr(self.step_hid[i - 1:i]), dm, None, 0,
                          ptr(self.step_out[i - 1:i]), dm, None, 0, None, ws, s)
            else:
                _lib.call("wc_draft_head_norm", dims, W, ptr(self.step_hid[i - 1:i]), dm, None, 0,
                          ptr(self.step_out[i - 1:i]), dm, None, 0, ptr(self.drafts[i:i + 1]), None, None, ws, s)
        # the speculative entries n..n+k-2 are simply overwritten later: the
        # drafter's committed count n is never advanced by the chain (spec.py:351-352)

    def enqueue_seq(self) -> None:
        """x_n (the last verdict's next token) into the verify block's first slot."""
        self.seq[0:1].copy_(self.x_n_dev())

    def enqueue_verify(self, target_logits: torch.Tensor) -> None:
        """Fused target argmax + greedy acceptance (spec.py:355-361) -> verdict;
        the chain length is the logits' row count - 1."""
        rows = target_logits.shape[0]
        self._k(rows - 1)
        _lib.call("wc_verify_chain_greedy", ptr(target_logits), rows, target_logits.shape[1],
                  target_logits.stride(0), ptr(self.drafts), ptr(self.verdict), ptr(self.vws), stream_ptr())

    def _enqueue_update(self, taps: list[torch.Tensor], rows: int) -> None:
        """fuse(taps at keep) + one drafter pass over the n_keep accepted tokens
        (spec.py:366-374), appended at n; n advances by n_keep (device)."""
        d = self.d
        V = _lib
        keep = self.verdict[V.V_KEEP:V.V_KEEP + V.WC_MAX_NODES + 1]
        n_keep = self.verdict[V.V_N_KEEP:V.V_N_KEEP + 1]
        dims, W, ws, s = C.byref(d.dims), C.byref(d.wstruct), ptr(d.ws), stream_ptr()
        dm = d.cfg.hidden_size
        tp = (C.c_void_p * len(taps))(*[t.data_ptr() for t in taps])
        tdt = V.WC_BF16 if taps[0].dtype == torch.bfloat16 else V.WC_F32
        V.call("wc_drafter_fuse", dims, W, tp, tdt, taps[0].stride(0), ptr(keep), taps[0].shape[0], rows,
               ptr(n_keep), ptr(self.g), dm, ws, s)
        self._enqueue_pass(rows)

    def _enqueue_pass(self, rows: int) -> None:
        """The drafter pass of the update over the n_keep accepted tokens and the
        fused rows in self.g; appends at n and advances n in place (its last kernel)."""
        d = self.d
        V = _lib
        n_keep = self.verdict[V.V_N_KEEP:V.V_N_KEEP + 1]
        V.call("wc_drafter_forward", C.byref(d.dims), C.byref(d.wstruct),
               ptr(self.verdict[V.V_TOKENS:V.V_TOKENS + rows]), ptr(self.g), d.cfg.hidden_size, None, 0, rows,
               ptr(n_keep), self._kp, self._vp, self._kvdt, self.cache[0].capacity, ptr(self.n_dev()), 0, None, None,
               0, ptr(self.upd_hid), None, ptr(self.n_dev()), ptr(d.ws), stream_ptr())

    def enqueue_commit(self, taps: list[torch.Tensor], k: int | None = None) -> None:
        """The chain's commit: the drafter update over the a+1 accepted tokens
        (spec.py:362-374), keyed off the verdict.  The target KV keeps the
        verify block's prefix in place, so nothing moves (target.py:170)."""
        self._enqueue_update(taps, self._k(k) + 1)

    def enqueue_verify_commit(self, target_logits: torch.Tensor, taps: list[torch.Tensor],
                              k: int | None = None) -> None:
        """enqueue_verify + enqueue_commit of a chain round with the verify and
        the fuse in one launch (wc_verify_chain_greedy_fuse): a chain keeps the
        prefix [0..a] of its verify block (spec.py:362-366) and the fuse is
        row-wise, so the fuse of all k + 1 tap rows need not wait for the
        verdict; the drafter pass then reads rows 0..a.  Verdict, drafter cache
        and state equal those of the two calls in sequence."""
        k = self._k(k)
        rows = k + 1
        if target_logits.shape[0] != rows or any(t.shape[0] < rows for t in taps):
            raise ValueError(f"a chain of {k} drafts verifies {rows} rows")
        d = self.d
        tp = (C.c_void_p * len(taps))(*[t.data_ptr() for t in taps])
        tdt = _lib.WC_BF16 if taps[0].dtype == torch.bfloat16 else _lib.WC_F32
        _lib.call("wc_verify_chain_greedy_fuse", ptr(target_logits), rows, target_logits.shape[1],
                  target_logits.stride(0), ptr(self.drafts), ptr(self.verdict), ptr(self.vws), C.byref(d.dims),
                  C.byref(d.wstruct), tp, tdt, taps[0].stride(0), ptr(self.g), d.cfg.hidden_size, ptr(d.ws),
                  stream_ptr())
        self._enqueue_pass(rows)

    def enqueue_readback(self) -> None:
        self.host_verdict.copy_(self.verdict, non_blocking=True)

    def enqueue_round(self, target, k: int | None = None) -> None:
        """A chain round against a target exposing device ``logits`` / ``taps``
        at [x_n, d_1..d_K] (a synthetic stand-in whose rows are already in place)."""
        k = self._k(k)
        self.enqueue_draft(k)
        self.enqueue_verify_commit(target.logits[:k + 1], [t[:k + 1] for t in target.taps], k)
        self.enqueue_readback()

    # ------------------------------------------------------------------ tree rounds

    def enqueue_tree_verify(self, logits: torch.Tensor, tokens: torch.Tensor, parents: torch.Tensor) -> None:
        """Target argmax + greedy tree walk (sampling.py:131-140; spec.py:318-319) -> verdict."""
        rows = logits.shape[0]
        _lib.call("wc_verify_tree_greedy", ptr(logits), rows, logits.shape[1], logits.stride(0), ptr(tokens),
                  ptr(parents), ptr(self.verdict), ptr(self.vws), stream_ptr())

    def enqueue_tree_commit(self, taps: list[torch.Tensor], rows: int, max_depth: int) -> None:
        """Compaction of the target KV along the accepted branch, keep = [0] + path
        (spec.py:325-326; target.py:159-175), then the update from the taps at
        the kept rows (spec.py:327-328,366-374).  rows: the verify block's rows;
        max_depth: the tree's depth (n_keep <= max_depth + 1)."""
        V = _lib
        if max_depth + 1 > self.max_keep:
            raise ValueError(f"a tree of depth {max_depth} keeps up to {max_depth + 1} rows; "
                             f"this round state holds {self.max_keep}")
        if self.target_cache is not None:
            keep = self.verdict[V.V_KEEP:V.V_KEEP + V.WC_MAX_NODES + 1]
            n_keep = self.verdict[V.V_N_KEEP:V.V_N_KEEP + 1]
            # start = n, read before the update advances it; the update writes the new n
            compact_cache_dev(self.target_cache, self.n_dev(), keep, n_keep, rows, None,
                              self.verdict[V.V_STATUS:V.V_STATUS + 1])
        self._enqueue_update(taps, max_depth + 1)

    # ------------------------------------------------------------------ host side

    def finish(self) -> RoundResult:
        """The round's single host synchronisation: wait for the verdict copy."""
        torch.cuda.current_stream().synchronize()
        self.syncs += 1
        v = check_verdict(_lib.Verdict.from_buffer_copy(self.host_verdict.numpy().tobytes()), self.vws)
        a = int(v.n_accepted)
        for c in self.cache:
            c.offset += a + 1
        if self.target_cache is not None:
            for c in self.target_cache:
                c.offset = self.cache[0].offset
        return RoundResult(a, [int(t) for t in v.tokens[: a + 1]])

    def run(self, target, k: int | None = None) -> RoundResult:
        self.enqueue_round(target, k)
        return self.finish()

    def committed(self) -> int:
        """Device committed count (reads device memory: a sync, for tests only)."""
        return int(self.state[S_N].item())

    def last_keep(self) -> list[int]:
        """The kept rows of the last round (its host verdict copy)."""
        v = _lib.Verdict.from_buffer_copy(self.host_verdict.numpy().tobytes())
        return [int(x) for x in v.keep[: v.n_keep]]


def verdict_of(t: torch.Tensor):
    return read_verdict(t)


# ---------------------------------------------------------------------- targets

class TargetRunner:
    """The verify forward of a ``target.TargetModel`` over its own KV cache, as
    the decoder calls it: tokens [rows] (device) at cache offset *offset_dev,
    optional positions and mask -> (logits [rows, V] fp32, taps [rows, hidden]
    fp32).  Output buffers are allocated once (graph capture reuses them)."""

    def __init__(self, model, cache: list[KVCache]):
        self.model = model
        self.cache = cache
        self.vocab_size = model.cfg.vocab_size
        rows = model.max_rows
        dev = model.device
        self.logits = torch.empty(rows, model.cfg.vocab_size, dtype=torch.float32, device=dev)
        self.taps = [torch.empty(rows, model.cfg.hidden_size, dtype=torch.float32, device=dev)
                     for _ in model.feature_layers]

    def prepare(self, rows: int) -> None:
        pass

    def verify_forward(self, tokens: torch.Tensor, rows: int, offset_dev: torch.Tensor,
                       positions: torch.Tensor | None = None, mask: torch.Tensor | None = None):
        logits, taps = self.model(tokens[:rows], self.cache, offset_dev, positions, mask, logits=self.logits[:rows],
                                  taps=self.taps)
        return logits, [t[:rows] for t in taps]


# ---------------------------------------------------------------------- decoder

@dataclass
class GenStats:
    """Per-generation counters (python/woodcock/spec.py:39-89)."""

    prompt_tokens: int = 0
    new_tokens: int = 0
    rounds: int = 0
    accepted: list[int] = field(default_factory=list)  # draft tokens accepted per round
    drafted: list[int] = field(default_factory=list)   # draft tokens verified per round
    depths: list[int] = field(default_factory=list)
    t_total: float = 0.0
    fused: bool = True  # every round has one host synchronisation

    @property
    def mean_accepted(self) -> float:
        return float(np.mean(self.accepted)) if self.accepted else 0.0

    @property
    def tokens_per_round(self) -> float:
        return self.mean_accepted + 1.0

    @property
    def acceptance_rate(self) -> float:
        d = sum(self.drafted)
        return sum(self.accepted) / d if d else 0.0

    def as_dict(self) -> dict:
        return {"prompt_tokens": self.prompt_tokens, "new_tokens": self.new_tokens, "rounds": self.rounds,
                "mean_accepted": self.mean_accepted, "tokens_per_round": self.tokens_per_round,
                "acceptance_rate": self.acceptance_rate,
                "mean_verified": float(np.mean(self.drafted)) if self.drafted else 0.0,
                "mean_depth": float(np.mean(self.depths)) if self.depths else 0.0, "t_total": self.t_total,
                "fused": self.fused}


class SpeculativeDecoder:
    """Speculative decoding: one drafter cache, one target, one policy, greedy
    or sampled (``sampling``: SamplingParams with temperature > 0).

    target: ``verify_forward(tokens, rows, offset_dev, positions, mask) ->
    (logits, taps)`` enqueued without a host synchronisation (``TargetRunner``
    over a TargetModel, or a synthetic stand-in), ``prepare(rows)`` called
    before each round is enqueued or replayed, and ``cache`` (the target KV
    list to compact after tree rounds, or None).

    Chain rounds can be captured as one HIP graph per chain length
    (``use_graphs``): the policy's choice selects the graph to replay.  Tree
    rounds are enqueued eagerly (their mask prefix is the host-known n)."""

    def __init__(self, drafter: Drafter, target, policy: Policy, capacity: int = 4096, k_max: int = 8,
                 max_tree_depth: int = 0, use_graphs: bool = False, timing: bool = False,
                 sampling: SamplingParams | None = None):
        self.d = drafter
        self.t = target
        self.policy = policy
        self.sp = sampling if sampling is not None else SamplingParams()
        self._p = None  # target probabilities of a sampled round's verify block
        self._host_tree = None
        self.rnd = ChainRound(drafter, k_max, capacity, getattr(target, "cache", None),
                              max_keep=max_tree_depth + 1)
        self.k_max = k_max
        self.use_graphs = use_graphs
        self._graphs: dict[int, tuple[torch.cuda.CUDAGraph, ...]] = {}
        self._trees: dict[tuple[int, int, int], object] = {}
        self._tree_mask = None
        self.n = 0
        self.x_n = 0
        # timing: GPU events around the round's three phases -- drafting, the
        # target's verify forward, verification + commit -- read at the sync
        self.timing = timing
        self.last_times: dict[str, float] = {}
        self._ev: list = []

    # ------------------------------------------------------------------ state

    def start(self, n: int, x_n: int, root_hidden: torch.Tensor) -> None:
        """State after prefill (spec.py:129-141): n committed tokens before x_n in
        both caches, x_n the newest token, root_hidden the drafter's pre-norm
        hidden state of entry n-1 (the cache entries 0..n-1 are the caller's)."""
        self.rnd.set_root(n, root_hidden, x_n)
        if self.rnd.target_cache is not None:
            for c in self.rnd.target_cache:
                c.offset = n
        self.n, self.x_n = n, int(x_n)
        self.policy.reset()

    # ------------------------------------------------------------------ chain rounds

    def _mark(self) -> None:
        if self.timing:
            e = torch.cuda.Event(enable_timing=True)
            e.record()
            self._ev.append(e)

    def _read_times(self) -> None:
        """After the round's sync: GPU µs of each phase between the marks."""
        if self.timing and len(self._ev) == 4:
            d, t, c = (1e3 * a.elapsed_time(b) for a, b in zip(self._ev, self._ev[1:]))
            self.last_times = {"draft_us": d, "target_us": t, "verify_commit_us": c, "round_us": d + c}
        self._ev = []

    def _chain_phases(self, k: int):
        r = self.rnd
        io = {}

        def draft():
            r.enqueue_seq()
            r.enqueue_draft(k)

        def target():
            io["out"] = self.t.verify_forward(r.seq, k + 1, r.n_dev())

        def commit():
            logits, taps = io["out"]
            r.enqueue_verify_commit(logits, taps, k)
            r.enqueue_readback()

        return draft, target, commit

    def chain_round(self, k: int) -> RoundResult:
        """The fused greedy chain round of length k (spec.py:331-364)."""
        self.t.prepare(k + 1)
        graphs = self._graphs.get(k)
        self._ev = []
        self._mark()
        if graphs is not None:
            for g in graphs:
                g.replay()
                self._mark()
        else:
            for phase in self._chain_phases(k):
                phase()
                self._mark()
        res = self.rnd.finish()
        self._read_times()
        if self.use_graphs and graphs is None:
            # captured after a first eager round of this length (kernel attributes,
            # workspaces and allocator pools are in place by then)
            self._graphs[k] = self._capture(k)
        res.k = res.depth = k
        return res

    def _capture(self, k: int) -> tuple[torch.cuda.CUDAGraph, ...]:
        """One graph per phase (drafting, target forward, verify + commit), so a
        timed replay can tell the target's share apart."""
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        out = []
        for phase in self._chain_phases(k):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):  # records without executing: the state does not move
                phase()
            out.append(g)
        torch.cuda.current_stream().wait_stream(s)
        return tuple(out)

    # ------------------------------------------------------------------ tree rounds

    def tree_drafter(self, plan: Plan, stochastic: bool = False):
        from .tree_draft import TreeDrafter

        key = (plan.max_depth, plan.width, plan.budget, stochastic)
        tdr = self._trees.get(key)
        if tdr is None:
            tdr = self._trees[key] = TreeDrafter(self.d, self.rnd.cache, plan.max_depth, plan.width, plan.budget,
                                                 stochastic=stochastic)
        return tdr

    def enqueue_tree_draft(self, plan: Plan):
        """Greedy tree drafting from the root (spec.py:216-303) -> (device tree, rows)."""
        r = self.rnd
        tdr = self.tree_drafter(plan)
        idx = (r.verdict[_lib.V_N_KEEP:_lib.V_N_KEEP + 1] - 1).long()
        root_hid = r.upd_hid.index_select(0, idx)
        tree = tdr.draft(r.x_n_dev(), None, None, r.n_dev(), root_hidden=root_hid)
        return tree, min(tdr.n_nodes, tdr.budget + 1)

    def enqueue_tree_target(self, tree, rows: int):
        """The verify forward over the tree block: positions n + depth and the
        tree attention mask over the cache slots (spec.py:313-317)."""
        r = self.rnd
        width = self.n + rows
        if r.target_cache is not None:
            width = max(width, r.target_cache[0].capacity)
        width = (width + 15) // 16 * 16  # 16-byte mask rows: the verify attention reads them 16 bytes at a time
        if self._tree_mask is None or self._tree_mask.shape[1] < width:
            self._tree_mask = torch.zeros(_lib.WC_MAX_NODES, width, dtype=torch.uint8, device=self.d.device)
        mask = self._tree_mask[:rows]
        _lib.call("wc_tree_mask", ptr(tree.parents), rows, self.n, ptr(mask), mask.stride(0), stream_ptr())
        positions = tree.depth[:rows] + r.n_dev()
        return self.t.verify_forward(tree.tokens, rows, r.n_dev(), positions, mask)

    def tree_round(self, plan: Plan) -> RoundResult:
        """Greedy tree round (spec.py:187-201) with one host synchronisation."""
        r = self.rnd
        self._ev = []
        self._mark()
        tree, rows = self.enqueue_tree_draft(plan)
        self._mark()
        self.t.prepare(rows)
        logits, taps = self.enqueue_tree_target(tree, rows)
        self._mark()
        r.enqueue_tree_verify(logits, tree.tokens[:rows], tree.parents[:rows])
        r.enqueue_tree_commit(taps, rows, plan.max_depth)
        r.enqueue_readback()
        self._mark()
        res = r.finish()
        self._read_times()
        res.k, res.depth = rows - 1, plan.max_depth
        return res

    # ------------------------------------------------------------------ sampled rounds

    def _uniforms(self, purpose: int) -> _lib.Uniforms:
        return _lib.Uniforms(int(self.sp.seed), ptr(self.rnd.state[S_ROUND:S_ROUND + 1]), purpose)

    def enqueue_sampled_draft(self, plan: Plan):
        """Sampled tree drafting from the root (spec.py:216-303, T > 0) under a
        fresh round counter -> (device tree, verify-block rows, drafter)."""
        r = self.rnd
        tdr = self.tree_drafter(plan, stochastic=True)
        r.state[S_ROUND:S_ROUND + 1].add_(1)
        idx = (r.verdict[_lib.V_N_KEEP:_lib.V_N_KEEP + 1] - 1).long()
        root_hid = r.upd_hid.index_select(0, idx)
        tree = tdr.draft(r.x_n_dev(), None, None, r.n_dev(), root_hidden=root_hid,
                         temperature=self.sp.temperature, rng=self._uniforms(PURPOSE_DRAFT))
        return tree, tdr.max_nodes, tdr

    def enqueue_sampled_verify(self, tdr, tree, logits: torch.Tensor, rows: int) -> torch.Tensor:
        """p = the warped target distribution at every node (spec.py:321), then
        recursive rejection down the tree with each node's draft distribution
        (spec.py:322-324) -> verdict.  Returns p."""
        r = self.rnd
        V = logits.shape[1]
        if self._p is None or self._p.shape[1] != V:
            self._p = torch.empty(_lib.WC_MAX_NODES, V, dtype=torch.float32, device=self.d.device)
        p = self._p[:rows]
        probs_from_logits(logits[:rows], self.sp, out=p)
        qs = tdr.q_store
        u = self._uniforms(PURPOSE_VERIFY)
        _lib.call("wc_verify_tree_stochastic_indexed", ptr(p), rows, V, p.stride(0), ptr(qs), qs.shape[0],
                  ptr(tree.q_rows), qs.shape[1], qs.stride(0), ptr(self.d.vocab_ids), ptr(tree.tokens),
                  ptr(tree.parents), ptr(tree.count), C.byref(u), ptr(r.verdict), ptr(r.vws), stream_ptr())
        return p

    def sampled_round(self, plan: Plan) -> RoundResult:
        """A T > 0 round (spec.py:187-201 with the stochastic branches of _draft
        and _verify): sampled drafting (a chain when width == 1), the target's
        verify forward over the tree block, recursive rejection, compaction
        along the accepted branch and the update -- one host synchronisation."""
        r = self.rnd
        self._ev = []
        self._mark()
        tree, rows, tdr = self.enqueue_sampled_draft(plan)
        self._mark()
        self.t.prepare(rows)
        logits, taps = self.enqueue_tree_target(tree, rows)
        self._mark()
        self.enqueue_sampled_verify(tdr, tree, logits, rows)
        r.enqueue_tree_commit(taps, rows, plan.max_depth)
        # the drawn tree's size and depths ride along with the verdict copy
        if self._host_tree is None:
            self._host_tree = torch.zeros(_lib.WC_MAX_NODES + 1, dtype=torch.int32, pin_memory=True)
        self._host_tree[:1].copy_(tree.count, non_blocking=True)
        self._host_tree[1:rows + 1].copy_(tree.depth[:rows], non_blocking=True)
        r.enqueue_readback()
        self._mark()
        res = r.finish()
        self._read_times()
        count = int(self._host_tree[0])
        res.k = count - 1
        res.depth = int(self._host_tree[1:count + 1].max())
        return res

    # ------------------------------------------------------------------ loop

    def round(self) -> RoundResult:
        """One round as the policy plans it (spec.py:169-201)."""
        stochastic = not self.sp.greedy
        plan = self.policy.plan(context_len=self.n, stochastic=stochastic)
        t0 = time.perf_counter()
        if stochastic:
            res = self.sampled_round(plan)
        elif plan.width == 1:
            if not 1 <= plan.max_depth <= self.k_max:
                raise ValueError(f"planned chain of {plan.max_depth} outside 1..{self.k_max}")
            res = self.chain_round(plan.max_depth)
        else:
            res = self.tree_round(plan)
        self.policy.observe(res.n_accepted, res.k, res.depth, 0.0, time.perf_counter() - t0)
        self.n += len(res.tokens)
        self.x_n = res.tokens[-1]
        return res

    def generate(self, max_new_tokens: int, eos=()) -> tuple[list[int], GenStats]:
        """Rounds from the started state until max_new_tokens (x_n counted) or an
        EOS token (spec.py:151-212, after the prefill)."""
        st = GenStats(prompt_tokens=self.n)
        eos = set(eos)
        out = [self.x_n]
        t0 = time.perf_counter()
        while len(out) < max_new_tokens and out[-1] not in eos:
            res = self.round()
            st.rounds += 1
            st.accepted.append(res.n_accepted)
            st.drafted.append(res.k)
            st.depths.append(res.depth)
            for tok in res.tokens:
                out.append(tok)
                if tok in eos or len(out) >= max_new_tokens:
                    break
        st.t_total = time.perf_counter() - t0
        st.new_tokens = len(out)
        return out, st


# ---------------------------------------------------------------------- baseline

def target_prefill(model, cache: list, prompt, offset_dev: torch.Tensor | None = None) -> tuple[int, torch.Tensor]:
    """The prompt through ``model`` (a ``target.TargetModel``) into ``cache``, in
    causal blocks of up to ``model.max_rows`` rows (Target.__call__ over the
    prompt, python/woodcock/spec.py:386).  Returns (n, logits of the last prompt
    row [vocab] fp32 on the device); the cache offsets (host and device) end at n."""
    dev = model.device
    toks = torch.as_tensor(list(prompt), dtype=torch.int32, device=dev)
    if toks.numel() < 1:
        raise ValueError("empty prompt")
    if offset_dev is None:
        offset_dev = torch.zeros(1, dtype=torch.int32, device=dev)
    n0 = int(cache[0].offset)
    last = None
    for b0 in range(0, toks.numel(), model.max_rows):
        blk = toks[b0:b0 + model.max_rows]
        logits, _ = model(blk, cache, offset_dev)
        offset_dev.add_(blk.numel())
        for c in cache:
            c.offset += blk.numel()
        last = logits[-1]
    return n0 + toks.numel(), last


def generate_autoregressive(model, cache: list, prompt, max_new_tokens: int, eos=(), on_logits=None
                            ) -> tuple[list[int], GenStats]:
    """Baseline A of python/woodcock/spec.py:377-397 (greedy): plain target
    decoding through the same target forward -- the prompt, then one row per
    token.  The argmax of each row is the library's (wc_verify_chain_greedy
    over one row: the verdict's `next`).  ``on_logits(step, logits_row)`` sees
    every row's logits before its argmax is read (step 0: the prompt's last)."""
    st = GenStats(prompt_tokens=len(prompt), fused=False)
    eos = set(eos)
    dev = model.device
    t0 = time.perf_counter()
    off = torch.full((1,), int(cache[0].offset), dtype=torch.int32, device=dev)
    _, logits = target_prefill(model, cache, prompt, off)
    verdict = new_verdict(dev)
    n = int(_lib.lib().wc_workspace_bytes())
    ws = torch.empty((n + 255) // 256 * 256, dtype=torch.uint8, device=dev)
    _lib.call("wc_workspace_init", ptr(ws), ws.numel(), stream_ptr())
    tok_dev = torch.zeros(1, dtype=torch.int32, device=dev)

    def argmax(row: torch.Tensor, step: int) -> int:
        if on_logits is not None:
            on_logits(step, row)
        _lib.call("wc_verify_chain_greedy", ptr(row), 1, row.shape[-1], row.shape[-1], None, ptr(verdict), ptr(ws),
                  stream_ptr())
        return int(read_verdict(verdict, ws).next)

    tok = argmax(logits, 0)
    out = [tok]
    while len(out) < max_new_tokens and tok not in eos:
        tok_dev.fill_(tok)
        logits, _ = model(tok_dev, cache, off)
        off.add_(1)
        for c in cache:
            c.offset += 1
        tok = argmax(logits[0], len(out))
        out.append(tok)
    st.t_total = time.perf_counter() - t0
    st.new_tokens = len(out)
    st.rounds = len(out) - 1
    return out, st
