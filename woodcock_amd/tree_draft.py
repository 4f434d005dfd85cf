"""Tree drafting on the device: the level loop of SpeculativeDecoder._draft
with a StaticPolicy (python/woodcock/spec.py:216-303; python/woodcock/policies.py:49-75)
without a host round trip per level, greedy or sampled (T > 0).

Per level the frontier's drafter outputs go through the draft head (logits over
the head rows), ``wc_tree_draft_expand_logits`` (top-``width`` children per
frontier row under the T = 1 softmax of spec.py:120-121, whose q it forms only
for those children; phat products) and, unless the level
is the last, ``wc_tree_draft_frontier`` (top-``width`` nodes by phat become the
next frontier; it writes their tokens, parent-feedback rows, positions and
attention mask) and one drafter forward over the frontier rows, appended to
the drafter cache at offset + tree entries so far.  The cache offset itself
never moves: the reference rolls it back to the round's base after drafting
(spec.py:295-296).  ``wc_tree_draft_select`` then writes the verified tree.

At T > 0 (``stochastic=True``, spec.py:238-249) the level's q is the draft
distribution at the temperature, each frontier row draws its children without
replacement (``wc_tree_draft_expand_sample``: the number fixed before drawing,
Plan.children_for, policies.py:32-36), every drawn node is verified
(select_verify, policies.py:67-69), and each expanded node keeps its q row for
the verification (spec.py:247,322).  The drawn node counts live on the device,
so the host runs every level over upper-bound shapes: ``min(width, budget)``
frontier rows (padding rows are harmless), cache slots in strides of that many
rows per level, and a verify block of ``budget + 1`` rows whose live count is
``tree.count``.

Every launch is stream-ordered and nothing is read back: ``draft`` returns
device tensors (tokens, parents, depth, count).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import torch

from . import _lib
from .drafter import Drafter
from .runtime import device_of, ptr, stream_ptr, workspace


@dataclass
class DeviceTree:
    tokens: torch.Tensor   # [max_nodes] int32, the first `count` valid
    parents: torch.Tensor  # [max_nodes] int32 (-1 for the root)
    depth: torch.Tensor    # [max_nodes] int32
    count: torch.Tensor    # [1] int32
    q_rows: torch.Tensor | None = None  # [max_nodes] int32: row of each node's draft distribution (sampled trees)


class TreeDrafter:
    """Static tree shape: ``max_depth`` levels, ``width`` children per frontier
    node and ``width`` frontier nodes per level, ``budget`` verified nodes
    besides the root (StaticPolicy(depth, width, budget)).  ``stochastic``:
    sampled drafting at T > 0, where the budget caps the draws instead."""

    def __init__(self, drafter: Drafter, cache, max_depth: int, width: int, budget: int | None = None,
                 stochastic: bool = False):
        if width < 1 or width > 8:
            raise ValueError("width must be in 1..8")
        if max_depth < 1:
            raise ValueError("max_depth must be positive")
        self.d = drafter
        self.cache = cache
        self.max_depth, self.width = max_depth, width
        self.budget = budget if budget is not None else (max_depth if width == 1 else 4 * max_depth)
        self.stochastic = stochastic
        dev = drafter.device
        self.device = dev
        # static shape: level 1 has `width` nodes, every later level width * width
        self.levels = []  # (node_base, rows) of each level's expansion
        n, rows = 1, 1
        for _ in range(max_depth):
            self.levels.append((n, rows))
            n += rows * width
            rows = min(width, rows * width)
        self.n_nodes = n
        if self.n_nodes > 512 and not stochastic:
            raise ValueError(f"tree of {self.n_nodes} nodes exceeds the 512-node table")
        if stochastic:
            if not 0 <= self.budget <= _lib.WC_MAX_NODES - 1:
                raise ValueError(f"a sampled tree verifies budget + 1 <= {_lib.WC_MAX_NODES} rows")
            self.fwd_rows = min(width, self.budget)  # frontier rows forwarded per level (upper bound)
            self.max_nodes = self.budget + 1
        hid = drafter.cfg.hidden_size
        self.n_store = 1 + (max_depth - 1) * width  # root + every forwarded frontier row
        self.store_hid = torch.zeros(self.n_store, hid, dtype=torch.float32, device=dev)
        self.store_out = torch.zeros(self.n_store, hid, dtype=torch.float32, device=dev)
        head_rows = drafter._head.shape[0]
        self.logits = torch.empty(width, head_rows, dtype=torch.float32, device=dev)
        self.tokens = torch.empty(width, dtype=torch.int32, device=dev)
        self.feat_rows = torch.empty(width, dtype=torch.int32, device=dev)
        self.positions = torch.empty(width, dtype=torch.int32, device=dev)
        cap = cache[0].capacity
        self.mask = torch.zeros(width, cap, dtype=torch.uint8, device=dev)
        self.state = torch.zeros(int(_lib.lib().wc_tree_draft_state_bytes()), dtype=torch.uint8, device=dev)
        nt = self.max_nodes if stochastic else self.n_nodes
        self.tree = DeviceTree(torch.zeros(nt, dtype=torch.int32, device=dev),
                               torch.zeros(nt, dtype=torch.int32, device=dev),
                               torch.zeros(nt, dtype=torch.int32, device=dev),
                               torch.zeros(1, dtype=torch.int32, device=dev),
                               torch.zeros(nt, dtype=torch.int32, device=dev) if stochastic else None)
        # sampled trees: the q rows of every frontier, at the frontier's feedback-store rows
        self.q_store = (torch.zeros(self.n_store, head_rows, dtype=torch.float32, device=dev) if stochastic
                        else None)

    def draft(self, root_token: torch.Tensor, root_out: torch.Tensor | None, root_fb: torch.Tensor | None,
              offset_dev: torch.Tensor, root_hidden: torch.Tensor | None = None, temperature: float = 1.0,
              rng=None) -> DeviceTree:
        """root_token [1] int32 (device), root_out / root_fb [hidden] fp32 rows, the
        drafter's context length n = *offset_dev.  Enqueue only.  With post_norm
        the feedback of a node is its `out` (drafter.py:193-194), so root_fb is
        read only when post_norm is off.  Alternatively root_hidden, the root's
        pre-norm hidden row: the first level's head then applies the final
        RMSNorm itself (out = RMSNorm(hidden), drafter.py:190) and root_out /
        root_fb are not used.  A stochastic drafter draws at ``temperature``
        from ``rng`` (a ``wc_uniforms``)."""
        if self.stochastic:
            if rng is None:
                raise ValueError("sampled tree drafting needs a uniform stream")
            return self._draft_sample(root_token, root_out, root_fb, offset_dev, root_hidden, float(temperature), rng)
        d, w = self.d, self.width
        cfg = d.cfg
        hidden = cfg.hidden_size
        s = stream_ptr()
        # store row 0: the root; row 1 + (level - 1) * width + r: frontier row r of a level
        if root_hidden is not None:
            device_of(root_hidden)
            self.store_hid[0].copy_(root_hidden.reshape(hidden))
        else:
            device_of(root_out)
            self.store_out[0].copy_(root_out.reshape(hidden))
            self.store_hid[0].copy_(root_fb.reshape(hidden))
        fb_store = self.store_out if cfg.post_norm else self.store_hid
        _lib.call("wc_tree_draft_begin", ptr(self.state), ptr(root_token), s)
        cache = self.cache
        cap = cache[0].capacity
        kp = (C.c_void_p * len(cache))(*[c.keys.data_ptr() for c in cache])
        vp = (C.c_void_p * len(cache))(*[c.values.data_ptr() for c in cache])
        kvdt = _lib.WC_BF16 if cache[0].keys.dtype == torch.bfloat16 else _lib.WC_F32
        head_rows = self.logits.shape[1]
        tree_cache = 0
        store_row = 0  # first store row of the current frontier
        for depth, (node_base, rows) in enumerate(self.levels, start=1):
            # (a) children of every frontier node: head logits, q = softmax(z), top-width
            if depth == 1 and root_hidden is not None:  # final norm of the root, its `out` -> store row 0
                _lib.call("wc_draft_head_norm", C.byref(d.dims), C.byref(d.wstruct), ptr(self.store_hid), hidden,
                          None, 0, ptr(self.store_out), hidden, ptr(self.logits), self.logits.stride(0),
                          None, None, None, ptr(d.ws), s)
            else:
                _lib.call("wc_draft_head", C.byref(d.dims), C.byref(d.wstruct), ptr(self.store_out[store_row]),
                          hidden, None, 0, rows, ptr(self.logits), self.logits.stride(0), None, None,
                          None, ptr(d.ws), s)
            # q = softmax(z) formed only for the chosen children, in the expansion itself
            _lib.call("wc_tree_draft_expand_logits", ptr(self.state), ptr(self.logits), rows, head_rows,
                      self.logits.stride(0), ptr(d._vocab_ids), w, node_base, s)
            if depth == self.max_depth:
                break
            # (b) the most probable nodes of this level become the frontier and are forwarded
            lb, le = node_base, node_base + rows * w
            m = min(w, le - lb)
            store_base = 1 + (depth - 1) * w
            _lib.call("wc_tree_draft_frontier", ptr(self.state), lb, le, w, ptr(offset_dev), tree_cache,
                      int(cfg.window or 0), store_base, ptr(self.tokens), ptr(self.feat_rows), ptr(self.positions),
                      ptr(self.mask), self.mask.stride(0), s)
            _lib.call("wc_drafter_forward", C.byref(d.dims), C.byref(d.wstruct), ptr(self.tokens), ptr(fb_store),
                      fb_store.stride(0), ptr(self.feat_rows), 0, m, None, kp, vp, kvdt, cap, ptr(offset_dev),
                      tree_cache, ptr(self.positions), ptr(self.mask), self.mask.stride(0),
                      ptr(self.store_hid[store_base]), ptr(self.store_out[store_base]), None, ptr(d.ws), s)
            tree_cache += m
            store_row = store_base
        t = self.tree
        _lib.call("wc_tree_draft_select", ptr(self.state), self.n_nodes, self.budget, ptr(t.tokens), ptr(t.parents),
                  ptr(t.depth), ptr(t.count), s)
        return t

    def _draft_sample(self, root_token, root_out, root_fb, offset_dev, root_hidden, temperature, rng) -> DeviceTree:
        """The T > 0 level loop (spec.py:216-303, stochastic branch 238-249)."""
        d, w = self.d, self.width
        cfg = d.cfg
        hidden = cfg.hidden_size
        s = stream_ptr()
        if root_hidden is not None:
            device_of(root_hidden)
            self.store_hid[0].copy_(root_hidden.reshape(hidden))
        else:
            device_of(root_out)
            self.store_out[0].copy_(root_out.reshape(hidden))
            self.store_hid[0].copy_(root_fb.reshape(hidden))
        fb_store = self.store_out if cfg.post_norm else self.store_hid
        _lib.call("wc_tree_draft_begin", ptr(self.state), ptr(root_token), s)
        cache = self.cache
        cap = cache[0].capacity
        kp = (C.c_void_p * len(cache))(*[c.keys.data_ptr() for c in cache])
        vp = (C.c_void_p * len(cache))(*[c.values.data_ptr() for c in cache])
        kvdt = _lib.WC_BF16 if cache[0].keys.dtype == torch.bfloat16 else _lib.WC_F32
        head_rows = self.logits.shape[1]
        qs = self.q_store
        rows, store_row, tree_cache = 1, 0, 0
        levels = self.max_depth if self.budget > 0 else 0  # no budget: the root alone
        for depth in range(1, levels + 1):
            # (a) the frontier's draft distributions q = softmax(z / T) (spec.py:113-125), the draws
            if depth == 1 and root_hidden is not None:
                _lib.call("wc_draft_head_norm", C.byref(d.dims), C.byref(d.wstruct), ptr(self.store_hid), hidden,
                          None, 0, ptr(self.store_out), hidden, ptr(self.logits), self.logits.stride(0),
                          None, None, None, ptr(d.ws), s)
            else:
                _lib.call("wc_draft_head", C.byref(d.dims), C.byref(d.wstruct), ptr(self.store_out[store_row]),
                          hidden, None, 0, rows, ptr(self.logits), self.logits.stride(0), None, None,
                          None, ptr(d.ws), s)
            _lib.call("wc_probs_from_logits", ptr(self.logits), rows, head_rows, self.logits.stride(0), temperature,
                      0, 1.0, ptr(qs[store_row]), qs.stride(0), ptr(workspace(d.device)), s)
            _lib.call("wc_tree_draft_expand_sample", ptr(self.state), ptr(qs[store_row]), rows, head_rows,
                      qs.stride(0), ptr(d._vocab_ids), w, self.budget, C.byref(rng), s)
            if depth == self.max_depth:
                break
            # (b) the most probable nodes of the level become the frontier and are forwarded
            store_base = 1 + (depth - 1) * w
            _lib.call("wc_tree_draft_frontier", ptr(self.state), 0, 0, w, ptr(offset_dev), tree_cache,
                      int(cfg.window or 0), store_base, ptr(self.tokens), ptr(self.feat_rows), ptr(self.positions),
                      ptr(self.mask), self.mask.stride(0), s)
            m = self.fwd_rows
            _lib.call("wc_drafter_forward", C.byref(d.dims), C.byref(d.wstruct), ptr(self.tokens), ptr(fb_store),
                      fb_store.stride(0), ptr(self.feat_rows), 0, m, None, kp, vp, kvdt, cap, ptr(offset_dev),
                      tree_cache, ptr(self.positions), ptr(self.mask), self.mask.stride(0),
                      ptr(self.store_hid[store_base]), ptr(self.store_out[store_base]), None, ptr(d.ws), s)
            tree_cache += m
            store_row, rows = store_base, m
        t = self.tree
        _lib.call("wc_tree_draft_select_all", ptr(self.state), self.max_nodes, ptr(t.tokens), ptr(t.parents),
                  ptr(t.depth), ptr(t.q_rows), ptr(t.count), s)
        return t
