"""Draft-vocabulary (d2t map) construction (python/woodcock/vocab.py:35-47,83-87).

The drafter's LM head is restricted to K target ids; row r of the restricted
head drafts token ids[r].  ids are absolute target ids, sorted ascending, with
the end-of-sequence ids always included.
"""
from __future__ import annotations

import numpy as np


def top_ids(counts: np.ndarray, k: int, always=frozenset()) -> np.ndarray:
    """The k most frequent ids (a tie goes to the smaller id), always containing
    `always`, sorted ascending, int32 (vocab.py:35-47)."""
    counts = np.asarray(counts)
    if not 0 < k <= len(counts):
        raise ValueError(f"vocabulary size {k} not in 1..{len(counts)}")
    forced_ids = sorted(set(int(a) for a in always))
    if len(forced_ids) > k:
        raise ValueError("more forced ids than k")
    by_count = np.argsort(-counts, kind="stable")  # stable: equal counts keep ascending id order
    is_forced = np.zeros(len(counts), dtype=bool)
    is_forced[forced_ids] = True
    chosen = by_count[~is_forced[by_count]][: k - len(forced_ids)]
    return np.sort(np.concatenate([np.asarray(forced_ids, dtype=np.int64), chosen])).astype(np.int32)


def load_ids(spec: str) -> np.ndarray:
    """'<counts.npz>:<K>' -> draft vocabulary ids, EOS always included (vocab.py:83-87)."""
    path, _, k = spec.rpartition(":")
    z = np.load(path)  # allow_pickle stays False
    return top_ids(z["counts"], int(k), set(int(e) for e in z["eos"]))
