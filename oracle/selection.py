"""Oracle restatement of ``AKVLayer._select_demote_indices`` (akv/drop_in.py:392-413).

    protect_initial = 4 ; protect_recent = min(16, hot_budget // 4)
    FIFO arange(n) when the score vector does not match hot_len
    scores[:4] = +inf ; scores[max(0, hot_len - protect_recent):] = +inf
    topk(n_demote, largest=False) then ascending sort of the indices

Pinning: brute force over all subsets on tiny tie-free inputs; order among
exactly equal scores (torch.topk tie order) is parity unpinned -- the oracle
takes the lowest index first.
"""
from __future__ import annotations

import numpy as np


def select_demote_indices(importance, n_demote: int, hot_len: int, hot_budget: int) -> np.ndarray:
    if importance is None or np.asarray(importance).shape[0] != hot_len:
        return np.arange(n_demote, dtype=np.int64)
    s = np.array(importance, dtype=np.float32, copy=True)
    protect_recent = min(16, hot_budget // 4)
    s[:4] = np.inf
    s[max(0, hot_len - protect_recent):] = np.inf
    order = np.argsort(s, kind="stable")[:n_demote]
    return np.sort(order).astype(np.int64)
