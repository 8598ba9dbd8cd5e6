"""Oracle restatement of the attention-sum importance update.

``fused_importance_update`` (akv/triton_ops.py:604-650, the torch path):
    imp = attn.float().mean(dim=(0, 1)).sum(dim=0)       # (N,)
    truncate imp to len(scores) or zero-pad it
    scores.mul_(decay).add_(imp)                         # in place, returned
(The Triton kernel at akv/triton_ops.py:288-323 divides by M; the torch path
and ``ImportanceScorer`` sum over queries -- the sum is followed here.)

``ImportanceScorer.get_eviction_candidates`` (akv/importance.py:245-300): the
lowest scores of the first seq_len positions with the first / last protected
windows kept, ascending; FIFO takes the oldest unprotected positions.

``ImportanceScorer.update`` (akv/importance.py:73-164): ATTENTION_ACCUMULATION
and IMPORTANCE apply the same EMA on the first kv_len scores (growing the
per-layer score vector with zeros); OBSERVATION_WINDOW sums only the last
``observation_window`` queries and average-pools with ``pooling_kernel``
(count_include_pad) before the EMA; HEAVY_HITTER keeps the elementwise maximum;
RECENCY_WEIGHTED and FIFO replace the scores by linspace(0, 1) / arange;
HYBRID normalises the EMA by its maximum (clamped at 1e-10) and mixes in
recency.

This module is test infrastructure: only the tests, the smoke check and the
benchmark's CPU-baseline leg use it, as the checker.

Pinning: the decay KAT ``ones(32)``, zero attention, decay 0.5 -> 0.5
(tests/test_triton_ops.py:169-174); float64 evaluation of the closed form;
sum-over-queries vs mean checked at M > 1; the window and pooling against a
direct float64 loop (tests/test_oracle_pinning.py); the policy strategies
against their closed forms evaluated elementwise in float64; the eviction
candidates against brute force over all subsets on tie-free inputs and the
protected windows (tests/test_oracle_pinning.py).
"""
from __future__ import annotations

import numpy as np


def importance_from_attn(attn: np.ndarray) -> np.ndarray:
    a = np.asarray(attn, dtype=np.float32)
    return a.mean(axis=(0, 1), dtype=np.float32).sum(axis=0, dtype=np.float32)


def fused_importance_update(attn: np.ndarray, scores: np.ndarray, decay: float = 0.95) -> np.ndarray:
    """akv/triton_ops.py:604-650 (returns the updated copy)."""
    imp = importance_from_attn(attn)
    n = scores.shape[0]
    if imp.shape[0] > n:
        imp = imp[:n]
    elif imp.shape[0] < n:
        imp = np.concatenate([imp, np.zeros(n - imp.shape[0], np.float32)])
    s = np.asarray(scores, dtype=np.float32) * np.float32(decay)
    return (s.astype(np.float32) + imp).astype(np.float32)


def scorer_update(scores, attn, strategy="attention_accumulation", decay=0.95,
                  observation_window=32, pooling_kernel=7, attention_weight=0.7, recency_weight=0.3):
    """akv/importance.py:73-164 (every strategy); returns new scores."""
    a = np.asarray(attn, dtype=np.float32)
    avg = a.mean(axis=(0, 1), dtype=np.float32)  # (M, N)
    key_imp = avg.sum(axis=0, dtype=np.float32)
    kv_len = key_imp.shape[0]
    if strategy == "observation_window":
        ql = avg.shape[0]
        w = min(observation_window, ql)
        key_imp = avg[ql - w:, :].sum(axis=0, dtype=np.float32)
        ks = pooling_kernel
        if ks > 1 and kv_len > ks:
            pad = ks // 2
            xp = np.concatenate([np.zeros(pad, np.float32), key_imp, np.zeros(pad, np.float32)])
            L = xp.shape[0] - ks + 1
            pooled = np.array([xp[i:i + ks].sum(dtype=np.float32) for i in range(L)], np.float32) / np.float32(ks)
            key_imp = pooled[:kv_len].astype(np.float32)
    if scores is None or scores.shape[0] < kv_len:
        new = np.zeros(kv_len, np.float32)
        if scores is not None:
            new[: scores.shape[0]] = scores
        scores = new
    scores = np.array(scores, dtype=np.float32, copy=True)
    head = scores[:kv_len]
    if strategy in ("attention_accumulation", "importance", "observation_window"):  # :127-128, :146-151
        head[:] = (head * np.float32(decay)).astype(np.float32) + key_imp
    elif strategy == "heavy_hitter":  # :130-132
        head[:] = np.maximum(head, key_imp)
    elif strategy == "recency_weighted":  # :134-137
        head[:] = np.linspace(0, 1, kv_len, dtype=np.float32)
    elif strategy == "hybrid":  # :139-146
        ema = (head * np.float32(decay)).astype(np.float32) + key_imp
        rec = np.linspace(0, 1, kv_len, dtype=np.float32)
        head[:] = (np.float32(attention_weight) * ema / max(np.float32(ema.max()), np.float32(1e-10))
                   + np.float32(recency_weight) * rec).astype(np.float32)
    elif strategy == "fifo":  # :148-150
        head[:] = np.arange(kv_len, dtype=np.float32)
    else:
        raise ValueError(f"unknown strategy {strategy}")
    return scores


def eviction_candidates(scores, seq_len: int, num_to_evict: int, strategy="importance", initial=4, recent=32):
    """akv/importance.py:245-300 (ties: lowest index first, as oracle.selection)."""
    if num_to_evict <= 0:
        return np.zeros(0, np.int64)
    n_start, n_end = min(initial, seq_len), min(recent, seq_len)
    if strategy == "fifo":
        n = min(num_to_evict, max(0, seq_len - n_end - n_start))
        return np.arange(n_start, n_start + n, dtype=np.int64)
    if scores is None:
        return np.zeros(0, np.int64)
    s = np.array(scores[:seq_len], dtype=np.float32, copy=True)
    s[:n_start] = np.inf
    if n_end > 0:
        s[-n_end:] = np.inf
    n = min(num_to_evict, int(np.sum(s != np.inf)))
    if n <= 0:
        return np.zeros(0, np.int64)
    return np.sort(np.argsort(s, kind="stable")[:n]).astype(np.int64)
