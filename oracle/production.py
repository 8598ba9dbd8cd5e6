"""Oracle restatement of ProductionCache's update path with the minmax warm tier
(akv/production_cache.py:73-541) and of its attention.

Per layer: a float16 hot tier (the contiguous buffer, akv/production_cache.py:182-195),
two arenas (PackedKVArena, akv/packed_layout.py:56-281) holding K and V as packed
codes + per-(head, token, group) scales / zeros, and the scorer's per-layer scores.

``update`` (:360-405): append to the hot tier; ``ImportanceScorer.update`` when
attention weights are given; the call counter; migration when the counter is a
multiple of 8, weights were given or the hot tier is over budget, and the hot
length exceeds ``hot_budget * migration_threshold``.  ``_maybe_migrate``
(:471-505): nothing at or under budget; else ``min(batch_migration_size, hot_len -
hot_budget)`` eviction candidates of the scorer (ascending hot positions), their K / V
quantized into the arenas (an append that would overflow an arena first drops its
N oldest tokens, N the append's size, or empties it when N is at least the held
count, :106-161 / :267-281), the survivors compacted in order (:266-295).
``get_kv`` (:407-427): dequantized warm (float16) then hot, along tokens.
``attention``: softmax(q K^T * D^-0.5) V in float32 over ``get_kv`` with the query
rounded to float16 (the reference's ``fused_attention``, :429-469, computes the
same expression in float16 torch matmuls).

This module is test infrastructure: only the tests, the smoke check and the
benchmark's CPU-baseline leg use it, as the checker.

Pinning: the arena quantize / dequantize restatements are pinned by the reference's
arena tests and closed forms (tests/test_oracle_pinning_legacy.py), the scorer update
and eviction candidates by their KATs and brute force (tests/test_oracle_pinning.py);
the composition here is pinned by invariants checked in tests/test_oracle_production.py:
token conservation (every appended token is in the hot tier or in the demoted
stream, the arena holding the stream's newest rows and the rest dropped by its
overflow), the hot tier's rows equal to the appended float16 rows in order, exactly
``hot_budget`` hot tokens after each update once over budget, FIFO demotions at
their closed-form positions, the warm rows within half a quantization step of their
sources, and the attention equal to a float64 softmax over the same rows.
"""
from __future__ import annotations

import numpy as np

from .fp import F16, to_dtype
from .importance import eviction_candidates, scorer_update
from .legacy import arena_dequantize, arena_quantize


class ArenaOracle:
    """PackedKVArena's contents: (H, length, D*bits/8) codes and (H, length, G)
    scales / zeros, float16 stored."""

    def __init__(self, heads: int, capacity: int, head_dim: int, bits: int, group_size: int):
        self.H, self.cap, self.D, self.bits, self.gs = heads, capacity, head_dim, bits, group_size
        G = (head_dim + group_size - 1) // group_size
        self.packed = np.zeros((heads, 0, head_dim * bits // 8), np.uint8)
        self.scales = np.zeros((heads, 0, G), np.float32)
        self.zeros = np.zeros((heads, 0, G), np.float32)
        self.dropped = 0

    @property
    def length(self) -> int:
        return self.packed.shape[1]

    def append(self, x: np.ndarray) -> int:
        n = x.shape[1]
        if n > self.cap:
            raise RuntimeError(f"{n} tokens exceed the arena's {self.cap} slots")
        if self.length + n > self.cap:  # _evict_oldest(n)
            k = min(n, self.length)
            self.dropped += k
            self.packed, self.scales, self.zeros = self.packed[:, k:], self.scales[:, k:], self.zeros[:, k:]
        start = self.length
        if n:
            p, s, z = arena_quantize(x, self.bits, self.gs, dt=F16, store=F16)
            self.packed = np.concatenate([self.packed, p], axis=1)
            self.scales = np.concatenate([self.scales, s.astype(np.float32)], axis=1)
            self.zeros = np.concatenate([self.zeros, z.astype(np.float32)], axis=1)
        return start

    def dequantize(self) -> np.ndarray:
        return arena_dequantize(self.packed, self.scales, self.zeros, self.bits, self.gs, self.D, store=F16)


class ProductionCacheOracle:
    """akv/production_cache.py:323-541 with ``warm_quantizer='minmax'``."""

    def __init__(self, num_layers: int, num_heads: int, head_dim: int, hot_budget: int, warm_budget: int,
                 warm_bits: int, group_size: int, migration_threshold: float = 0.9, batch_migration_size: int = 64,
                 decay: float = 0.3, protect_initial: int = 4, protect_recent: int = 32,
                 strategy: str = "importance"):
        self.H, self.D = num_heads, head_dim
        self.hot_budget, self.threshold, self.batch = hot_budget, migration_threshold, batch_migration_size
        self.decay, self.initial, self.recent, self.strategy = decay, protect_initial, protect_recent, strategy
        self.hot_k = [np.zeros((num_heads, 0, head_dim), np.float32) for _ in range(num_layers)]
        self.hot_v = [np.zeros((num_heads, 0, head_dim), np.float32) for _ in range(num_layers)]
        self.warm_k = [ArenaOracle(num_heads, warm_budget, head_dim, warm_bits, group_size) for _ in range(num_layers)]
        self.warm_v = [ArenaOracle(num_heads, warm_budget, head_dim, warm_bits, group_size) for _ in range(num_layers)]
        self.scores: dict = {}
        self.seq_len = [0] * num_layers
        self.decode_count = self.migrations = self.total_demoted = 0
        self.demoted_rows: list = [[] for _ in range(num_layers)]  # fp16 K rows in demotion order (invariants)

    def update(self, keys: np.ndarray, values: np.ndarray, layer: int, attn=None):
        k = to_dtype(np.asarray(keys, np.float32), F16).astype(np.float32)
        v = to_dtype(np.asarray(values, np.float32), F16).astype(np.float32)
        self.hot_k[layer] = np.concatenate([self.hot_k[layer], k], axis=1)
        self.hot_v[layer] = np.concatenate([self.hot_v[layer], v], axis=1)
        self.seq_len[layer] += k.shape[1]
        if attn is not None:
            self.scores[layer] = scorer_update(self.scores.get(layer), attn, strategy=self.strategy, decay=self.decay)
        self.decode_count += 1
        hot_len = self.hot_k[layer].shape[1]
        if self.decode_count % 8 == 0 or attn is not None or hot_len > self.hot_budget:
            if hot_len > self.hot_budget * self.threshold:
                self._migrate(layer)

    def _migrate(self, layer: int):
        hot_len = self.hot_k[layer].shape[1]
        if hot_len <= self.hot_budget:
            return
        n = min(self.batch, hot_len - self.hot_budget)
        cand = eviction_candidates(self.scores.get(layer), hot_len, n, strategy=self.strategy,
                                   initial=self.initial, recent=self.recent)
        if cand.size == 0:
            return
        dk, dv = self.hot_k[layer][:, cand], self.hot_v[layer][:, cand]
        self.warm_k[layer].append(dk)
        self.warm_v[layer].append(dv)
        self.demoted_rows[layer].append(dk)
        keep = np.ones(hot_len, bool)
        keep[cand] = False
        self.hot_k[layer], self.hot_v[layer] = self.hot_k[layer][:, keep], self.hot_v[layer][:, keep]
        self.migrations += 1
        self.total_demoted += n

    def get_kv(self, layer: int):
        """(H, N_warm + N_hot, D) float32 holding float16 values, warm first."""
        if self.warm_k[layer].length == 0:
            return self.hot_k[layer], self.hot_v[layer]
        wk = self.warm_k[layer].dequantize().astype(np.float32)
        wv = self.warm_v[layer].dequantize().astype(np.float32)
        return np.concatenate([wk, self.hot_k[layer]], axis=1), np.concatenate([wv, self.hot_v[layer]], axis=1)

    def attention(self, q: np.ndarray, layer: int, sm_scale=None) -> np.ndarray:
        """q (B, H, M, D) -> (B, H, M, D) float32; sm_scale D^-0.5 unless given."""
        k, v = self.get_kv(layer)
        qf = to_dtype(np.asarray(q, np.float32), F16).astype(np.float32)
        scale = self.D ** -0.5 if sm_scale is None else sm_scale
        s = np.einsum("bhmd,hnd->bhmn", qf, k, dtype=np.float32) * np.float32(scale)
        s = s - s.max(axis=-1, keepdims=True)
        p = np.exp(s, dtype=np.float32)
        p /= p.sum(axis=-1, keepdims=True, dtype=np.float32)
        return np.einsum("bhmn,hnd->bhmd", p, v, dtype=np.float32)
