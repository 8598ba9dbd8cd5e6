"""ImportanceScorer on the device (akv/importance.py:19-164).

The per-key importance (the only pass over the attention weights) is
    imp[n] = sum_q mean_{b,h} attn[b, h, q, n]
computed by ``akv_importance_update``; OBSERVATION_WINDOW sums only the last
``observation_window`` queries and average-pools imp over ``pooling_kernel``
keys in the same kernel (akv/importance.py:96-115).  The accumulate strategies
(ATTENTION_ACCUMULATION, IMPORTANCE, OBSERVATION_WINDOW) fold imp into the EMA
    scores[:N] = scores[:N] * decay + imp
in that kernel too.  The other strategies (akv/importance.py:131-151) are small
operations on the (N,) score vector on the device: HEAVY_HITTER keeps the
running maximum, RECENCY_WEIGHTED and FIFO replace the scores by position,
HYBRID mixes the normalised EMA with recency.  The per-layer score vector grows
with zeros when the context grows (akv/importance.py:117-123).
"""
from __future__ import annotations

import ctypes
import logging
from dataclasses import dataclass
from enum import Enum
from typing import Optional

import torch

from . import _native as nat

logger = logging.getLogger(__name__)


class ScoringStrategy(str, Enum):
    ATTENTION_ACCUMULATION = "attention_accumulation"
    HEAVY_HITTER = "heavy_hitter"
    RECENCY_WEIGHTED = "recency_weighted"
    HYBRID = "hybrid"
    IMPORTANCE = "importance"
    FIFO = "fifo"
    OBSERVATION_WINDOW = "observation_window"


@dataclass
class ImportanceConfig:
    """akv/importance.py:30-43."""
    strategy: ScoringStrategy = ScoringStrategy.HYBRID
    decay_factor: float = 0.95
    recency_weight: float = 0.3
    attention_weight: float = 0.7
    window_size: int = 64
    initial_tokens_protected: int = 4
    recent_tokens_protected: int = 32
    observation_window: int = 32
    pooling_kernel: int = 7


_ACCUMULATE = (ScoringStrategy.ATTENTION_ACCUMULATION, ScoringStrategy.IMPORTANCE)


def accumulate(scores: torch.Tensor, attention_weights: torch.Tensor, decay: float,
               q_window: int = 0, pool_kernel: int = 1) -> torch.Tensor:
    """scores (n,) fp32 on the device, in place: scores = scores*decay + sum_q mean_{b,h} attn
    (truncated / zero-padded to n); q_window > 0 sums only the last q_window queries and
    pool_kernel > 1 average-pools the per-key sum first (OBSERVATION_WINDOW)."""
    nat.require_device(scores, attention_weights)
    lib = nat.load()
    B, H, M, N = attention_weights.shape
    attn = attention_weights
    if attn.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        attn = attn.float()
    attn = nat.dev_contig(attn)
    a = nat.ImportanceArgs()
    a.abi_version = nat.ABI_VERSION
    a.attn_dtype = nat.dtype_code(attn.dtype)
    a.attn = attn.data_ptr()
    a.B, a.H, a.M, a.N = B, H, M, N
    a.scores = scores.data_ptr()
    a.n_scores = scores.numel()
    a.decay = float(decay)
    a.q_window = int(q_window)
    a.pool_kernel = int(pool_kernel)
    nat.check(lib.akv_importance_update(ctypes.byref(a), nat.stream_of(scores)), "importance update")
    return scores


class ImportanceScorer:
    """Per-layer running importance scores (akv/importance.py:46-164)."""

    def __init__(self, config: Optional[ImportanceConfig] = None):
        self.config = config or ImportanceConfig()
        self._scores: dict[int, torch.Tensor] = {}
        self._step_count: int = 0
        self._total_seq_len: int = 0

    def reset(self):
        self._scores.clear()
        self._step_count = 0
        self._total_seq_len = 0

    @property
    def step_count(self) -> int:
        return self._step_count

    def update(self, attention_weights: Optional[torch.Tensor], layer_idx: int):
        """akv/importance.py:73-156: fold one step's attention weights (B, H, M, N) into
        the layer's scores."""
        if attention_weights is None:
            return
        cfg = self.config
        kv_len = attention_weights.shape[-1]
        device = attention_weights.device
        old = self._scores.get(layer_idx)
        if old is None or old.shape[0] < kv_len:
            new = torch.zeros(kv_len, dtype=torch.float32, device=device)
            if old is not None:
                new[: old.shape[0]] = old.to(device)
            self._scores[layer_idx] = new
        scores = self._scores[layer_idx]
        head = scores[:kv_len] if scores.shape[0] > kv_len else scores  # only the first kv_len entries change
        st = cfg.strategy
        if st in _ACCUMULATE:
            accumulate(head, attention_weights, cfg.decay_factor)
        elif st == ScoringStrategy.OBSERVATION_WINDOW:
            accumulate(head, attention_weights, cfg.decay_factor, q_window=cfg.observation_window,
                       pool_kernel=cfg.pooling_kernel)
        else:
            imp = accumulate(torch.zeros(kv_len, dtype=torch.float32, device=device), attention_weights, 0.0)
            if st == ScoringStrategy.HEAVY_HITTER:
                torch.maximum(head, imp, out=head)
            elif st == ScoringStrategy.RECENCY_WEIGHTED:
                head.copy_(torch.linspace(0, 1, kv_len, device=device))
            elif st == ScoringStrategy.HYBRID:
                head.mul_(cfg.decay_factor).add_(imp)
                recency = torch.linspace(0, 1, kv_len, device=device)
                head.copy_(cfg.attention_weight * head / head.max().clamp(min=1e-10) + cfg.recency_weight * recency)
            elif st == ScoringStrategy.FIFO:
                head.copy_(torch.arange(kv_len, dtype=torch.float32, device=device))
            else:
                raise ValueError(f"unknown strategy {st}")
        self._total_seq_len = max(self._total_seq_len, kv_len)
        self._step_count += 1

    def get_scores(self, layer_idx: int) -> Optional[torch.Tensor]:
        return self._scores.get(layer_idx)

    def get_aggregated_scores(self) -> Optional[torch.Tensor]:
        """akv/importance.py:174-188: the layers' scores, each zero-padded to the longest,
        averaged over layers (float32); None before any update."""
        if not self._scores:
            return None
        longest = max(int(s.shape[0]) for s in self._scores.values())
        dev = next(iter(self._scores.values())).device
        total = torch.zeros(longest, dtype=torch.float32, device=dev)
        for s in self._scores.values():
            total[: s.shape[0]] += s.to(device=dev, dtype=torch.float32)
        return total / len(self._scores)

    def get_tier_assignments(self, layer_idx: int, seq_len: int, hot_budget: int,
                             warm_budget: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """akv/importance.py:190-243: positions 0..seq_len-1 split into (hot, warm, cold),
        each ascending: the ``hot_budget`` most important, the next ``warm_budget``, the
        rest, with the first ``initial_tokens_protected`` and last
        ``recent_tokens_protected`` ranked above every scored position.  Without scores
        the split is by position.  Equal scores rank the lower index as less important,
        as ``get_eviction_candidates`` does (the reference's argsort leaves their order
        open)."""
        scores = self._scores.get(layer_idx)
        cfg = self.config
        if scores is None or seq_len == 0:
            pos = torch.arange(seq_len)
            h, w = min(hot_budget, seq_len), min(hot_budget + warm_budget, seq_len)
            return pos[:h], pos[h:w], pos[w:]
        s = scores[:seq_len].to(torch.float32).clone()
        n_start = min(cfg.initial_tokens_protected, s.shape[0])
        n_end = min(cfg.recent_tokens_protected, s.shape[0])
        s[:n_start] = float("inf")
        if n_end > 0:
            s[-n_end:] = float("inf")
        # least important first (stable: equal scores keep index order), read backwards
        rank = torch.sort(s, stable=True).indices.flip(0)
        total = rank.shape[0]
        h, w = min(hot_budget, total), min(hot_budget + warm_budget, total)
        return rank[:h].sort().values, rank[h:w].sort().values, rank[w:].sort().values

    def get_eviction_candidates(self, layer_idx: int, seq_len: int, num_to_evict: int) -> torch.Tensor:
        """akv/importance.py:245-300: ascending indices of the ``num_to_evict`` least
        important of the first ``seq_len`` positions, the first
        ``initial_tokens_protected`` and last ``recent_tokens_protected`` kept; FIFO takes
        the oldest unprotected positions without scores.  Equal scores go lowest index
        first (the reference's ``topk`` leaves their order open).  Empty (int64, on the
        scores' device, or the host with none) when nothing is evictable."""
        cfg = self.config
        scores = self._scores.get(layer_idx)
        dev = scores.device if scores is not None else torch.device("cpu")
        empty = torch.empty(0, dtype=torch.long, device=dev)
        if num_to_evict <= 0:
            return empty
        n_start = min(cfg.initial_tokens_protected, seq_len)
        n_end = min(cfg.recent_tokens_protected, seq_len)
        if cfg.strategy == ScoringStrategy.FIFO:
            n = min(num_to_evict, max(0, seq_len - n_end - n_start))
            return torch.arange(n_start, n_start + n, dtype=torch.long, device=dev) if n > 0 else empty
        if scores is None:
            return empty
        s = scores[:seq_len].clone()
        s[:n_start] = float("inf")
        if n_end > 0:
            s[-n_end:] = float("inf")
        n = min(num_to_evict, int((s != float("inf")).sum().item()))
        if n <= 0:
            return empty
        # the n smallest, ascending, equal scores lowest index first (one select launch)
        src = nat.dev_contig(scores[:seq_len], torch.float32)
        idx = torch.empty(n, dtype=torch.long, device=dev)
        nat.check(nat.load().akv_select_demote(src.data_ptr(), 1, src.numel(), n, n_start, n_end, idx.data_ptr(),
                                               nat.stream_of(src)), "get_eviction_candidates")
        return idx

    def stats(self) -> dict:
        return {
            "num_layers_tracked": len(self._scores),
            "step_count": self._step_count,
            "total_seq_len": self._total_seq_len,
        }
