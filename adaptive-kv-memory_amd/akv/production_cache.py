"""ProductionCache (akv/production_cache.py) on the device.

Per layer: an fp16 hot tier in one device buffer per K and V (the reference keeps it
twice, in a page pool and a contiguous copy), and a warm tier of two
``PackedKVArena``s (K and V) in the reference's per-token-group layout.  ``update``
follows the reference's rules (akv/production_cache.py:360-405): append, importance from
attention weights when given, and an amortised migration (every 8 calls, or with
weights, or over budget) that demotes the scorer's eviction candidates into the
arenas.  ``fused_attention`` is one ``akv_decode_attn`` launch for all batch elements
that reads the packed arenas and the hot buffer in place (both through their token
strides), so no float16 copy of the warm tier is built or kept; the reference instead
dequantizes the arena into a cached float16 buffer and runs torch matmuls over it
(:429-469).  ``get_kv`` keeps the reference's cached float16 view for callers that
want dense tensors.

Differences on purpose: the migration runs on the caller's stream (the
reference's high-priority side stream is not synchronised with the reads that
follow it, akv/production_cache.py:498-502); ``fused_attention`` takes the
``sm_scale`` keyword its vLLM caller passes (akv/vllm_integration.py:332);
``ProductionLayerCache.reset`` also empties the hot buffer (the reference's leaves
its contiguous copy's length, :310-320); equal importance scores are demoted
lowest index first (the reference's ``topk`` leaves the order open); and the
TurboQuant warm tier (``warm_quantizer="turbo"``, akv/turbo_quant.py) is not part of
this build -- ``"minmax"`` selects the arenas.
"""
from __future__ import annotations

import ctypes
import logging
from dataclasses import dataclass
from typing import Optional

import torch

from . import _native as nat
from .importance import ImportanceConfig, ImportanceScorer, ScoringStrategy
from .packed_layout import PackedKVArena, PackedKVConfig

logger = logging.getLogger(__name__)


@dataclass
class ProductionCacheConfig:
    """akv/production_cache.py:33-70."""
    num_layers: int = 32
    num_heads: int = 32
    head_dim: int = 128
    hot_budget: int = 1024
    warm_budget: int = 4096
    cold_budget: int = 16384
    warm_bits: int = 3
    cold_bits: int = 2
    group_size: int = 64
    warm_quantizer: str = "turbo"
    page_size: int = 16
    max_hot_pages: int = 2048
    use_async_migration: bool = True
    migration_threshold: float = 0.9
    batch_migration_size: int = 64
    importance_decay: float = 0.3
    protect_initial: int = 4
    protect_recent: int = 32
    n_anchors: int = 16
    scoring_strategy: str = "importance"
    device: str = "cuda"
    dtype: torch.dtype = torch.float16


class ProductionLayerCache:
    """One layer of akv/production_cache.py:73-320 (the minmax warm tier).

    The hot tier is one device buffer per K and V, (heads, max_hot_pages * page_size,
    head_dim) fp16, filled from the front: it is what ``fused_attention``'s decode launch
    reads (token stride = its capacity), so the layer keeps no second copy of it.  The
    reference keeps the same tokens twice, in a page pool and in a contiguous buffer; its
    pages are accounted here from the hot length (ceil(hot_len / page_size) pages, which is
    what its pool holds after every append and compaction), and running out of them raises
    the reference's "Page pool exhausted".  Demotion compacts the buffer on the device: one
    stable sort of the kept-token mask gives the kept positions in order (no host sync; the
    candidate indices are distinct), then one gather and one copy per tensor.  The warm tier
    is two ``PackedKVArena``s read in place by the decode kernel; ``get_warm_fp16`` keeps
    the reference's cached float16 view for callers that want dense tensors."""

    def __init__(self, config: ProductionCacheConfig, layer_idx: int):
        self.config = config
        self.layer_idx = layer_idx
        self.device = config.device
        if config.warm_quantizer == "turbo":
            raise NotImplementedError("the TurboQuant warm tier (akv/turbo_quant.py) is not part of this build; "
                                      "use warm_quantizer='minmax' (PackedKVArena)")
        arena_cfg = PackedKVConfig(max_seq_len=config.warm_budget, num_heads=config.num_heads,
                                   head_dim=config.head_dim, bits=config.warm_bits, group_size=config.group_size,
                                   device=config.device, dtype=config.dtype)
        self._warm_k = PackedKVArena(arena_cfg)
        self._warm_v = PackedKVArena(arena_cfg)
        self._warm_fp16: Optional[tuple[torch.Tensor, torch.Tensor]] = None  # cached dequantized view
        H, D = config.num_heads, config.head_dim
        self._hot_k = torch.zeros(H, config.max_hot_pages * config.page_size, D, dtype=torch.float16,
                                  device=config.device)
        self._hot_v = torch.zeros_like(self._hot_k)
        self._hot_len = 0
        self._seq_len = 0
        self._ws = nat.DecodeWorkspace()  # decode workspace, reused across calls

    @property
    def hot_len(self) -> int:
        return self._hot_len

    @property
    def warm_len(self) -> int:
        return self._warm_k.length

    @property
    def seq_len(self) -> int:
        return self._seq_len

    @property
    def hot_capacity(self) -> int:
        return self._hot_k.shape[1]

    def append_hot(self, keys: torch.Tensor, values: torch.Tensor):
        """keys / values (heads, N, head_dim) after the hot tier's last token."""
        n, a = int(keys.shape[1]), self._hot_len
        if a + n > self.hot_capacity:
            raise RuntimeError("Page pool exhausted")
        self._hot_k[:, a:a + n] = keys
        self._hot_v[:, a:a + n] = values
        self._hot_len = a + n
        self._seq_len += n

    def get_hot_kv(self) -> tuple[torch.Tensor, torch.Tensor]:
        """Views (heads, hot_len, head_dim) of the hot buffer."""
        return self._hot_k[:, :self._hot_len], self._hot_v[:, :self._hot_len]

    def get_warm_fp16(self) -> tuple[Optional[torch.Tensor], Optional[torch.Tensor]]:
        """The dequantized warm tier (heads, N_warm, head_dim), rebuilt only after a demotion."""
        n = self._warm_k.length
        if n == 0:
            return None, None
        if self._warm_fp16 is None:
            self._warm_fp16 = (self._warm_k.dequantize_slice(0, n), self._warm_v.dequantize_slice(0, n))
        return self._warm_fp16

    def get_warm_packed(self):
        n = self._warm_k.length
        if n == 0:
            return None, None, None, None, None, None
        return self._warm_k.get_packed_slice(0, n) + self._warm_v.get_packed_slice(0, n)

    def demote_to_warm(self, indices: torch.Tensor, keys: torch.Tensor, values: torch.Tensor):
        """Quantize the demoted tokens into the arenas, then drop them from the hot tier."""
        self._warm_k.quantize_and_append(keys)
        self._warm_v.quantize_and_append(values)
        self._warm_fp16 = None
        self._compact_hot(indices)

    def _compact_hot(self, remove_indices: torch.Tensor):
        n = self._hot_len
        if n == 0:
            return
        idx = remove_indices.to(self._hot_k.device, torch.int64)
        n_keep = n - int(idx.numel())
        removed = torch.zeros(n, dtype=torch.int8, device=self._hot_k.device)
        removed.index_fill_(0, idx, 1)
        # stable: the kept positions (key 0) come first, in increasing order
        kept = torch.sort(removed, stable=True).indices[:n_keep]
        for buf in (self._hot_k, self._hot_v):
            buf[:, :n_keep] = buf.index_select(1, kept)
        self._hot_len = n_keep

    def memory_usage(self) -> dict:
        cfg = self.config
        pages = -(-self._hot_len // cfg.page_size)
        hot_bytes = pages * cfg.num_heads * cfg.page_size * cfg.head_dim * 2 * 2
        warm_bytes = self._warm_k.bytes_used + self._warm_v.bytes_used
        return {"hot_mb": hot_bytes / 1e6, "warm_mb": warm_bytes / 1e6, "total_mb": (hot_bytes + warm_bytes) / 1e6}

    def reset(self):
        self._warm_k.reset()
        self._warm_v.reset()
        self._warm_fp16 = None
        self._hot_len = 0
        self._seq_len = 0

    def attention(self, query: torch.Tensor, sm_scale: Optional[float] = None) -> torch.Tensor:
        """softmax(q K^T * sm_scale) V over [warm, hot] for query (B, H, M, D), sm_scale D^-0.5
        unless given, float16 out.  Every batch element attends to the layer's one cache, so the
        B x M query rows of a head go to one decode launch as B * M rows (the kernel shares each
        dequantized tile between a head's rows); it reads the arenas' packed rows in place
        (legacy layout, per head, token stride = the arena's capacity) and the hot buffer
        (token stride = its capacity)."""
        cfg = self.config
        H, D = cfg.num_heads, cfg.head_dim
        if D % cfg.group_size:
            raise NotImplementedError("fused_attention reads the arena in place, which needs group_size | head_dim")
        B, Hq, M, _ = query.shape
        # (B, Hq, M, D) -> (1, Hq, B*M, D): row b*M + m of a head is query (b, m)
        q = query.to(torch.float16)
        q = q.transpose(0, 1).reshape(1, Hq, B * M, D).contiguous() if B > 1 else nat.dev_contig(q)
        n_hot, n_warm = self._hot_len, self._warm_k.length
        if n_hot + n_warm == 0:
            raise RuntimeError("fused_attention on an empty layer")
        out = torch.empty_like(q)
        a = nat.DecodeArgs()
        a.abi_version = nat.ABI_VERSION
        a.B, a.Hq, a.Hkv, a.M, a.D = 1, Hq, H, B * M, D
        a.q_dtype = nat.DT_F16
        a.q = q.data_ptr()
        if n_hot:
            a.k_hot, a.v_hot = self._hot_k.data_ptr(), self._hot_v.data_ptr()
        a.n_hot = n_hot
        a.hot_stride = self.hot_capacity
        a.hot_first = 0
        a.sm_scale = D ** -0.5 if sm_scale is None else float(sm_scale)
        if n_warm:
            w = a.warm
            w.kind = nat.WARM_LEGACY
            w.bits_k = w.bits_v = cfg.warm_bits
            w.n_warm = n_warm
            w.token_stride = self._warm_k.capacity
            w.k_codes, w.v_codes = self._warm_k.data.data_ptr(), self._warm_v.data.data_ptr()
            w.k_scale, w.k_zero = self._warm_k.scales.data_ptr(), self._warm_k.zeros.data_ptr()
            w.v_scale, w.v_zero = self._warm_v.scales.data_ptr(), self._warm_v.zeros.data_ptr()
            w.group_size = cfg.group_size
            w.meta_dtype = nat.dtype_code(self._warm_k.scales.dtype)
            w.warm_heads = H
            w.legacy_sym = 0  # dequantize_slice has no symmetric branch
        else:
            a.warm.kind = nat.WARM_NONE
        a.out = out.data_ptr()
        lib = nat.load()
        nbytes = lib.akv_decode_workspace_bytes(ctypes.byref(a))
        if nbytes < 0:
            nat.check(lib.akv_decode_attn(ctypes.byref(a), None), "ProductionCache.fused_attention")
        # the layer's workspace, kept across calls (calls on one layer are ordered on one stream)
        ws = self._ws.get(nbytes, lib.akv_decode_counter_bytes(ctypes.byref(a)), q.device)
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
        nat.check(lib.akv_decode_attn(ctypes.byref(a), nat.stream_of(q)), "ProductionCache.fused_attention")
        if B > 1:
            out = out.reshape(Hq, B, M, D).transpose(0, 1).contiguous()
        return out


class ProductionCache:
    """akv/production_cache.py:323-541."""

    def __init__(self, config: Optional[ProductionCacheConfig] = None):
        self.config = config or ProductionCacheConfig()
        cfg = self.config
        self._layers = [ProductionLayerCache(cfg, i) for i in range(cfg.num_layers)]
        self._scorer = ImportanceScorer(ImportanceConfig(
            strategy=ScoringStrategy(cfg.scoring_strategy), decay_factor=cfg.importance_decay,
            initial_tokens_protected=cfg.protect_initial, recent_tokens_protected=cfg.protect_recent))
        self._migration_stream = None  # migrations are ordered on the caller's stream
        self._decode_count = 0
        self._migration_count = 0
        self._total_demoted = 0

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int,
               attention_weights: Optional[torch.Tensor] = None) -> tuple[torch.Tensor, torch.Tensor]:
        """akv/production_cache.py:360-405."""
        nat.require_device(key_states, value_states)
        keys = key_states.squeeze(0) if key_states.dim() == 4 else key_states
        values = value_states.squeeze(0) if value_states.dim() == 4 else value_states
        layer = self._layers[layer_idx]
        layer.append_hot(keys, values)
        if attention_weights is not None:
            self._scorer.update(attention_weights, layer_idx)
        self._decode_count += 1
        if (self._decode_count % 8 == 0 or attention_weights is not None
                or layer.hot_len > self.config.hot_budget):
            if layer.hot_len > self.config.hot_budget * self.config.migration_threshold:
                self._maybe_migrate(layer_idx)
        return self.get_kv(layer_idx)

    def get_kv(self, layer_idx: int) -> tuple[torch.Tensor, torch.Tensor]:
        """akv/production_cache.py:407-427: (1, H, N_warm + N_hot, D), warm tokens first."""
        layer = self._layers[layer_idx]
        hot = layer.get_hot_kv()
        warm = layer.get_warm_fp16()
        if warm[0] is None:
            return hot[0].unsqueeze(0), hot[1].unsqueeze(0)
        return tuple(torch.cat([w, h], dim=1).unsqueeze(0) for w, h in zip(warm, hot))

    def fused_attention(self, query: torch.Tensor, layer_idx: int, sm_scale: Optional[float] = None) -> torch.Tensor:
        """akv/production_cache.py:429-469 for query (B, H, M, D): attention over the
        layer's warm and hot tiers, float16 out, one decode launch (every batch element
        attends to the layer's one cache, as the reference's broadcast does).  ``sm_scale`` (default
        D^-0.5) is the keyword the reference's vLLM backend passes
        (akv/vllm_integration.py:332) and its method lacks."""
        nat.require_device(query)
        return self._layers[layer_idx].attention(query, sm_scale)

    def _maybe_migrate(self, layer_idx: int):
        """akv/production_cache.py:471-505, on the caller's stream: while the hot tier is over
        its budget, demote up to batch_migration_size of the scorer's eviction candidates."""
        layer, cfg = self._layers[layer_idx], self.config
        excess = layer.hot_len - cfg.hot_budget
        if excess <= 0:
            return
        n_demote = min(cfg.batch_migration_size, excess)
        cand = self._scorer.get_eviction_candidates(layer_idx, layer.hot_len, n_demote)
        if cand.numel() == 0:
            return
        k, v = layer.get_hot_kv()
        cand = cand.to(k.device, torch.int64)
        layer.demote_to_warm(cand, k.index_select(1, cand), v.index_select(1, cand))
        self._migration_count += 1
        self._total_demoted += n_demote

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self._layers[layer_idx].seq_len if layer_idx < len(self._layers) else 0

    def memory_usage(self) -> dict:
        hot = warm = 0.0
        for layer in self._layers:
            u = layer.memory_usage()
            hot += u["hot_mb"]
            warm += u["warm_mb"]
        return {"hot_mb": hot, "warm_mb": warm, "total_mb": hot + warm, "num_layers": len(self._layers),
                "decode_count": self._decode_count, "migrations": self._migration_count,
                "total_demoted": self._total_demoted}

    def reset(self):
        for layer in self._layers:
            layer.reset()
        self._scorer.reset()
        self._decode_count = self._migration_count = self._total_demoted = 0

    def __len__(self):
        return len(self._layers)

    def __getitem__(self, layer_idx):
        return self.get_kv(layer_idx)
