"""AKVCache presets and the demotion primitives of the drop-in cache.

``_PRESETS`` and the preset resolution of ``AKVCache.__init__`` follow
akv/drop_in.py:89-124 and :910-964.  Demotion follows ``AKVLayer``:
``select_demote_indices`` is akv/drop_in.py:392-413 (first 4 and last
min(16, hot_budget // 4) hot tokens protected, lowest scores first, indices
returned in ascending order) and ``demote`` gathers the selected tokens and
quantizes them into the packed warm tier on the device (the reference's
_quantize_per_head at akv/drop_in.py:315-374 quantizes and immediately
dequantizes back to fp16; here the packed codes are what is kept).
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _native as nat
from .warm_tier import WarmTier, quantize_kv

_PRESETS = {
    "quality": {
        "warm_bits": 4,
        "hot_budget": 256,
        "description": "Near-lossless 4-bit. +1-2% PPL.",
    },
    "balanced": {
        "warm_bits": 3,
        "hot_budget": 128,
        "description": "Block-affine 3-bit. +3.3% PPL, 5x compression.",
    },
    "compact": {
        "warm_bits": 2,
        "hot_budget": 64,
        "description": "Block-affine 2-bit. +11% PPL, 8x compression.",
    },
    "k4v2": {
        "warm_bits": 4,
        "warm_key_bits": 4,
        "warm_value_bits": 2,
        "hot_budget": 128,
        "description": "Asymmetric K4/V2. Keys preserved, values aggressively compressed.",
    },
    "k4v3": {
        "warm_bits": 4,
        "warm_key_bits": 4,
        "warm_value_bits": 3,
        "hot_budget": 128,
        "description": "Asymmetric K4/V3. Near-quality keys with balanced value compression.",
    },
}


def select_demote_indices(importance: Optional[torch.Tensor], n_demote: int, hot_len: int,
                          hot_budget: int, device=None) -> torch.Tensor:
    """akv/drop_in.py:392-413 on the device (importance (hot_len,) or (B, hot_len)).

    With no scores, or scores of another length, the reference falls back to FIFO
    (``arange(n_demote)``, akv/drop_in.py:401-403); that index lands on ``device``
    (else on the scores' device), where the gather that consumes it runs."""
    if importance is None or importance.shape[-1] != hot_len:
        dev = device if device is not None else (importance.device if importance is not None else None)
        if dev is None:
            raise ValueError("select_demote_indices: no scores and no device for the FIFO fallback")
        return torch.arange(n_demote, device=dev)
    nat.require_device(importance)
    if not 0 <= n_demote <= hot_len:
        raise ValueError(f"n_demote {n_demote} outside [0, {hot_len}]")
    protect_initial = 4
    protect_recent = min(16, hot_budget // 4)
    scores = nat.dev_contig(importance, torch.float32)
    rows = scores.numel() // hot_len if hot_len else 0
    idx = torch.empty(importance.shape[:-1] + (n_demote,), dtype=torch.int64, device=importance.device)
    lib = nat.load()
    nat.check(lib.akv_select_demote(scores.data_ptr(), rows, hot_len, n_demote, protect_initial, protect_recent,
                                    idx.data_ptr(), nat.stream_of(scores)), "select_demote_indices")
    return idx


def quantize_per_head(k: torch.Tensor, v: torch.Tensor, key_bits: int = 3, value_bits: int = 3,
                      per_head_bits: Optional[list] = None, group_size: int = 64,
                      outlier_fraction: float = 0.0) -> tuple[torch.Tensor, torch.Tensor, int]:
    """AKVLayer._quantize_per_head (akv/drop_in.py:315-374) on the device.

    k, v (B, H, n, D): one AffineQuantizer call per batch element over the n tokens
    (K per channel, V per token, outliers shared by the heads) -- or, when
    ``per_head_bits`` names a width for each head, one call per (batch element, head)
    with a quantizer of that width for K and V (the reference's pool keyed by bits;
    a head-count mismatch falls back to the global widths).  Returns the dequantized
    K, V (fp16, bit-exact with the reference) and the measured packed bytes of the
    event (packed_layout.measure_packed_bytes).  The reference squeezes a batch of
    one; here each batch element is its own call."""
    from .affine_quantizer import AffineQuantConfig, AffineQuantizer
    from .packed_layout import measure_packed_bytes
    nat.require_device(k, v)
    B, H, n, D = k.shape
    out_k = torch.empty(B, H, n, D, dtype=torch.float16, device=k.device)
    out_v = torch.empty_like(out_k)
    packed = 0
    if not per_head_bits or len(per_head_bits) != H:
        qz = AffineQuantizer(AffineQuantConfig(key_bits=key_bits, value_bits=value_bits, group_size=group_size,
                                               outlier_fraction=outlier_fraction))
        for b in range(B):
            qk, qv = qz.quantize_keys(k[b]), qz.quantize_values(v[b])
            packed += measure_packed_bytes(qk, key_bits) + measure_packed_bytes(qv, value_bits)
            out_k[b] = qz.dequantize_keys(qk)
            out_v[b] = qz.dequantize_values(qv)
        return out_k, out_v, packed
    pool = {}
    for bits in set(per_head_bits):
        pool[bits] = AffineQuantizer(AffineQuantConfig(key_bits=bits, value_bits=bits, group_size=group_size,
                                                       outlier_fraction=outlier_fraction))
    for b in range(B):
        for h, bits in enumerate(per_head_bits):
            qz = pool[bits]
            qk, qv = qz.quantize_keys(k[b, h:h + 1]), qz.quantize_values(v[b, h:h + 1])
            packed += measure_packed_bytes(qk, bits) + measure_packed_bytes(qv, bits)
            out_k[b, h] = qz.dequantize_keys(qk)[0]
            out_v[b, h] = qz.dequantize_values(qv)[0]
    return out_k, out_v, packed


class AKVCache:
    """Preset resolution and warm-tier settings of the drop-in cache
    (akv/drop_in.py:885-964).  The HF ``DynamicCache`` wiring is not part of
    this build; ``demote`` is the warm-tier hot path it drives."""

    def __init__(self, preset: Optional[str] = None, warm_bits: Optional[int] = None,
                 warm_key_bits: Optional[int] = None, warm_value_bits: Optional[int] = None,
                 hot_budget: Optional[int] = None, group_size: int = 64, outlier_fraction: float = 0.0,
                 protect_first: int = 0, protect_last: int = 0, protect_layers: Optional[list] = None,
                 num_hidden_layers: Optional[int] = None, enable_promotion: bool = True,
                 promotion_threshold: float = 0.05, enable_promotion_proxy: bool = True,
                 proxy_decay: float = 0.7, adaptive_hot_frac: float = 0.0,
                 block_t: int = 32, group_v: int = 32):
        if preset is not None:
            if preset not in _PRESETS:
                raise ValueError(f"Unknown preset {preset!r}. Choose from: {sorted(_PRESETS.keys())}")
            if warm_bits is not None or hot_budget is not None:
                raise ValueError(
                    "preset= is mutually exclusive with warm_bits/hot_budget. "
                    "Pick a preset OR pass explicit params.")
            p = _PRESETS[preset]
            self.warm_bits = p["warm_bits"]
            self.hot_budget = p["hot_budget"]
        else:
            self.warm_bits = warm_bits or 3
            self.hot_budget = hot_budget or 128
        if preset and "warm_key_bits" in _PRESETS.get(preset, {}):
            self.warm_key_bits = _PRESETS[preset]["warm_key_bits"]
            self.warm_value_bits = _PRESETS[preset]["warm_value_bits"]
        else:
            self.warm_key_bits = warm_key_bits or self.warm_bits
            self.warm_value_bits = warm_value_bits or self.warm_bits
        self.preset = preset
        self.group_size = group_size
        self.outlier_fraction = outlier_fraction
        self.num_hidden_layers = num_hidden_layers
        self.enable_promotion = enable_promotion
        self.promotion_threshold = promotion_threshold
        self.enable_promotion_proxy = enable_promotion_proxy
        self.proxy_decay = proxy_decay
        self.adaptive_hot_frac = adaptive_hot_frac
        self._protect_first = protect_first
        self._protect_last = protect_last
        self._protect_explicit = list(protect_layers) if protect_layers else []
        self.block_t = block_t
        self.group_v = group_v

    def demote(self, keys: torch.Tensor, values: torch.Tensor, importance: Optional[torch.Tensor],
               n_demote: int) -> tuple[WarmTier, torch.Tensor]:
        """Pick ``n_demote`` hot tokens per sequence (lowest importance, protected
        ends kept) and quantize them into a packed warm tier.

        keys / values: (B, H, hot_len, D) on the device; importance: (B, hot_len)
        or (hot_len,).  Returns (warm tier, selected indices (B, n_demote))."""
        B, H, hot_len, D = keys.shape
        idx = select_demote_indices(importance, n_demote, hot_len, self.hot_budget, device=keys.device)
        if idx.dim() == 1:
            idx = idx.unsqueeze(0).expand(B, -1)
        warm = quantize_kv(keys, values, self.warm_key_bits, self.warm_value_bits, self.block_t,
                           self.group_v, self.outlier_fraction, sel=idx)
        return warm, idx
