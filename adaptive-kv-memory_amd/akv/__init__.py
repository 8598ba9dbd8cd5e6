"""akv -- MI355X-native warm-tier hot path of Adaptive KV Memory.

Module paths, names and signatures follow the reference package
(akv/__init__.py:47-63 re-exports the fused ops); every op runs hand-written
gfx950 kernels from libakv_hip.so.
"""
from .affine_quantizer import AffineQuantConfig, AffineQuantizer
from .baselines import KIVICache, KIVIConfig, KIVIFusedCache, KIVIFusedConfig, create_baseline
from .bitpack import pack, unpack, packed_bytes
from .drop_in import AKVCache, AKVLayer, _PRESETS, recommend_preset, select_demote_indices
from .fused_attention import fused_int4_decode_attention, mixed_precision_decode_attention
from .importance import ImportanceConfig, ImportanceScorer, ScoringStrategy
from .packed_layout import PackedKVArena, PackedKVConfig, PagedKVCache
from .production_cache import ProductionCache, ProductionCacheConfig
from .quantizer import KVQuantizer, QuantConfig, QuantizedTensor
from .triton_kernels import fused_decode_attention, fused_quantize_evict
from .triton_ops import (
    HAS_TRITON,
    fused_importance_update,
    fused_mixed_precision_attention,
    fused_quantized_attention,
)
from .warm_tier import WarmTier, decode_attention, dequantize, prefill_attention, quantize_kv

__version__ = "0.1.0"

__all__ = [
    "AffineQuantConfig", "AffineQuantizer", "pack", "unpack", "packed_bytes",
    "KIVICache", "KIVIConfig", "KIVIFusedCache", "KIVIFusedConfig", "create_baseline",
    "AKVCache", "AKVLayer", "_PRESETS", "recommend_preset", "select_demote_indices",
    "fused_int4_decode_attention", "mixed_precision_decode_attention",
    "ImportanceConfig", "ImportanceScorer", "ScoringStrategy",
    "PackedKVArena", "PackedKVConfig", "PagedKVCache", "ProductionCache", "ProductionCacheConfig",
    "KVQuantizer", "QuantConfig", "QuantizedTensor",
    "fused_decode_attention", "fused_quantize_evict",
    "HAS_TRITON", "fused_importance_update", "fused_mixed_precision_attention", "fused_quantized_attention",
    "WarmTier", "decode_attention", "dequantize", "prefill_attention", "quantize_kv",
]
