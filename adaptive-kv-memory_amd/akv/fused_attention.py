"""Per-head int4 decode ops (akv/fused_attention.py) on libakv_hip.so.

``fused_int4_decode_attention`` and ``mixed_precision_decode_attention`` take
a per-head warm tier (H, N, D/2) uint8 + (H, N, G) scales shared by the batch;
dequant is fp32 ``u*s + z`` cast to fp16 and attention is fp32
(akv/fused_attention.py:213-366).  The reference's memory-limit switch between
a batched and a tiled torch path has no counterpart: one kernel serves both.
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from ._legacy import legacy_desc
from .warm_tier import run_decode

HAS_TRITON = False


def _int4_group(D: int, group_size: int, G: int) -> int:
    # _dequant_int4_tile indexes scales[..., arange(D) // group_size]
    if group_size >= D:
        return D
    if D % group_size:
        raise NotImplementedError("group_size must divide head_dim")
    if G < D // group_size:
        raise ValueError("scales hold fewer groups than head_dim // group_size")
    return group_size


def _int4_desc(kp, ks, kz, vp, vs, vz, D, group_size, keep):
    H, N, _ = kp.shape
    G = ks.shape[-1]
    gs = _int4_group(D, group_size, G)
    ng = D // gs
    ks, kz, vs, vz = (m[..., :ng] for m in (ks, kz, vs, vz))
    return legacy_desc(kp, ks, kz, vp, vs, vz, 4, gs, N, D, warm_heads=H, sym=0, keep=keep)


def fused_int4_decode_attention(
    query: torch.Tensor,
    k_packed: torch.Tensor,
    k_scales: torch.Tensor,
    k_zeros: torch.Tensor,
    v_packed: torch.Tensor,
    v_scales: torch.Tensor,
    v_zeros: torch.Tensor,
    group_size: int = 128,
    memory_limit_mb: float = 512.0,
) -> torch.Tensor:
    """akv/fused_attention.py:213-278 -> (B, H, 1, D) in the query dtype."""
    B, H, _, D = query.shape
    keep = []
    desc = _int4_desc(k_packed, k_scales, k_zeros, v_packed, v_scales, v_zeros, D, group_size, keep)
    out, _ = run_decode(query, None, None, desc, H, 1.0 / math.sqrt(D), True)
    return out


def mixed_precision_decode_attention(
    query: torch.Tensor,
    hot_keys: torch.Tensor,
    hot_values: torch.Tensor,
    warm_k_packed: Optional[torch.Tensor] = None,
    warm_k_scales: Optional[torch.Tensor] = None,
    warm_k_zeros: Optional[torch.Tensor] = None,
    warm_v_packed: Optional[torch.Tensor] = None,
    warm_v_scales: Optional[torch.Tensor] = None,
    warm_v_zeros: Optional[torch.Tensor] = None,
    group_size: int = 128,
) -> torch.Tensor:
    """Hot fp16 + per-head int4 warm, hot first (akv/fused_attention.py:324-366)."""
    B, H, _, D = query.shape
    desc = None
    keep = []
    if warm_k_packed is not None and warm_k_packed.shape[1] > 0:
        desc = _int4_desc(warm_k_packed, warm_k_scales, warm_k_zeros, warm_v_packed, warm_v_scales,
                          warm_v_zeros, D, group_size, keep)
    out, _ = run_decode(query, hot_keys, hot_values, desc, H, 1.0 / math.sqrt(D), True)
    return out


def fused_decode_attention(query, keys_quantized, values_quantized, quantizer):
    """Compatibility wrapper over KVQuantizer tensors (akv/fused_attention.py:373-390):
    the quantized K/V of shape (B, H, N, D) become a per-(batch, head) legacy warm
    tier and go through the same kernel."""
    B, H, M, D = query.shape
    kq, vq = keys_quantized, values_quantized
    N = kq.shape[-2]
    rows = B * H
    keep = []
    desc = legacy_desc(kq.data, kq.scales.reshape(rows * N, -1), kq.zeros.reshape(rows * N, -1),
                       vq.data, vq.scales.reshape(rows * N, -1), vq.zeros.reshape(rows * N, -1),
                       kq.bits, kq.group_size, N, D, warm_heads=rows, sym=-1, keep=keep)
    q = query.reshape(1, rows, M, D)
    out, _ = run_decode(q, None, None, desc, rows, 1.0 / math.sqrt(D), True)
    return out.reshape(B, H, M, D)


def fused_quantize_evict(keys, values, scores, evict_mask, quantizer):
    """Compatibility wrapper (akv/fused_attention.py:393-401)."""
    evict_idx = evict_mask.nonzero(as_tuple=True)[0]
    if evict_idx.numel() == 0:
        return None, None
    k_evict = keys[:, :, evict_idx, :]
    v_evict = values[:, :, evict_idx, :]
    return quantizer.quantize(k_evict), quantizer.quantize(v_evict)
