"""Reference-compatible fused ops (akv/triton_ops.py), lowered to libakv_hip.so.

Same names, signatures, defaults, return types and in-place semantics as the
reference module.  ``HAS_TRITON`` is kept as a constant for import
compatibility and is never used for dispatch: every op runs the hand-written
gfx950 kernels, and raises for tensors that are not on a ROCm device.
"""
from __future__ import annotations

import ctypes
import math
from typing import Optional

import torch

from . import _native as nat
from ._legacy import legacy_desc
from .warm_tier import run_decode

HAS_TRITON = False


def fused_quantized_attention(
    query: torch.Tensor,
    key_packed: torch.Tensor,
    key_scales: torch.Tensor,
    key_zeros: torch.Tensor,
    value_packed: torch.Tensor,
    value_scales: torch.Tensor,
    value_zeros: torch.Tensor,
    bits: int = 4,
    group_size: int = 128,
    sm_scale: Optional[float] = None,
) -> torch.Tensor:
    """softmax(Q . deq(K)^T * s) . deq(V) with the warm tier shared across (B, H)
    (akv/triton_ops.py:330-377; N = key_scales.shape[0])."""
    B, H, M, D = query.shape
    N = key_scales.shape[0]
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    keep = []
    desc = legacy_desc(key_packed, key_scales, key_zeros, value_packed, value_scales, value_zeros,
                       bits, group_size, N, D, warm_heads=1, keep=keep)
    out, _ = run_decode(query, None, None, desc, H, sm_scale, True)
    return out


def fused_mixed_precision_attention(
    query: torch.Tensor,
    key_hot: torch.Tensor,
    value_hot: torch.Tensor,
    key_warm_packed: torch.Tensor,
    key_warm_scales: torch.Tensor,
    key_warm_zeros: torch.Tensor,
    value_warm_packed: torch.Tensor,
    value_warm_scales: torch.Tensor,
    value_warm_zeros: torch.Tensor,
    bits: int = 4,
    group_size: int = 128,
    sm_scale: Optional[float] = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Exact attention over [hot, warm] (hot first); returns (out, attn_weights fp32)
    (akv/triton_ops.py:466-515, :554-601)."""
    B, H, M, D = query.shape
    N_warm = key_warm_scales.shape[0]
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    keep = []
    desc = legacy_desc(key_warm_packed, key_warm_scales, key_warm_zeros, value_warm_packed, value_warm_scales,
                       value_warm_zeros, bits, group_size, N_warm, D, warm_heads=1, keep=keep)
    return run_decode(query, key_hot, value_hot, desc, key_hot.shape[1], sm_scale, True, return_weights=True)


def fused_importance_update(
    attention_weights: torch.Tensor,
    scores: torch.Tensor,
    decay: float = 0.95,
) -> torch.Tensor:
    """scores = scores*decay + (mean over batch/heads, summed over queries) of the
    weights, truncated / zero-padded to len(scores); in place, returned
    (akv/triton_ops.py:604-650, torch-path semantics)."""
    nat.require_device(attention_weights, scores)
    lib = nat.load()
    B, H, M, N = attention_weights.shape
    attn = attention_weights
    if attn.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        attn = attn.float()
    attn = nat.dev_contig(attn)
    direct = scores.dtype == torch.float32 and scores.is_contiguous() and scores.data_ptr() % 16 == 0
    buf = scores if direct else nat.dev_contig(scores, torch.float32).clone()
    a = nat.ImportanceArgs()
    a.abi_version = nat.ABI_VERSION
    a.attn_dtype = nat.dtype_code(attn.dtype)
    a.attn = attn.data_ptr()
    a.B, a.H, a.M, a.N = B, H, M, N
    a.scores = buf.data_ptr()
    a.n_scores = buf.numel()
    a.decay = float(decay)
    nat.check(lib.akv_importance_update(ctypes.byref(a), nat.stream_of(buf)), "fused_importance_update")
    if not direct:
        scores.copy_(buf.view_as(scores))
    return scores


def _dequantize_packed(
    packed: torch.Tensor,
    scales: torch.Tensor,
    zeros: torch.Tensor,
    bits: int,
    group_size: int,
    N: int,
    D: int,
    device: torch.device,
    dtype: torch.dtype,
) -> torch.Tensor:
    """Legacy per-token-group dequant to (N, D) ``dtype`` (akv/triton_ops.py:657-713)."""
    if bits not in (2, 4, 8):
        raise ValueError(f"Unsupported bits: {bits}")
    lib = nat.load()
    packed = packed.to(device)
    keep = []
    desc = legacy_desc(packed, scales.to(device), zeros.to(device), packed, scales.to(device), zeros.to(device),
                       bits, group_size, N, D, warm_heads=1, sym=-1, keep=keep)
    out = torch.empty(N, D, dtype=dtype, device=packed.device)
    ws = nat.workspace(256, packed.device)
    a = nat.DequantArgs()
    a.abi_version = nat.ABI_VERSION
    a.B, a.Hkv, a.D = 1, 1, D
    a.out_dtype = nat.dtype_code(dtype)
    a.warm = desc
    a.k_out = out.data_ptr()
    a.workspace = ws.data_ptr()
    nat.check(lib.akv_dequant_unpack(ctypes.byref(a), nat.stream_of(out)), "_dequantize_packed")
    return out
