"""Reference-compatible decode / evict ops (akv/triton_kernels.py) on libakv_hip.so."""
from __future__ import annotations

import ctypes
import math
from typing import Optional

import torch

from . import _native as nat
from ._legacy import legacy_desc, padded_dim
from .warm_tier import run_decode

HAS_TRITON = False


def fused_decode_attention(
    query: torch.Tensor,
    key_hot: torch.Tensor,
    value_hot: torch.Tensor,
    key_warm_packed: Optional[torch.Tensor] = None,
    key_warm_scales: Optional[torch.Tensor] = None,
    key_warm_zeros: Optional[torch.Tensor] = None,
    value_warm_packed: Optional[torch.Tensor] = None,
    value_warm_scales: Optional[torch.Tensor] = None,
    value_warm_zeros: Optional[torch.Tensor] = None,
    bits: int = 4,
    group_size: int = 128,
    sm_scale: Optional[float] = None,
) -> torch.Tensor:
    """Single-query decode over hot (B, H, Nh, D) + shared warm tier, fp32
    softmax, output in the query dtype (akv/triton_kernels.py:281-387)."""
    B, H, M, D = query.shape
    assert M == 1, "Decode attention expects single query (M=1)"
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    desc = None
    keep = []
    if key_warm_packed is not None:
        N_warm = key_warm_scales.shape[0]
        desc = legacy_desc(key_warm_packed, key_warm_scales, key_warm_zeros, value_warm_packed,
                           value_warm_scales, value_warm_zeros, bits, group_size, N_warm, D,
                           warm_heads=1, keep=keep)
    out, _ = run_decode(query, key_hot, value_hot, desc, key_hot.shape[1], sm_scale, True)
    return out


def fused_quantize_evict(
    keys: torch.Tensor,
    values: torch.Tensor,
    evict_mask: torch.Tensor,
    bits: int = 4,
    group_size: int = 128,
):
    """Gather the masked rows and quantize them per token over groups of
    ``group_size`` channels in the input dtype; 4/2-bit codes packed, 3/8-bit
    one per byte (akv/triton_kernels.py:426-507).
    Returns (k_packed, k_scales, k_zeros, v_packed, v_scales, v_zeros)."""
    nat.require_device(keys, values, evict_mask)
    device = keys.device
    N, D = keys.shape
    evict_indices = evict_mask.nonzero(as_tuple=True)[0]
    n_evict = evict_indices.shape[0]
    if n_evict == 0:
        empty = torch.empty(0, device=device, dtype=torch.uint8)
        empty_f = torch.empty(0, device=device, dtype=keys.dtype)
        return empty, empty_f, empty_f, empty, empty_f, empty_f
    if bits not in (2, 3, 4, 8):
        raise ValueError(f"Unsupported bits: {bits}")
    if group_size not in (32, 64, 128):
        raise NotImplementedError("the MI355X evict quantizer takes group_size 32, 64 or 128")
    lib = nat.load()
    k = nat.dev_contig(keys)
    v = nat.dev_contig(values, keys.dtype)
    sel = nat.dev_contig(evict_indices, torch.int64)
    pD = padded_dim(D, group_size)
    G = pD // group_size
    sbits = bits if bits in (2, 4) else 8
    row = pD * sbits // 8
    kp = torch.empty(n_evict, row, dtype=torch.uint8, device=device)
    vp = torch.empty_like(kp)
    ks = torch.empty(n_evict, G, dtype=keys.dtype, device=device)
    kz, vs, vz = torch.empty_like(ks), torch.empty_like(ks), torch.empty_like(ks)
    a = nat.QuantArgs()
    a.abi_version = nat.ABI_VERSION
    a.B, a.H, a.D = 1, 1, D
    a.in_dtype = nat.dtype_code(keys.dtype)
    a.layout = nat.QUANT_TOKEN_GROUPS
    a.k, a.v = k.data_ptr(), v.data_ptr()
    a.n_src = N
    a.sel = sel.data_ptr()
    a.n_sel = n_evict
    a.bits_k = a.bits_v = bits
    a.block_t = 32
    a.group_v = group_size
    a.k_codes, a.k_scale, a.k_zero = kp.data_ptr(), ks.data_ptr(), kz.data_ptr()
    a.v_codes, a.v_scale, a.v_zero = vp.data_ptr(), vs.data_ptr(), vz.data_ptr()
    nat.check(lib.akv_quant_pack(ctypes.byref(a), nat.stream_of(k)), "fused_quantize_evict")
    return kp, ks, kz, vp, vs, vz
