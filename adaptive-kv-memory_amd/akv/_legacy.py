"""Descriptor for the reference's legacy per-token-group warm tier.

The reference's public attention ops take the warm tier as a flat uint8
buffer of per-token rows plus (N, G) scales / zeros, shared by every batch
element and head (akv/triton_ops.py:657-713), or one per head
(akv/fused_attention.py:281-317).  This builds the matching
``AKV_WARM_LEGACY`` descriptor for libakv_hip.so.
"""
from __future__ import annotations

import torch

from . import _native as nat


def padded_dim(D: int, group_size: int) -> int:
    return D if D % group_size == 0 else D + (group_size - D % group_size)


def legacy_desc(kp, ks, kz, vp, vs, vz, bits: int, group_size: int, n_warm: int, D: int,
                warm_heads: int = 1, sym: int = -1, keep: list = None) -> nat.WarmDesc:
    """Validate shapes the way the reference's reshape would and fill the descriptor.

    ``keep`` collects the contiguous device tensors the descriptor points at;
    the caller holds it until the launch is enqueued."""
    if bits not in (2, 4, 8):
        raise ValueError(f"Unsupported bits: {bits}")
    nat.require_device(kp, ks, kz, vp, vs, vz)
    pD = padded_dim(D, group_size)
    G = pD // group_size
    row = pD * bits // 8
    need = warm_heads * n_warm * row
    ts = []
    for p in (kp, vp):
        if p.numel() < need:
            raise ValueError(f"packed warm tier has {p.numel()} bytes, {need} needed")
        ts.append(nat.dev_contig(p.reshape(-1)[:need], torch.uint8) if p.dtype == torch.uint8
                  else nat.dev_contig(p.reshape(-1).to(torch.uint8)[:need]))
    for m in (ks, kz, vs, vz):
        if m.numel() != warm_heads * n_warm * G:
            raise ValueError(f"scales/zeros must hold {warm_heads}x{n_warm}x{G} values, got {tuple(m.shape)}")
    mdt = ks.dtype if ks.dtype in (torch.float16, torch.bfloat16, torch.float32) else torch.float32
    metas = [nat.dev_contig(m.reshape(-1), mdt) for m in (ks, kz, vs, vz)]
    d = nat.WarmDesc()
    d.kind = nat.WARM_LEGACY
    d.bits_k = d.bits_v = bits
    d.n_warm = n_warm
    d.k_codes, d.v_codes = ts[0].data_ptr(), ts[1].data_ptr()
    d.k_scale, d.k_zero, d.v_scale, d.v_zero = (m.data_ptr() for m in metas)
    d.group_size = group_size
    d.meta_dtype = nat.dtype_code(mdt)
    d.warm_heads = warm_heads
    d.legacy_sym = sym
    if keep is not None:
        keep.extend(ts + metas)
    return d
