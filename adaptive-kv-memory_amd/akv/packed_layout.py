"""Packed-layout helpers of the warm tier: measured byte accounting and the
preallocated per-head arena (akv/packed_layout.py).

``measure_packed_bytes`` follows akv/packed_layout.py:501-543: the bytes of a
quantizer dict after bit-packing -- ``codes`` as stored when the dict carries
``'bits'`` (AffineQuantizer packs them already), else packed at 2/3/4 bits --
plus the ``group_mean`` / ``group_std`` / ``scale`` / ``zero`` tensors at their
stored dtype.  Outlier channels are not counted (as in the reference).
"""
from __future__ import annotations

import torch

from . import bitpack

pack_uint4 = bitpack.pack_uint4
pack_uint3 = bitpack.pack_uint3
pack_uint2 = bitpack.pack_uint2


def measure_packed_bytes(qdata: dict, bits: int) -> int:
    """akv/packed_layout.py:501-543."""
    if "codes" not in qdata:
        return 0
    codes = qdata["codes"]
    if "bits" in qdata:
        total = codes.element_size() * codes.numel()
    else:
        total = bitpack.packed_bytes(codes, bits)
    for key in ("group_mean", "group_std", "scale", "zero"):
        t = qdata.get(key)
        if isinstance(t, torch.Tensor):
            total += t.element_size() * t.numel()
    return int(total)
