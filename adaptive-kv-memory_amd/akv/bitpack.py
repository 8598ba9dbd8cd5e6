"""Bit-packing of 2/3/4-bit codes on the device (layout of akv/bitpack.py).

  4-bit: byte i = c[2i] << 4 | c[2i+1]; odd length zero-padded  (akv/bitpack.py:13-19)
  3-bit: 8 codes -> w = c0<<21 | ... | c7 -> bytes [w>>16, w>>8, w]   (:35-51)
  2-bit: byte = c0<<6 | c1<<4 | c2<<2 | c3                      (:73-79)
  other widths pass through unchanged                            (:95-114)
"""
from __future__ import annotations

import ctypes

import torch

from . import _native as nat
from .warm_tier import packed_row_bytes


def _pack(indices: torch.Tensor, bits: int) -> torch.Tensor:
    nat.require_device(indices)
    lib = nat.load()
    dim = indices.shape[-1]
    c = nat.dev_contig(indices, torch.uint8)
    rows = c.numel() // dim if dim else 0
    out = torch.empty(indices.shape[:-1] + (packed_row_bytes(dim, bits),), dtype=torch.uint8, device=c.device)
    nat.check(lib.akv_bitpack(c.data_ptr(), out.data_ptr(), rows, dim, bits, nat.stream_of(c)), "pack")
    return out


def _unpack(packed: torch.Tensor, bits: int, orig_dim: int) -> torch.Tensor:
    nat.require_device(packed)
    lib = nat.load()
    p = nat.dev_contig(packed, torch.uint8)
    pdim = p.shape[-1]
    rows = p.numel() // pdim if pdim else 0
    out = torch.empty(packed.shape[:-1] + (orig_dim,), dtype=torch.uint8, device=p.device)
    nat.check(lib.akv_bitunpack(p.data_ptr(), out.data_ptr(), rows, pdim, orig_dim, bits, nat.stream_of(p)), "unpack")
    return out


def pack_uint4(indices: torch.Tensor) -> torch.Tensor:
    return _pack(indices, 4)


def unpack_uint4(packed: torch.Tensor, orig_dim: int) -> torch.Tensor:
    return _unpack(packed, 4, orig_dim)


def pack_uint3(indices: torch.Tensor) -> torch.Tensor:
    return _pack(indices, 3)


def unpack_uint3(packed: torch.Tensor, orig_dim: int) -> torch.Tensor:
    return _unpack(packed, 3, orig_dim)


def pack_uint2(indices: torch.Tensor) -> torch.Tensor:
    return _pack(indices, 2)


def unpack_uint2(packed: torch.Tensor, orig_dim: int) -> torch.Tensor:
    return _unpack(packed, 2, orig_dim)


def pack(indices: torch.Tensor, bits: int) -> torch.Tensor:
    """akv/bitpack.py:95-103."""
    if bits in (2, 3, 4):
        return _pack(indices, bits)
    return indices


def unpack(packed: torch.Tensor, bits: int, orig_dim: int) -> torch.Tensor:
    """akv/bitpack.py:106-114."""
    if bits in (2, 3, 4):
        return _unpack(packed, bits, orig_dim)
    return packed


def packed_bytes(codes: torch.Tensor, bits: int) -> int:
    """akv/bitpack.py:117-120 (the size ``pack`` would produce)."""
    if bits in (2, 3, 4):
        dim = codes.shape[-1]
        rows = codes.numel() // dim if dim else 0
        return rows * packed_row_bytes(dim, bits)
    return codes.element_size() * codes.numel()
