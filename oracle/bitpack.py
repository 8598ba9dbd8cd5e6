"""Oracle restatement of ``akv/bitpack.py`` (the warm-tier byte layout).

Layouts (all along the last axis, uint8 in / uint8 out):
  * 4-bit: byte i = (c[2i] & 15) << 4 | (c[2i+1] & 15); odd length zero-padded
    (akv/bitpack.py:13-19); unpack keeps ``orig_dim`` codes (:22-30).
  * 3-bit: 8 codes -> 24-bit word w = c0<<21 | ... | c7, stored big-endian as
    bytes [w>>16, w>>8, w]; length padded to a multiple of 8 (:35-51); unpack
    trims to ``orig_dim`` (:54-68).
  * 2-bit: byte = c0<<6 | c1<<4 | c2<<2 | c3; padded to a multiple of 4
    (:73-79); unpack requires the padded length to match (:82-90).
  * any other width passes through (:95-114); ``packed_bytes`` (:117-120).

Pinning: hand-derived byte vectors (``tests/golden/bitpack_kat.json``: 4-bit
[3,7]->0x37, [1,15]->0x1F; 2-bit [0,1,2,3]->0x1B; 3-bit
[1,2,3,4,5,6,7,0]->[0x29,0xCB,0xB8]) plus a bit-by-bit brute-force packer
written independently in the tests (bit position arithmetic rather than
shifts of whole lanes), and round trips at the reference test sizes.
"""
from __future__ import annotations

import numpy as np


def _pad_last(x: np.ndarray, mult: int) -> np.ndarray:
    r = x.shape[-1] % mult
    if r == 0:
        return x
    pad = [(0, 0)] * (x.ndim - 1) + [(0, mult - r)]
    return np.pad(x, pad)


def pack_uint4(codes: np.ndarray) -> np.ndarray:
    """akv/bitpack.py:13-19."""
    c = _pad_last(np.asarray(codes).astype(np.uint8), 2)
    return (((c[..., 0::2] & 0x0F) << 4) | (c[..., 1::2] & 0x0F)).astype(np.uint8)


def unpack_uint4(packed: np.ndarray, orig_dim: int) -> np.ndarray:
    """akv/bitpack.py:22-30."""
    p = np.asarray(packed, dtype=np.uint8)
    out = np.empty(p.shape[:-1] + (orig_dim,), dtype=np.uint8)
    out[..., 0::2] = ((p >> 4) & 0x0F)[..., : orig_dim // 2 + orig_dim % 2]
    out[..., 1::2] = (p & 0x0F)[..., : orig_dim // 2]
    return out


def pack_uint3(codes: np.ndarray) -> np.ndarray:
    """akv/bitpack.py:35-51."""
    c = _pad_last(np.asarray(codes).astype(np.int64), 8) & 0x07
    g = c.reshape(c.shape[:-1] + (-1, 8))
    w = np.zeros(g.shape[:-1], dtype=np.int64)
    for i in range(8):
        w |= g[..., i] << (21 - 3 * i)
    b = np.stack([(w >> 16) & 0xFF, (w >> 8) & 0xFF, w & 0xFF], axis=-1)
    return b.reshape(c.shape[:-1] + (-1,)).astype(np.uint8)


def unpack_uint3(packed: np.ndarray, orig_dim: int) -> np.ndarray:
    """akv/bitpack.py:54-68."""
    p = np.asarray(packed, dtype=np.uint8)
    k = p.shape[-1] // 3
    q = p[..., : 3 * k].reshape(p.shape[:-1] + (k, 3)).astype(np.int64)
    w = (q[..., 0] << 16) | (q[..., 1] << 8) | q[..., 2]
    out = np.stack([(w >> (21 - 3 * i)) & 0x7 for i in range(8)], axis=-1)
    return out.reshape(p.shape[:-1] + (k * 8,))[..., :orig_dim].astype(np.uint8)


def pack_uint2(codes: np.ndarray) -> np.ndarray:
    """akv/bitpack.py:73-79."""
    c = _pad_last(np.asarray(codes).astype(np.uint8), 4) & 0x03
    return ((c[..., 0::4] << 6) | (c[..., 1::4] << 4) | (c[..., 2::4] << 2) | c[..., 3::4]).astype(np.uint8)


def unpack_uint2(packed: np.ndarray, orig_dim: int) -> np.ndarray:
    """akv/bitpack.py:82-90 (the reference's strided assignment only succeeds
    when every one of the four crumb slots has as many entries as there are
    packed bytes, i.e. orig_dim == 4 * packed_len; other lengths raise)."""
    p = np.asarray(packed, dtype=np.uint8)
    if orig_dim != 4 * p.shape[-1]:
        raise ValueError("unpack_uint2: orig_dim must equal 4 * packed length")
    out = np.empty(p.shape[:-1] + (orig_dim,), dtype=np.uint8)
    out[..., 0::4] = (p >> 6) & 0x03
    out[..., 1::4] = (p >> 4) & 0x03
    out[..., 2::4] = (p >> 2) & 0x03
    out[..., 3::4] = p & 0x03
    return out


def pack(codes: np.ndarray, bits: int) -> np.ndarray:
    """akv/bitpack.py:95-103."""
    if bits == 4:
        return pack_uint4(codes)
    if bits == 3:
        return pack_uint3(codes)
    if bits == 2:
        return pack_uint2(codes)
    return np.asarray(codes)


def unpack(packed: np.ndarray, bits: int, orig_dim: int) -> np.ndarray:
    """akv/bitpack.py:106-114."""
    if bits == 4:
        return unpack_uint4(packed, orig_dim)
    if bits == 3:
        return unpack_uint3(packed, orig_dim)
    if bits == 2:
        return unpack_uint2(packed, orig_dim)
    return np.asarray(packed)


def packed_bytes(codes: np.ndarray, bits: int) -> int:
    """akv/bitpack.py:117-120."""
    p = pack(codes, bits)
    return int(p.size * p.itemsize)


def packed_row_bytes(dim: int, bits: int) -> int:
    """Bytes one packed row of ``dim`` codes occupies (padding included)."""
    if bits == 4:
        return (dim + 1) // 2
    if bits == 3:
        return 3 * ((dim + 7) // 8)
    if bits == 2:
        return (dim + 3) // 4
    return dim
