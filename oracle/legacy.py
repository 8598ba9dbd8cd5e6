"""Oracle restatement of the reference's legacy per-token-group layout.

This is the layout the reference's public attention ops take (warm tier
shared by every batch element and head):

  * ``KVQuantizer.quantize / dequantize / _pack / _unpack``
    (akv/quantizer.py:71-247): rows of the last axis split into groups of
    ``group_size``; fp32 arithmetic; scale clamp 1e-10; scales/zeros cast back
    to the input dtype; symmetric mode stores zero = 0 and offsets by maxv//2.
  * ``_dequantize_packed`` (akv/triton_ops.py:657-713): flat unpack (4-bit high
    then low, 2-bit MSB first, 8-bit raw, 3-bit -> ValueError), reshape to
    (N, G, gs); if ALL zero-points are 0 use (u - maxv//2)*s, else u*s + z, in
    fp32; trim to D; cast to dtype.
  * ``fused_quantize_evict`` (akv/triton_kernels.py:426-507): gather of masked
    rows, per-token groups in the INPUT dtype with clamp(1e-8); packs 4/2-bit,
    leaves 3- and 8-bit codes unpacked.
  * ``_dequant_int4_tile`` (akv/fused_attention.py:281-317): per-head int4,
    fp32 ``u*s + z`` cast to fp16.
  * ``PackedKVArena`` (akv/packed_layout.py:106-265): per (head, token, group)
    quantize in the input dtype with clamp(1e-10), padding dropped before the
    4-bit high-nibble-first / 2-bit MSB-first pack; dequant fp32 ``u*s + z``
    (no symmetric branch) cast to the store dtype.

This module is test infrastructure: only the tests, the smoke check and the
benchmark's CPU-baseline leg use it, as the checker.

Pinning: the pack/unpack vectors of tests/test_quantizer.py:88-108 and the
8-bit MSE bound of tests/test_triton_ops.py:40-50 are restated as tests;
dequant arithmetic is checked against float64 evaluation of the closed form
on every code value; the symmetric branch and the uint8 wrap of code -1
(torch prints 255 for float(-1).to(uint8)) are checked on hand-built inputs.
``kvq_quantize`` (asymmetric, 2/4/8 bits, fp16 and fp32 inputs, ragged last
group), ``quantize_evict`` (2/3/4/8 bits, group sizes below, at and above D)
``arena_quantize`` (2/4/8 bits, fp16 / bf16 / fp32 inputs, constant groups where
the 1e-10 clamp is active, D below the group size), ``arena_dequantize``
and ``dequant_int4_tile`` are checked against exact rational arithmetic with
per-op round-to-nearest-even, levels enumerated for the nearest code, and a
bit-position packer (tests/test_oracle_pinning_legacy.py), plus tie, constant
group, active-clamp and zero-padding cases.  In ``dequant_int4_tile`` the
fp32 product of a 4-bit code and an fp16 scale is exact, and no fp16 scale /
zero searched (every scale below 2^-13, zeros in several binades) makes the
fp32 sum round to fp16 differently from one rounding of the exact value, so
the order of the reference's fp32 ops there is immaterial.
"""
from __future__ import annotations

import numpy as np

from .fp import F16, F32, op, scalar_in, to_dtype, to_u8


def _np_dt(dt: str):
    return np.float16 if dt == F16 else np.float32


# ---------------------------------------------------------------- KVQuantizer

def kvq_pack(data: np.ndarray, bits: int) -> np.ndarray:
    """akv/quantizer.py:194-223 (flat)."""
    flat = np.asarray(data).astype(np.uint8).reshape(-1)
    if bits == 8:
        return flat.copy()
    if bits == 4:
        if flat.size % 2:
            flat = np.pad(flat, (0, 1))
        return ((flat[0::2] << 4).astype(np.uint8) | (flat[1::2] & 0x0F)).astype(np.uint8)
    if bits == 2:
        pad = (4 - flat.size % 4) % 4
        if pad:
            flat = np.pad(flat, (0, pad))
        return (((flat[0::4] & 3) << 6) | ((flat[1::4] & 3) << 4) | ((flat[2::4] & 3) << 2) | (flat[3::4] & 3)).astype(np.uint8)
    raise ValueError(f"Unsupported bits: {bits}")


def kvq_unpack(packed: np.ndarray, bits: int, num_elements: int) -> np.ndarray:
    """akv/quantizer.py:225-247 -> float32."""
    p = np.asarray(packed, dtype=np.uint8).reshape(-1)
    if bits == 8:
        return p[:num_elements].astype(np.float32)
    if bits == 4:
        u = np.stack([(p >> 4) & 0x0F, p & 0x0F], axis=-1).reshape(-1)
        return u[:num_elements].astype(np.float32)
    if bits == 2:
        u = np.stack([(p >> 6) & 3, (p >> 4) & 3, (p >> 2) & 3, p & 3], axis=-1).reshape(-1)
        return u[:num_elements].astype(np.float32)
    raise ValueError(f"Unsupported bits: {bits}")


def kvq_quantize(tensor: np.ndarray, bits: int = 4, group_size: int = 128,
                 symmetric: bool = False) -> dict:
    """akv/quantizer.py:71-143 (fp32 arithmetic; scales/zeros in the input dtype)."""
    if bits not in (2, 4, 8):
        raise ValueError(f"bits must be 2, 4, or 8, got {bits}")
    x = np.asarray(tensor)
    in_dt = F16 if x.dtype == np.float16 else F32
    shape = x.shape
    flat = x.reshape(-1, shape[-1]).astype(np.float32)
    rows, feats = flat.shape
    if feats % group_size:
        flat = np.pad(flat, ((0, 0), (0, group_size - feats % group_size)))
    g = flat.reshape(rows, -1, group_size)
    gmin = g.min(axis=-1, keepdims=True)
    gmax = g.max(axis=-1, keepdims=True)
    maxv = (1 << bits) - 1
    with np.errstate(divide="ignore", invalid="ignore"):
        if symmetric:
            absmax = np.maximum(np.abs(gmin), np.abs(gmax))
            scales = (absmax / np.float32(maxv / 2)).astype(np.float32)
            scales = np.maximum(scales, np.float32(1e-10))
            zeros = np.zeros_like(scales)
            q = np.clip(np.rint(g / scales), -maxv // 2, maxv // 2)
            q = to_u8(q + maxv // 2)
        else:
            scales = ((gmax - gmin) / np.float32(maxv)).astype(np.float32)
            scales = np.maximum(scales, np.float32(1e-10))
            zeros = gmin
            q = to_u8(np.clip(np.rint((g - zeros) / scales), 0, maxv))
    packed = kvq_pack(q.reshape(rows, -1), bits)
    return dict(data=packed, scales=to_dtype(scales[..., 0], in_dt), zeros=to_dtype(zeros[..., 0], in_dt),
                shape=shape, bits=bits, group_size=group_size, dtype=in_dt)


def kvq_dequantize(qt: dict) -> np.ndarray:
    """akv/quantizer.py:145-192 -> array in the scales' dtype."""
    bits, gs, shape = qt["bits"], qt["group_size"], qt["shape"]
    rows = int(np.prod(shape[:-1]))
    feats = shape[-1]
    pf = feats + ((gs - feats % gs) if feats % gs else 0)
    u = kvq_unpack(qt["data"], bits, rows * pf).reshape(rows, -1, gs)
    s = qt["scales"].astype(np.float32)[..., None]
    z = qt["zeros"].astype(np.float32)[..., None]
    if np.all(z == 0):
        d = ((u - np.float32((1 << bits) - 1) // 2) * s).astype(np.float32)
    else:
        d = ((u * s).astype(np.float32) + z).astype(np.float32)
    d = d.reshape(rows, -1)[:, :feats]
    return to_dtype(d.reshape(shape), qt["dtype"])


# ---------------------------------------------------------- _dequantize_packed

def dequantize_packed(packed, scales, zeros, bits, group_size, N, D, dtype=F16) -> np.ndarray:
    """akv/triton_ops.py:657-713."""
    p = np.asarray(packed, dtype=np.uint8).reshape(-1)
    if bits == 4:
        u = np.stack([(p >> 4) & 0x0F, p & 0x0F], axis=-1).reshape(-1).astype(np.float32)
    elif bits == 2:
        u = np.stack([(p >> 6) & 3, (p >> 4) & 3, (p >> 2) & 3, p & 3], axis=-1).reshape(-1).astype(np.float32)
    elif bits == 8:
        u = p.astype(np.float32)
    else:
        raise ValueError(f"Unsupported bits: {bits}")
    pD = D if D % group_size == 0 else D + (group_size - D % group_size)
    u = u[: N * pD].reshape(N, -1, group_size)
    s = np.asarray(scales).astype(np.float32)[..., None]
    z = np.asarray(zeros).astype(np.float32)[..., None]
    if np.all(z == 0):
        d = ((u - np.float32((1 << bits) - 1) // 2) * s).astype(np.float32)
    else:
        d = ((u * s).astype(np.float32) + z).astype(np.float32)
    return to_dtype(d.reshape(N, -1)[:, :D], dtype)


# ------------------------------------------------------- fused_quantize_evict

def quantize_evict(keys, values, evict_mask, bits=4, group_size=128):
    """akv/triton_kernels.py:426-507 (input-dtype arithmetic)."""
    keys = np.asarray(keys)
    dt = F16 if keys.dtype == np.float16 else F32
    idx = np.nonzero(np.asarray(evict_mask))[0]
    if idx.size == 0:
        e8 = np.zeros((0,), np.uint8)
        ef = np.zeros((0,), _np_dt(dt))
        return e8, ef, ef, e8, ef, ef
    maxi = (1 << bits) - 1

    def qt(t):
        n, d = t.shape
        if d % group_size:
            t = np.pad(t, ((0, 0), (0, group_size - d % group_size)))
        g = t.reshape(n, -1, group_size)
        gmin = g.min(axis=-1, keepdims=True)
        gmax = g.max(axis=-1, keepdims=True)
        sc = op(np.subtract, gmax, gmin, dt)
        sc = op(np.divide, sc, np.float32(maxi), dt)
        lo = scalar_in(1e-8, dt)
        sc = to_dtype(np.maximum(sc.astype(np.float32), lo), dt)
        with np.errstate(divide="ignore", invalid="ignore"):
            q = op(np.divide, op(np.subtract, g, gmin, dt), sc, dt)
        q = to_u8(np.clip(np.rint(q.astype(np.float32)), 0, maxi))
        if bits == 4:
            pk = ((q[:, :, ::2] << 4) | q[:, :, 1::2]).astype(np.uint8).reshape(n, -1)
        elif bits == 2:
            pk = ((q[:, :, ::4] << 6) | (q[:, :, 1::4] << 4) | (q[:, :, 2::4] << 2) | q[:, :, 3::4]).astype(np.uint8).reshape(n, -1)
        else:
            pk = q.reshape(n, -1)
        return pk, sc[..., 0], gmin[..., 0]

    kp, ks, kz = qt(keys[idx])
    vp, vs, vz = qt(np.asarray(values)[idx])
    return kp, ks, kz, vp, vs, vz


# ------------------------------------------------------------ PackedKVArena

def arena_pack(q: np.ndarray, bits: int) -> np.ndarray:
    """PackedKVArena._pack (akv/packed_layout.py:203-229): 4-bit even channel in the
    high nibble, 2-bit MSB first, 8-bit raw; along the last axis."""
    q = np.asarray(q, dtype=np.uint8)
    if bits == 4:
        return ((q[..., 0::2] << 4) | (q[..., 1::2] & 0x0F)).astype(np.uint8)
    if bits == 2:
        return (((q[..., 0::4] & 3) << 6) | ((q[..., 1::4] & 3) << 4) | ((q[..., 2::4] & 3) << 2)
                | (q[..., 3::4] & 3)).astype(np.uint8)
    return q


def arena_unpack(packed: np.ndarray, bits: int, target_dim: int) -> np.ndarray:
    """PackedKVArena._unpack (akv/packed_layout.py:231-265), as float32."""
    p = np.asarray(packed, dtype=np.uint8)
    if bits == 4:
        u = np.stack([(p >> 4) & 0x0F, p & 0x0F], axis=-1)
    elif bits == 2:
        u = np.stack([(p >> 6) & 3, (p >> 4) & 3, (p >> 2) & 3, p & 3], axis=-1)
    else:
        return p.astype(np.float32)
    return u.reshape(p.shape[:-1] + (-1,)).astype(np.float32)[..., :target_dim]


def arena_quantize(keys: np.ndarray, bits: int = 4, group_size: int = 128, dt: str = F16, store: str = F16):
    """PackedKVArena.quantize_and_append's arithmetic (akv/packed_layout.py:127-153):
    keys (H, N, D) in dtype ``dt`` (bf16 given as float32 holding bf16 values);
    D zero-padded to the group size, per (head, token, group) min / max, scale =
    (max - min) / maxv clamped at 1e-10, every op rounded to ``dt``; codes rounded
    half-to-even and clamped to [0, maxv]; the padding dropped before packing;
    scales and zeros cast to ``store``.  Returns (packed, scales, zeros)."""
    if bits not in (2, 4, 8):
        raise ValueError(f"bits must be 2, 4 or 8, got {bits}")
    x = to_dtype(np.asarray(keys, dtype=np.float32), dt).astype(np.float32)
    H, N, D = x.shape
    G = (D + group_size - 1) // group_size
    if G * group_size > D:
        x = np.concatenate([x, np.zeros((H, N, G * group_size - D), np.float32)], axis=-1)
    g = x.reshape(H, N, G, group_size)
    gmin, gmax = g.min(axis=-1), g.max(axis=-1)
    maxv = (1 << bits) - 1
    sc = op(np.subtract, gmax, gmin, dt)
    sc = op(np.divide, sc, np.float32(maxv), dt).astype(np.float32)
    sc = np.where(np.isnan(sc), sc, np.maximum(sc, scalar_in(1e-10, dt)))
    with np.errstate(divide="ignore", invalid="ignore"):
        q = op(np.divide, op(np.subtract, g, gmin[..., None], dt), sc[..., None], dt).astype(np.float32)
    q = to_u8(np.clip(np.rint(q), 0, maxv))
    q = q.reshape(H, N, -1)[:, :, :D]
    return arena_pack(q, bits), to_dtype(sc, store), to_dtype(gmin, store)


def arena_dequantize(packed, scales, zeros, bits: int, group_size: int, head_dim: int, store: str = F16):
    """PackedKVArena.dequantize_slice (akv/packed_layout.py:163-187): fp32 u * s, then
    + z in fp32 (two roundings), cast to the store dtype; (H, N, D)."""
    u = arena_unpack(packed, bits, head_dim)
    gi = np.arange(head_dim) // group_size
    s = np.asarray(scales, dtype=np.float32)[..., gi]
    z = np.asarray(zeros, dtype=np.float32)[..., gi]
    return to_dtype(((u * s).astype(np.float32) + z).astype(np.float32), store)


# ------------------------------------------------------- _dequant_int4_tile

def dequant_int4_tile(packed, scales, zeros, head_dim, group_size) -> np.ndarray:
    """akv/fused_attention.py:281-317 -> (H, N, D) float16."""
    p = np.asarray(packed, dtype=np.uint8)
    H, N, _ = p.shape
    r = np.empty((H, N, head_dim), np.float32)
    r[:, :, 0::2] = ((p >> 4) & 0x0F).astype(np.float32)
    r[:, :, 1::2] = (p & 0x0F).astype(np.float32)
    gi = np.arange(head_dim) // group_size
    s = np.asarray(scales)[:, :, gi].astype(np.float32)
    z = np.asarray(zeros)[:, :, gi].astype(np.float32)
    return ((r * s).astype(np.float32) + z).astype(np.float32).astype(np.float16)
