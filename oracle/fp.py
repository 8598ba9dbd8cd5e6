"""Per-operation rounding helpers for the oracle.

The reference runs its quantizer in the tensor's own dtype on the CPU.  In
PyTorch (CPU) every binary op on float16 / bfloat16 is computed in float32 and
rounded once to the storage type (round-to-nearest-even).  By the double
rounding theorem (24 >= 2*11+2, 24 >= 2*8+2) that equals a correctly rounded
fp16 / bf16 operation for + - * /.  numpy's float16 ufuncs do the same, which
``tests/test_oracle_fp.py`` checks on random operands against exact rational
arithmetic; bf16 has no numpy dtype, so it is emulated here on float32 bit
patterns.

Pinning: ``round_bf16`` is checked against exact rational rounding on random
and tie-forced inputs; ``to_u8`` against the conversion table PyTorch 2.10
prints on the CPU (NaN and +-inf -> 0, finite values truncate toward zero and
wrap modulo 256).
"""
from __future__ import annotations

import numpy as np

F16 = "float16"
F32 = "float32"
BF16 = "bfloat16"


def round_bf16(x: np.ndarray) -> np.ndarray:
    """Round float32 values to bfloat16 (RNE); returns float32 holding bf16 values."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    nan = np.isnan(a)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16) << 16
    out = (r & 0xFFFFFFFF).astype(np.uint32).view(np.float32)
    out = np.where(nan, np.float32(np.nan), out)
    return out.astype(np.float32)


def to_dtype(x: np.ndarray, dt: str) -> np.ndarray:
    """Round to the storage dtype ``dt`` (values returned as float16 or float32 arrays)."""
    if dt == F16:
        return np.asarray(x, dtype=np.float32).astype(np.float16)
    if dt == F32:
        return np.asarray(x, dtype=np.float32)
    if dt == BF16:
        return round_bf16(np.asarray(x, dtype=np.float32))
    raise ValueError(f"unknown dtype {dt}")


def op(fn, a, b, dt: str):
    """Apply ``fn`` in float32 and round the result once to ``dt``."""
    r = fn(np.asarray(a, dtype=np.float32), np.asarray(b, dtype=np.float32))
    return to_dtype(r, dt)


def scalar_in(v: float, dt: str) -> np.float32:
    """A Python scalar as the tensor dtype sees it (e.g. clamp(min=1e-8) on fp16 -> 0)."""
    return np.float32(to_dtype(np.array([v], dtype=np.float32), dt).astype(np.float32)[0])


def to_u8(x: np.ndarray) -> np.ndarray:
    """torch CPU ``float.to(torch.uint8)``: NaN/inf -> 0, else trunc toward zero mod 256."""
    a = np.asarray(x, dtype=np.float64)
    bad = ~np.isfinite(a)
    t = np.trunc(np.where(bad, 0.0, a)).astype(np.int64)
    return (t & 0xFF).astype(np.uint8)
