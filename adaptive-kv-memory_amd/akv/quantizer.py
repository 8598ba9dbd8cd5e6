"""Legacy per-token-group KV quantizer (akv/quantizer.py) on the device.

KVQuantizer.quantize / dequantize keep the reference's layout: the last axis
split into groups of ``group_size`` (zero-padded), fp32 arithmetic, scale
clamp 1e-10, scales and zeros stored in the input dtype, codes packed into a
flat uint8 buffer (4-bit high nibble first, 2-bit MSB first, 8-bit raw);
symmetric mode stores zero-points of 0 and offsets codes by maxv // 2.
"""
from __future__ import annotations

import ctypes
import logging
from dataclasses import dataclass
from enum import IntEnum
from typing import Optional

import torch

from . import _native as nat
from ._legacy import legacy_desc, padded_dim

logger = logging.getLogger(__name__)


class QuantBits(IntEnum):
    INT2 = 2
    INT4 = 4
    INT8 = 8


@dataclass
class QuantConfig:
    """akv/quantizer.py:25-35."""
    bits: int = 4
    group_size: int = 128
    symmetric: bool = False

    def __post_init__(self):
        if self.bits not in (2, 4, 8):
            raise ValueError(f"bits must be 2, 4, or 8, got {self.bits}")
        if self.group_size <= 0:
            raise ValueError(f"group_size must be positive, got {self.group_size}")


@dataclass
class QuantizedTensor:
    """akv/quantizer.py:38-56."""
    data: torch.Tensor
    scales: torch.Tensor
    zeros: torch.Tensor
    shape: tuple
    bits: int
    group_size: int

    @property
    def nbytes(self) -> int:
        return self.data.nbytes + self.scales.nbytes + self.zeros.nbytes

    @property
    def compression_ratio(self) -> float:
        original_bytes = 1
        for s in self.shape:
            original_bytes *= s
        original_bytes *= 2
        return original_bytes / max(self.nbytes, 1)


class KVQuantizer:
    """akv/quantizer.py:60-272 (quantize / dequantize run on the device)."""

    def __init__(self, config: Optional[QuantConfig] = None):
        self.config = config or QuantConfig()

    def quantize(self, tensor: torch.Tensor, bits: Optional[int] = None,
                 group_size: Optional[int] = None) -> QuantizedTensor:
        bits = bits or self.config.bits
        group_size = group_size or self.config.group_size
        nat.require_device(tensor)
        if bits not in (2, 4, 8):
            raise ValueError(f"Unsupported bits: {bits}")
        if group_size not in (32, 64, 128):
            raise NotImplementedError("the MI355X quantizer takes group_size 32, 64 or 128")
        D = tensor.shape[-1]
        if D not in (64, 128):
            raise NotImplementedError("the MI355X quantizer takes a last dim of 64 or 128")
        lib = nat.load()
        x = nat.dev_contig(tensor)
        rows = x.numel() // D
        pD = padded_dim(D, group_size)
        G = pD // group_size
        data = torch.empty(rows, pD * bits // 8, dtype=torch.uint8, device=x.device)
        scales = torch.empty(rows, G, dtype=x.dtype, device=x.device)
        zeros = torch.empty_like(scales)
        a = nat.QuantArgs()
        a.abi_version = nat.ABI_VERSION
        a.B, a.H, a.D = 1, 1, D
        a.in_dtype = nat.dtype_code(x.dtype)
        a.layout = nat.QUANT_KVQ
        a.v = x.data_ptr()
        a.n_src = a.n_sel = rows
        a.bits_k = a.bits_v = bits
        a.block_t = 32
        a.group_v = group_size
        a.symmetric = 1 if self.config.symmetric else 0
        a.v_codes, a.v_scale, a.v_zero = data.data_ptr(), scales.data_ptr(), zeros.data_ptr()
        nat.check(lib.akv_quant_pack(ctypes.byref(a), nat.stream_of(x)), "KVQuantizer.quantize")
        return QuantizedTensor(data=data.reshape(-1), scales=scales, zeros=zeros, shape=tuple(tensor.shape),
                               bits=bits, group_size=group_size)

    def dequantize(self, qtensor: QuantizedTensor) -> torch.Tensor:
        from .triton_ops import _dequantize_packed
        shape = qtensor.shape
        D = shape[-1]
        rows = 1
        for s in shape[:-1]:
            rows *= s
        out = _dequantize_packed(qtensor.data, qtensor.scales.reshape(rows, -1), qtensor.zeros.reshape(rows, -1),
                                 qtensor.bits, qtensor.group_size, rows, D, qtensor.scales.device,
                                 qtensor.scales.dtype)
        return out.reshape(shape)

    def estimate_error(self, tensor: torch.Tensor, bits: Optional[int] = None) -> float:
        qt = self.quantize(tensor, bits=bits)
        rec = self.dequantize(qt)
        return (tensor.float() - rec.float()).pow(2).mean().item()

    def estimate_memory_savings(self, num_layers: int, num_heads: int, seq_len: int, head_dim: int,
                                bits: Optional[int] = None) -> dict:
        """akv/quantizer.py:256-272 (arithmetic only)."""
        bits = bits or self.config.bits
        original_bytes = num_layers * 2 * num_heads * seq_len * head_dim * 2
        data_bytes = num_layers * 2 * num_heads * seq_len * head_dim * bits / 8
        num_groups = (head_dim + self.config.group_size - 1) // self.config.group_size
        meta_bytes = num_layers * 2 * num_heads * seq_len * num_groups * 2 * 2
        total_quant = data_bytes + meta_bytes
        return {
            "original_mb": original_bytes / 1e6,
            "quantized_mb": total_quant / 1e6,
            "savings_mb": (original_bytes - total_quant) / 1e6,
            "compression_ratio": original_bytes / max(total_quant, 1),
        }
