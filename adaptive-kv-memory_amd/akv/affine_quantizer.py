"""Block-affine (min/max) quantizer on the device -- AffineQuantizer's API.

Keys: per-channel asymmetric scale/zero over the tokens of the call; values:
per-token over all channels; optional fp16 outlier channels chosen by the
L2-norm ranking; codes bit-packed (akv/affine_quantizer.py:26-189).  The work
is one ``akv_quant_pack`` launch (one block of N tokens, one group of D
channels) and one ``akv_dequant_unpack`` launch for the inverse, bit-exact
with the reference's fp16 arithmetic.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _native as nat
from . import bitpack
from .warm_tier import n_outliers, packed_row_bytes


@dataclass
class AffineQuantConfig:
    """akv/affine_quantizer.py:26-32 (``group_size`` is accepted and, as in the
    reference, not used: V keeps one scale per token)."""
    key_bits: int = 3
    value_bits: int = 3
    group_size: int = 64
    packed: bool = True
    outlier_fraction: float = 0.0


class AffineQuantizer:
    """akv/affine_quantizer.py:35-189.  Inputs (H, N, D) on the device."""

    def __init__(self, config: AffineQuantConfig):
        self.key_bits = config.key_bits
        self.value_bits = config.value_bits
        self.group_size = config.group_size
        self.packed = config.packed
        self.outlier_fraction = config.outlier_fraction

    # one launch quantizes K (per channel over all N) or V (per token over all D)
    def _quantize(self, x: torch.Tensor, bits: int, which: str) -> dict:
        nat.require_device(x)
        if bits not in (2, 3, 4, 8):
            raise NotImplementedError(f"the MI355X quantizer takes 2/3/4-bit (packed) or 8-bit (raw) codes, got {bits}")
        lib = nat.load()
        if x.dim() != 3:
            raise ValueError("expected (H, N, D)")
        H, N, D = x.shape
        x = nat.dev_contig(x)
        dev = x.device
        n_out = n_outliers(D, self.outlier_fraction)
        codes = torch.empty(1, H, N, packed_row_bytes(D, bits), dtype=torch.uint8, device=dev)
        if which == "k":
            sc = torch.empty(1, H, 1, D, dtype=torch.float16, device=dev)
        else:
            sc = torch.empty(1, H, N, 1, dtype=torch.float16, device=dev)
        ze = torch.empty_like(sc)
        oidx = torch.empty(1, 1, n_out, dtype=torch.int64, device=dev) if n_out else None
        odata = torch.empty(1, H, N, n_out, dtype=torch.float16, device=dev) if n_out else None
        a = nat.QuantArgs()
        a.abi_version = nat.ABI_VERSION
        a.B, a.H, a.D = 1, H, D
        a.in_dtype = nat.dtype_code(x.dtype)
        a.layout = nat.QUANT_AFFINE
        a.n_src = a.n_sel = N
        a.block_t = max(N, 1)
        a.group_v = D
        a.n_out = n_out
        if which == "k":
            a.k = x.data_ptr()
            a.bits_k, a.bits_v = bits, 2
            a.k_codes, a.k_scale, a.k_zero = codes.data_ptr(), sc.data_ptr(), ze.data_ptr()
            if n_out:
                a.k_oidx, a.k_odata = oidx.data_ptr(), odata.data_ptr()
        else:
            a.v = x.data_ptr()
            a.bits_k, a.bits_v = 2, bits
            a.v_codes, a.v_scale, a.v_zero = codes.data_ptr(), sc.data_ptr(), ze.data_ptr()
            if n_out:
                a.v_oidx, a.v_odata = oidx.data_ptr(), odata.data_ptr()
        nat.check(lib.akv_quant_pack(ctypes.byref(a), nat.stream_of(x)), "quantize")
        res = {
            "scale": sc[0],
            "zero": ze[0],
            "orig_dim": D,
            "bits": bits,
        }
        if n_out:
            res["outlier_idx"] = oidx.reshape(n_out)
            res["outlier_data"] = odata[0]
        # 8-bit codes are stored raw, packed or not (bitpack passes them through)
        res["codes"] = codes[0] if (self.packed or bits == 8) else bitpack.unpack(codes[0], bits, D)
        return res

    def _dequantize(self, q: dict, which: str) -> torch.Tensor:
        lib = nat.load()
        bits = q.get("bits", self.key_bits if which == "k" else self.value_bits)
        codes = q["codes"]
        D = q["orig_dim"]
        if bits not in (2, 3, 4, 8):
            raise NotImplementedError(f"the MI355X dequant takes 2/3/4/8-bit codes, got {bits}")
        if not self.packed and bits != 8:
            codes = bitpack.pack(codes, bits)
        nat.require_device(codes)
        H, N = codes.shape[0], codes.shape[1]
        codes = nat.dev_contig(codes, torch.uint8)
        sc = nat.dev_contig(q["scale"], torch.float16)
        ze = nat.dev_contig(q["zero"], torch.float16)
        out = torch.empty(1, H, N, D, dtype=torch.float16, device=codes.device)
        d = nat.WarmDesc()
        d.kind = nat.WARM_AFFINE
        d.bits_k = d.bits_v = bits
        d.n_warm = N
        d.block_t = max(N, 1)
        d.group_v = D
        keep = []
        if "outlier_idx" in q:
            oi = nat.dev_contig(q["outlier_idx"], torch.int64)
            od = nat.dev_contig(q["outlier_data"], torch.float16)
            keep += [oi, od]
            d.n_out = oi.numel()
            d.k_oidx = d.v_oidx = oi.data_ptr()
            d.k_odata = d.v_odata = od.data_ptr()
        d.k_codes = d.v_codes = codes.data_ptr()
        d.k_scale = d.v_scale = sc.data_ptr()
        d.k_zero = d.v_zero = ze.data_ptr()
        a = nat.DequantArgs()
        a.abi_version = nat.ABI_VERSION
        a.B, a.Hkv, a.D = 1, H, D
        a.out_dtype = nat.DT_F16
        a.warm = d
        if which == "k":
            a.k_out = out.data_ptr()
        else:
            a.v_out = out.data_ptr()
        nat.check(lib.akv_dequant_unpack(ctypes.byref(a), nat.stream_of(codes)), "dequantize")
        return out[0]

    def quantize_keys(self, k: torch.Tensor) -> dict:
        """akv/affine_quantizer.py:63-110."""
        return self._quantize(k, self.key_bits, "k")

    def dequantize_keys(self, qk: dict) -> torch.Tensor:
        """akv/affine_quantizer.py:112-124."""
        return self._dequantize(qk, "k")

    def quantize_values(self, v: torch.Tensor) -> dict:
        """akv/affine_quantizer.py:131-176."""
        return self._quantize(v, self.value_bits, "v")

    def dequantize_values(self, qv: dict) -> torch.Tensor:
        """akv/affine_quantizer.py:178-189."""
        return self._dequantize(qv, "v")
