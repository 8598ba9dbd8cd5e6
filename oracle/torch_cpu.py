"""Torch-on-CPU restatement of the reference's CPU decode path (test infrastructure).

Only ``tests/`` and the ``cpu_baseline`` leg of ``bench.py`` use this module: it is the
CPU baseline the GPU path is timed beside, and it is checked against the numpy
restatement (``oracle.affine`` / ``oracle.attention`` / ``oracle.importance``) in
``tests/test_oracle_torch_cpu.py`` (dequantized K/V bit-exact, attention and importance
within fp32 summation-order differences).

The steps follow the reference source with torch CPU ops:

1. unpack the bit-packed codes (akv/bitpack.py:13-120: 4-bit high nibble first, 3-bit
   eight codes in three bytes most significant first, 2-bit most significant first);
2. dequantize in fp16, ``codes.half() * scale + zero`` with one fp16 rounding per op
   (akv/affine_quantizer.py:112-124, :178-189), K's scale and zero per (block, channel),
   V's per (token, channel group), then the fp16 outlier channels written over
   (akv/affine_quantizer.py:121-123);
3. expand the kv heads to the query heads (HF ``repeat_kv``) and concatenate the warm
   and hot tokens in cache order (akv/drop_in.py:762-787);
4. attend in fp32: ``.float()``, matmul times ``sm_scale``, softmax, matmul
   (akv/triton_kernels.py:350-387);
5. update the importance: ``scores * decay + attn.mean((0, 1)).sum(0)``
   (akv/triton_ops.py:604-650).
"""
from __future__ import annotations

import math

import torch


def unpack_codes(packed: torch.Tensor, bits: int, dim: int) -> torch.Tensor:
    """uint8 [..., P] in the bitpack layout -> uint8 codes [..., dim]."""
    p = packed.to(torch.int32)
    if bits == 8:
        return packed[..., :dim]
    if bits == 4:
        c = torch.stack([(p >> 4) & 15, p & 15], dim=-1)
    elif bits == 2:
        c = torch.stack([(p >> 6) & 3, (p >> 4) & 3, (p >> 2) & 3, p & 3], dim=-1)
    elif bits == 3:
        t = p.reshape(*p.shape[:-1], -1, 3)
        w = (t[..., 0] << 16) | (t[..., 1] << 8) | t[..., 2]
        c = torch.stack([(w >> (21 - 3 * i)) & 7 for i in range(8)], dim=-1)
    else:
        raise ValueError(f"bits={bits}")
    return c.reshape(*p.shape[:-1], -1)[..., :dim].to(torch.uint8)


def dequant_kv_blocked(w: dict):
    """fp16 K and V (B, H, N, D) from the warm-tier arrays (torch CPU tensors): the
    same arithmetic as ``oracle.affine.dequant_kv_blocked``."""
    D, N, T, G = w["D"], w["N"], w["T"], w["G"]
    ck = unpack_codes(w["k_codes"], w["bits_k"], D)
    cv = unpack_codes(w["v_codes"], w["bits_v"], D)
    blk = torch.arange(N) // T
    kd = ck.half() * w["k_scale"][:, :, blk, :] + w["k_zero"][:, :, blk, :]
    grp = torch.arange(D) // G
    vd = cv.half() * w["v_scale"][..., grp] + w["v_zero"][..., grp]
    if w.get("n_out", 0):
        B, H = kd.shape[:2]
        for x, key in ((kd, "k"), (vd, "v")):
            idx = w[key + "_oidx"][:, blk, :]  # (B, N, n_out)
            gi = idx[:, None].expand(B, H, N, idx.shape[-1])
            x.scatter_(3, gi, w[key + "_odata"])
    return kd, vd


def decode_attention(q, k_hot, v_hot, k_warm, v_warm, hot_first: bool = False, sm_scale=None,
                     return_weights: bool = True):
    """q (B, Hq, M, D); hot and warm (B, Hkv, n, D) fp16 -> (out fp32, attn fp32 or None)."""
    B, Hq, M, D = q.shape
    g = Hq // k_hot.shape[1]
    parts = [k_hot, k_warm] if hot_first else [k_warm, k_hot]
    vparts = [v_hot, v_warm] if hot_first else [v_warm, v_hot]
    k = torch.cat(parts, dim=2).repeat_interleave(g, dim=1)
    v = torch.cat(vparts, dim=2).repeat_interleave(g, dim=1)
    scale = 1.0 / math.sqrt(D) if sm_scale is None else sm_scale
    s = torch.matmul(q.float(), k.float().transpose(-1, -2)) * scale
    p = torch.softmax(s, dim=-1)
    out = torch.matmul(p, v.float())
    return out, (p if return_weights else None)


def importance_update(attn: torch.Tensor, scores: torch.Tensor, decay: float) -> torch.Tensor:
    """scores * decay + attn.mean((0, 1)).sum(0), padded or truncated to len(scores)."""
    imp = attn.float().mean(dim=(0, 1)).sum(dim=0)
    n = scores.shape[0]
    imp = imp[:n] if imp.shape[0] >= n else torch.cat([imp, imp.new_zeros(n - imp.shape[0])])
    return scores * decay + imp
