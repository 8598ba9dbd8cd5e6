"""Synthetic workloads of the warm-tier hot path (seeded, reproducible).

Convention: one ``torch.Generator`` per tensor role, seeded 0 (K), 1 (V),
2 (Q), 3 (outlier / heavy-tailed channel choice), 4 (importance scores),
each offset by 16 * layer for multi-layer workloads; values drawn in fp32 and
cast to the storage dtype.  The hot window is the last ``n_hot`` positions,
the warm tier positions [0, n_warm) in order.

Shapes:
  qwen_decode_4k   B1, Hq12/Hkv2, D128, N 4096 (512 hot, 3584 warm), K4/V4,
                   2 K channels per kv head scaled x10, no outlier protection.
  qwen_decode_32k  B8, Hq12/Hkv2, D128, N 32768 (1024 hot, 31744 warm), K3/V3
                   (balanced preset), 28 layers, K outliers as above,
                   importance EMA decay 0.9.
  llama7b_decode_16k  B4, Hq=Hkv=32, D128, N 16384 (512 hot), K4/V2,
                   outlier_fraction 0.01 (1 protected channel per block),
                   4 of 128 channels per head Student-t(3).
  llama3_demote_64k   B16, Hkv8, D128, S 65536 fp16, importance U(0,1),
                   demote S-1024 tokens (first 4 / last 16 protected).
  llama70b_prefill_128k  B1, Hq64/Hkv8, D128, M 512 bf16 queries,
                   N 131072 (4096 hot, 126976 warm at K2/V2).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

SEED_K, SEED_V, SEED_Q, SEED_CH, SEED_IMP = 0, 1, 2, 3, 4


@dataclass(frozen=True)
class DecodeShape:
    name: str
    B: int
    Hq: int
    Hkv: int
    D: int
    n_hot: int
    n_warm: int
    bits_k: int
    bits_v: int
    layers: int = 1
    outlier_fraction: float = 0.0
    k_outlier_channels: int = 0     # channels per kv head scaled x10 (data only)
    heavy_tail_channels: int = 0    # channels per kv head drawn Student-t(3)
    decay: Optional[float] = None
    block_t: int = 32
    group_v: int = 32
    M: int = 1

    @property
    def N(self) -> int:
        return self.n_hot + self.n_warm


QWEN_DECODE_4K = DecodeShape("qwen_decode_4k", 1, 12, 2, 128, 512, 3584, 4, 4, k_outlier_channels=2)
QWEN_DECODE_32K = DecodeShape("qwen_decode_32k", 8, 12, 2, 128, 1024, 31744, 3, 3, layers=28,
                              k_outlier_channels=2, decay=0.9)
LLAMA7B_DECODE_16K = DecodeShape("llama7b_decode_16k", 4, 32, 32, 128, 512, 15872, 4, 2,
                                 outlier_fraction=0.01, heavy_tail_channels=4)
LLAMA70B_PREFILL_128K = DecodeShape("llama70b_prefill_128k", 1, 64, 8, 128, 4096, 126976, 2, 2, M=512)

SHAPES = {s.name: s for s in (QWEN_DECODE_4K, QWEN_DECODE_32K, LLAMA7B_DECODE_16K, LLAMA70B_PREFILL_128K)}


@dataclass(frozen=True)
class DemoteShape:
    name: str = "llama3_demote_64k"
    B: int = 16
    H: int = 8
    D: int = 128
    S: int = 65536
    keep_hot: int = 1024
    hot_budget: int = 64  # protect_recent = min(16, hot_budget // 4) = 16
    block_t: int = 32
    group_v: int = 32


LLAMA3_DEMOTE_64K = DemoteShape()


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def _student_t3(shape, g, device) -> torch.Tensor:
    z = torch.randn(shape, generator=g, device=device)
    c = torch.randn((3,) + tuple(shape), generator=g, device=device).pow(2).sum(0)
    return z / torch.sqrt(c / 3.0)


def make_kv(shape: DecodeShape, layer: int = 0, device="cpu", dtype=torch.float16):
    """K, V (B, Hkv, N, D) with the shape's channel structure."""
    B, H, N, D = shape.B, shape.Hkv, shape.N, shape.D
    off = 16 * layer
    k = torch.randn((B, H, N, D), generator=_gen(SEED_K + off, device), device=device)
    v = torch.randn((B, H, N, D), generator=_gen(SEED_V + off, device), device=device)
    gch = _gen(SEED_CH + off, "cpu")
    if shape.k_outlier_channels:
        for h in range(H):
            ch = torch.randperm(D, generator=gch)[: shape.k_outlier_channels].to(device)
            k[:, h, :, ch] *= 10.0
    if shape.heavy_tail_channels:
        gt = _gen(SEED_CH + off + 8, device)
        for h in range(H):
            ch = torch.randperm(D, generator=gch)[: shape.heavy_tail_channels].to(device)
            k[:, h, :, ch] = _student_t3((B, N, len(ch)), gt, device)
            v[:, h, :, ch] = _student_t3((B, N, len(ch)), gt, device)
    return k.to(dtype), v.to(dtype)


def make_q(shape: DecodeShape, layer: int = 0, device="cpu", dtype=torch.float16) -> torch.Tensor:
    g = _gen(SEED_Q + 16 * layer, device)
    return torch.randn((shape.B, shape.Hq, shape.M, shape.D), generator=g, device=device).to(dtype)


def split_hot_warm(k: torch.Tensor, v: torch.Tensor, n_hot: int):
    """warm = positions [0, N - n_hot), hot = the last n_hot positions."""
    nw = k.shape[2] - n_hot
    return (k[:, :, :nw], v[:, :, :nw]), (k[:, :, nw:].contiguous(), v[:, :, nw:].contiguous())


def make_demote_inputs(shape: DemoteShape = LLAMA3_DEMOTE_64K, device="cpu", batch: Optional[int] = None):
    """K, V (B, H, S, D) fp16 and importance (B, S) fp32 ~ U(0, 1)."""
    B = shape.B if batch is None else batch
    k = torch.randn((B, shape.H, shape.S, shape.D), generator=_gen(SEED_K, device), device=device).half()
    v = torch.randn((B, shape.H, shape.S, shape.D), generator=_gen(SEED_V, device), device=device).half()
    imp = torch.rand((B, shape.S), generator=_gen(SEED_IMP, device), device=device)
    return k, v, imp
