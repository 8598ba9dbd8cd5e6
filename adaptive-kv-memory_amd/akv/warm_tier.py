"""Block-affine warm tier on the device: quantize + pack, dequant, fused decode.

This is the MI355X-native form of AKV's warm tier.  Per (batch, kv-head):

  * K: AffineQuantizer.quantize_keys (akv/affine_quantizer.py:63-110) on each
    block of ``block_t`` tokens -- one fp16 scale/zero per channel per block;
  * V: AffineQuantizer.quantize_values (akv/affine_quantizer.py:131-176) per
    token, over each group of ``group_v`` channels (group_v = D is the
    reference's single per-token scale);
  * codes bit-packed along D in the akv/bitpack.py layout;
  * optional fp16 outlier channels per (batch, block), shared by the heads.

``block_t = N`` and ``group_v = D`` reproduce one AffineQuantizer call.
Everything runs in libakv_hip.so; there is no CPU path.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional, Tuple

import torch

from . import _native as nat


def packed_row_bytes(dim: int, bits: int) -> int:
    """Bytes of one bit-packed row of ``dim`` codes (akv/bitpack.py padding rules)."""
    if bits == 4:
        return (dim + 1) // 2
    if bits == 3:
        return 3 * ((dim + 7) // 8)
    if bits == 2:
        return (dim + 3) // 4
    return dim


@dataclass
class WarmTier:
    """Packed warm tier of a (B, Hkv, Nw, D) K/V cache."""
    k_codes: torch.Tensor          # (B, Hkv, Nw, D*bits_k/8) uint8
    k_scale: torch.Tensor          # (B, Hkv, nblk, D) float16
    k_zero: torch.Tensor
    v_codes: torch.Tensor          # (B, Hkv, Nw, D*bits_v/8) uint8
    v_scale: torch.Tensor          # (B, Hkv, Nw, D/group_v) float16
    v_zero: torch.Tensor
    bits_k: int
    bits_v: int
    block_t: int
    group_v: int
    head_dim: int
    k_oidx: Optional[torch.Tensor] = None   # (B, nblk, n_out) int64
    v_oidx: Optional[torch.Tensor] = None
    k_odata: Optional[torch.Tensor] = None  # (B, Hkv, Nw, n_out) float16
    v_odata: Optional[torch.Tensor] = None

    @property
    def batch(self) -> int:
        return self.k_codes.shape[0]

    @property
    def heads(self) -> int:
        return self.k_codes.shape[1]

    @property
    def n_warm(self) -> int:
        return self.k_codes.shape[2]

    @property
    def n_out(self) -> int:
        return 0 if self.k_oidx is None else self.k_oidx.shape[-1]

    @property
    def device(self):
        return self.k_codes.device

    def nbytes(self) -> int:
        """Bytes the packed tier occupies (codes + scale/zero + outliers)."""
        ts = [self.k_codes, self.k_scale, self.k_zero, self.v_codes, self.v_scale, self.v_zero,
              self.k_oidx, self.v_oidx, self.k_odata, self.v_odata]
        return int(sum(t.numel() * t.element_size() for t in ts if t is not None))

    def desc(self) -> nat.WarmDesc:
        d = nat.WarmDesc()
        d.kind = nat.WARM_AFFINE
        d.bits_k, d.bits_v = self.bits_k, self.bits_v
        d.n_warm = self.n_warm
        d.block_t, d.group_v, d.n_out = self.block_t, self.group_v, self.n_out
        d.k_codes, d.v_codes = self.k_codes.data_ptr(), self.v_codes.data_ptr()
        d.k_scale, d.k_zero = self.k_scale.data_ptr(), self.k_zero.data_ptr()
        d.v_scale, d.v_zero = self.v_scale.data_ptr(), self.v_zero.data_ptr()
        if self.n_out:
            d.k_oidx, d.v_oidx = self.k_oidx.data_ptr(), self.v_oidx.data_ptr()
            d.k_odata, d.v_odata = self.k_odata.data_ptr(), self.v_odata.data_ptr()
        d.legacy_sym = 0
        return d


def n_outliers(head_dim: int, outlier_fraction: float) -> int:
    """akv/affine_quantizer.py:77: max(1, int(D * f)) when f > 0."""
    return max(1, int(head_dim * outlier_fraction)) if outlier_fraction > 0 else 0


def quantize_kv(k: torch.Tensor, v: torch.Tensor, bits_k: int = 3, bits_v: int = 3,
                block_t: int = 32, group_v: int = 32, outlier_fraction: float = 0.0,
                sel: Optional[torch.Tensor] = None) -> WarmTier:
    """Gather (optional ``sel`` (B, n) token indices) -> quantize -> pack.

    k, v: (B, Hkv, N, D) float16 / bfloat16 / float32 on the device."""
    nat.require_device(k, v, sel)
    lib = nat.load()
    if k.shape != v.shape or k.dim() != 4:
        raise ValueError("k and v must both be (B, H, N, D)")
    k = nat.dev_contig(k)
    v = nat.dev_contig(v, k.dtype)
    B, H, N, D = k.shape
    n_sel = N if sel is None else sel.shape[-1]
    if sel is not None:
        sel = nat.dev_contig(sel.reshape(B, n_sel), torch.int64)
    nblk = (n_sel + block_t - 1) // block_t if n_sel else 0
    dev = k.device
    u8 = torch.uint8
    kc = torch.empty(B, H, n_sel, packed_row_bytes(D, bits_k), dtype=u8, device=dev)
    vc = torch.empty(B, H, n_sel, packed_row_bytes(D, bits_v), dtype=u8, device=dev)
    ks = torch.empty(B, H, nblk, D, dtype=torch.float16, device=dev)
    kz = torch.empty_like(ks)
    if D % group_v:
        raise ValueError("group_v must divide head_dim")
    vs = torch.empty(B, H, n_sel, D // group_v, dtype=torch.float16, device=dev)
    vz = torch.empty_like(vs)
    n_out = n_outliers(D, outlier_fraction)
    koi = voi = kod = vod = None
    if n_out:
        koi = torch.empty(B, nblk, n_out, dtype=torch.int64, device=dev)
        voi = torch.empty_like(koi)
        kod = torch.empty(B, H, n_sel, n_out, dtype=torch.float16, device=dev)
        vod = torch.empty_like(kod)
    a = nat.QuantArgs()
    a.abi_version = nat.ABI_VERSION
    a.B, a.H, a.D = B, H, D
    a.in_dtype = nat.dtype_code(k.dtype)
    a.layout = nat.QUANT_AFFINE
    a.k, a.v = k.data_ptr(), v.data_ptr()
    a.n_src = N
    a.sel = sel.data_ptr() if sel is not None else None
    a.n_sel = n_sel
    a.bits_k, a.bits_v, a.block_t, a.group_v, a.n_out = bits_k, bits_v, block_t, group_v, n_out
    a.k_codes, a.k_scale, a.k_zero = kc.data_ptr(), ks.data_ptr(), kz.data_ptr()
    a.v_codes, a.v_scale, a.v_zero = vc.data_ptr(), vs.data_ptr(), vz.data_ptr()
    if n_out:
        a.k_oidx, a.v_oidx = koi.data_ptr(), voi.data_ptr()
        a.k_odata, a.v_odata = kod.data_ptr(), vod.data_ptr()
    nat.check(lib.akv_quant_pack(ctypes.byref(a), nat.stream_of(k)), "quantize_kv")
    return WarmTier(kc, ks, kz, vc, vs, vz, bits_k, bits_v, block_t, group_v, D, koi, voi, kod, vod)


def dequantize(warm: WarmTier, which: str = "kv") -> Tuple[Optional[torch.Tensor], Optional[torch.Tensor]]:
    """fp16 (B, Hkv, Nw, D) K and/or V, bit-exact with AffineQuantizer.dequantize_*."""
    lib = nat.load()
    B, H, Nw, D = warm.batch, warm.heads, warm.n_warm, warm.head_dim
    dev = warm.device
    ko = torch.empty(B, H, Nw, D, dtype=torch.float16, device=dev) if "k" in which else None
    vo = torch.empty(B, H, Nw, D, dtype=torch.float16, device=dev) if "v" in which else None
    a = nat.DequantArgs()
    a.abi_version = nat.ABI_VERSION
    a.B, a.Hkv, a.D = B, H, D
    a.out_dtype = nat.DT_F16
    a.warm = warm.desc()
    a.k_out = ko.data_ptr() if ko is not None else None
    a.v_out = vo.data_ptr() if vo is not None else None
    nat.check(lib.akv_dequant_unpack(ctypes.byref(a), nat.stream_of(warm.k_codes)), "dequantize")
    return ko, vo


def _hot_ptrs(k_hot, v_hot, q):
    if k_hot is None or k_hot.shape[2] == 0:
        return None, None, 0
    k_hot = nat.dev_contig(k_hot, q.dtype)
    v_hot = nat.dev_contig(v_hot, q.dtype)
    return k_hot, v_hot, k_hot.shape[2]


def run_decode(q: torch.Tensor, k_hot, v_hot, desc: Optional[nat.WarmDesc], Hkv: int,
               sm_scale: Optional[float] = None, hot_first: bool = True,
               scores: Optional[torch.Tensor] = None, decay: float = 0.9,
               return_weights: bool = False, num_splits: int = 0, keep=()):
    """Shared launcher of akv_decode_attn.  Returns (out, weights or None)."""
    lib = nat.load()
    nat.require_device(q, k_hot, v_hot, scores)
    if q.dtype != torch.float16:
        raise TypeError("the MI355X decode kernel takes float16 queries")
    q = nat.dev_contig(q)
    B, Hq, M, D = q.shape
    k_hot, v_hot, n_hot = _hot_ptrs(k_hot, v_hot, q)
    n_warm = desc.n_warm if desc is not None and desc.kind != nat.WARM_NONE else 0
    N = n_hot + n_warm
    out = torch.empty_like(q)
    attn = torch.empty(B, Hq, M, N, dtype=torch.float32, device=q.device) if return_weights else None
    a = nat.DecodeArgs()
    a.abi_version = nat.ABI_VERSION
    a.B, a.Hq, a.Hkv, a.M, a.D = B, Hq, Hkv, M, D
    a.q_dtype = nat.DT_F16
    a.q = q.data_ptr()
    if n_hot:
        a.k_hot, a.v_hot = k_hot.data_ptr(), v_hot.data_ptr()
    a.n_hot = n_hot
    a.hot_first = 1 if hot_first else 0
    a.sm_scale = nat.default_sm_scale(D) if sm_scale is None else float(sm_scale)
    if desc is not None:
        a.warm = desc
    else:
        a.warm.kind = nat.WARM_NONE
    a.out = out.data_ptr()
    a.attn_weights = attn.data_ptr() if attn is not None else None
    sc_buf = None
    if scores is not None:
        if scores.dtype == torch.float32 and scores.is_contiguous() and scores.data_ptr() % 16 == 0:
            sc_buf = scores
        else:
            sc_buf = nat.dev_contig(scores, torch.float32).clone()
        a.scores = sc_buf.data_ptr()
        a.n_scores = sc_buf.numel()
        a.decay = float(decay)
    a.num_splits = int(num_splits)
    nbytes = lib.akv_decode_workspace_bytes(ctypes.byref(a))
    if nbytes < 0:
        nat.check(lib.akv_decode_attn(ctypes.byref(a), None), "decode_attention")
    ws = nat.workspace(nbytes, q.device, zero_prefix=lib.akv_decode_counter_bytes(ctypes.byref(a)))
    a.workspace = ws.data_ptr()
    a.workspace_bytes = ws.numel()
    nat.check(lib.akv_decode_attn(ctypes.byref(a), nat.stream_of(q)), "decode_attention")
    if scores is not None and sc_buf is not scores:
        scores.copy_(sc_buf.view_as(scores))
    return out, attn


def decode_attention(q: torch.Tensor, k_hot: Optional[torch.Tensor], v_hot: Optional[torch.Tensor],
                     warm: Optional[WarmTier], sm_scale: Optional[float] = None, hot_first: bool = False,
                     scores: Optional[torch.Tensor] = None, decay: float = 0.9,
                     return_weights: bool = False, num_splits: int = 0):
    """Fused dequant-attention of q (B, Hq, M, D) fp16 over hot fp16 (B, Hkv, Nh, D)
    and the packed warm tier; grouped-query heads share kv head h // (Hq // Hkv).

    ``hot_first`` picks the logical token order of the returned weights and of
    ``scores`` ([hot, warm] like the reference's mixed ops, or chronological
    [warm, hot] like AKVLayer).  ``scores`` (N,) fp32 gets the importance EMA
    scores = scores*decay + sum_m mean_{b,h} attn in place."""
    Hkv = warm.heads if warm is not None else k_hot.shape[1]
    out, attn = run_decode(q, k_hot, v_hot, warm.desc() if warm is not None else None, Hkv, sm_scale,
                           hot_first, scores, decay, return_weights, num_splits)
    return (out, attn) if return_weights else out


def prefill_attention(q: torch.Tensor, k_hot: Optional[torch.Tensor], v_hot: Optional[torch.Tensor],
                      warm: Optional[WarmTier], sm_scale: Optional[float] = None,
                      num_splits: int = 0, k_chunk: Optional[torch.Tensor] = None,
                      v_chunk: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Chunked-prefill attention: q (B, Hq, M, D) fp16 or bf16 -- M positions
    after every cached token, so no mask over the cache -- over hot fp16
    (B, Hkv, Nh, D) and the packed warm tier; returns (B, Hq, M, D) in q's
    dtype.  No attention weights (the M x N matrix is never formed).

    ``k_chunk`` / ``v_chunk`` (B, Hkv, M, D) in q's dtype are the chunk's own keys
    and values: with them every position m also attends to chunk tokens 0..m
    (causal self-attention of the chunk, after the cache)."""
    lib = nat.load()
    nat.require_device(q, k_hot, v_hot, k_chunk, v_chunk)
    if q.dtype not in (torch.float16, torch.bfloat16):
        raise TypeError("prefill takes float16 or bfloat16 queries")
    q = nat.dev_contig(q)
    B, Hq, M, D = q.shape
    k_hot, v_hot, n_hot = _hot_ptrs(k_hot, v_hot, q.new_empty(0, dtype=torch.float16))
    Hkv = warm.heads if warm is not None else (k_hot.shape[1] if n_hot else
                                               (k_chunk.shape[1] if k_chunk is not None else 0))
    if (k_chunk is None) != (v_chunk is None):
        raise ValueError("k_chunk and v_chunk go together")
    if k_chunk is not None:
        for t in (k_chunk, v_chunk):
            if t.dtype != q.dtype or tuple(t.shape) != (B, Hkv, M, D):
                raise ValueError(f"k_chunk / v_chunk must be ({B}, {Hkv}, {M}, {D}) in {q.dtype}")
        k_chunk, v_chunk = nat.dev_contig(k_chunk), nat.dev_contig(v_chunk)
    out = torch.empty_like(q)
    a = nat.PrefillArgs()
    a.abi_version = nat.ABI_VERSION
    a.B, a.Hq, a.Hkv, a.M, a.D = B, Hq, Hkv, M, D
    a.q_dtype = nat.dtype_code(q.dtype)
    a.q = q.data_ptr()
    if n_hot:
        a.k_hot, a.v_hot = k_hot.data_ptr(), v_hot.data_ptr()
    a.n_hot = n_hot
    a.sm_scale = nat.default_sm_scale(D) if sm_scale is None else float(sm_scale)
    if warm is not None:
        a.warm = warm.desc()
    else:
        a.warm.kind = nat.WARM_NONE
    a.out = out.data_ptr()
    a.num_splits = int(num_splits)
    if k_chunk is not None:
        a.k_chunk, a.v_chunk = k_chunk.data_ptr(), v_chunk.data_ptr()
    nbytes = lib.akv_prefill_workspace_bytes(ctypes.byref(a))
    if nbytes < 0:
        nat.check(lib.akv_prefill_attn(ctypes.byref(a), None), "prefill_attention")
    ws = nat.workspace(nbytes, q.device) if nbytes > 0 else None
    if ws is not None:
        a.workspace = ws.data_ptr()
        a.workspace_bytes = ws.numel()
    nat.check(lib.akv_prefill_attn(ctypes.byref(a), nat.stream_of(q)), "prefill_attention")
    return out


class DecodeCall:
    """A prepared ``akv_decode_attn`` call on fixed device tensors.

    The args struct and workspace are built once; ``__call__`` only enqueues
    the kernels on the current stream, so the call can be replayed in a tight
    loop or captured in a HIP graph (the library issues no memset and no
    allocation)."""

    def __init__(self, q, k_hot, v_hot, warm: Optional[WarmTier], out: Optional[torch.Tensor] = None,
                 sm_scale: Optional[float] = None, hot_first: bool = False,
                 scores: Optional[torch.Tensor] = None, decay: float = 0.9,
                 attn_weights: Optional[torch.Tensor] = None, num_splits: int = 0):
        lib = nat.load()
        nat.require_device(q, k_hot, v_hot, scores, attn_weights)
        if q.dtype != torch.float16:
            raise TypeError("the MI355X decode kernel takes float16 queries")
        for t in (q, k_hot, v_hot, scores, attn_weights, out):
            if t is not None and (not t.is_contiguous() or t.data_ptr() % 16):
                raise ValueError("DecodeCall takes contiguous 16-byte-aligned tensors")
        if scores is not None and scores.dtype != torch.float32:
            raise TypeError("scores must be float32")
        B, Hq, M, D = q.shape
        self.q, self.k_hot, self.v_hot, self.warm = q, k_hot, v_hot, warm
        self.out = torch.empty_like(q) if out is None else out
        self.scores, self.attn_weights = scores, attn_weights
        a = nat.DecodeArgs()
        a.abi_version = nat.ABI_VERSION
        a.B, a.Hq, a.M, a.D = B, Hq, M, D
        a.Hkv = warm.heads if warm is not None else k_hot.shape[1]
        a.q_dtype = nat.DT_F16
        a.q = q.data_ptr()
        n_hot = 0 if k_hot is None else k_hot.shape[2]
        if n_hot:
            a.k_hot, a.v_hot = k_hot.data_ptr(), v_hot.data_ptr()
        a.n_hot = n_hot
        a.hot_first = 1 if hot_first else 0
        a.sm_scale = nat.default_sm_scale(D) if sm_scale is None else float(sm_scale)
        if warm is not None:
            a.warm = warm.desc()
        else:
            a.warm.kind = nat.WARM_NONE
        a.out = self.out.data_ptr()
        a.attn_weights = attn_weights.data_ptr() if attn_weights is not None else None
        if scores is not None:
            a.scores = scores.data_ptr()
            a.n_scores = scores.numel()
            a.decay = float(decay)
        a.num_splits = int(num_splits)
        nbytes = lib.akv_decode_workspace_bytes(ctypes.byref(a))
        if nbytes < 0:
            nat.check(nat.AKV_E_INVALID, "DecodeCall: " + (lib.akv_last_error() or b"").decode())
        self.workspace = nat.workspace(nbytes, q.device, zero_prefix=lib.akv_decode_counter_bytes(ctypes.byref(a)))
        a.workspace = self.workspace.data_ptr()
        a.workspace_bytes = self.workspace.numel()
        self.args = a
        self._lib = lib
        self._ref = ctypes.byref(a)

    def __call__(self) -> torch.Tensor:
        rc = self._lib.akv_decode_attn(self._ref, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        if rc:
            nat.check(rc, "DecodeCall")
        return self.out
