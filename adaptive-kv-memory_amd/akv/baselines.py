"""The KIVI baselines of akv/baselines.py on the device.

``KIVICache`` (akv/baselines.py:249-403) quantizes the tokens that overflow a
full-precision residual window; ``KIVIFusedCache`` (:426-510) is its fused-kernel
cost profile: each overflow chunk is quantized once, appended, and dequantized once
into a float16 working copy.  The quantizer (``_quantize_tensor``, :345-370) is fp32
min / max per (row, group) of the last axis, scale clamped at 1e-10, codes
rounded half-to-even; here it is one ``akv_quant_pack`` launch (layout
``AKV_QUANT_ARENA`` on fp32 input, which is that arithmetic) and the dequant
(``_dequantize_tensor``, :372-380: fp32 ``codes * s + z`` cast to fp16) one
``akv_dequant_unpack`` launch -- both bit-exact with the reference.

Storage: per layer and for K and V, the codes bit-packed (2 / 4 / 8 bits; 4-bit
high nibble first, 2-bit MSB first) in ``[B * H][capacity][pD * bits / 8]`` and the
fp32 scales / zeros in ``[B * H][capacity][G]``, tokens in order, the capacity
doubling as the cache grows.  The reference keeps unpacked uint8 codes and
concatenates chunk after chunk along its flattened row axis
(``_concat_quant_chunks``, :513-535); the ``_quant_keys`` / ``_quant_values``
tiers here (indexable like those dicts: 'data', 'scales', 'zeros', 'shape', ...)
hold the packed codes in (batch, head, token) order instead.
``memory_bytes`` counts what the dicts and the residual hold, as the reference does.

``KIVIFusedCache.fused_attention`` (not in the reference: the throughput leg that
compares the baseline on the same kernels) is one ``akv_decode_attn`` launch over
the packed tier, read in place (legacy layout, one tier per (batch, head), fp16
copies of the scales / zeros kept beside the fp32 ones) and the residual window.

Head_dim 64 or 128, group sizes 32 / 64 / 128 and 2 / 4 / 8 bits are supported, as
for every quantizer of this build; other shapes raise ``NotImplementedError``.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional

import torch

from . import _native as nat
from ._legacy import legacy_desc, padded_dim


@dataclass
class KIVIConfig:
    """akv/baselines.py:236-246."""
    key_bits: int = 2
    value_bits: int = 2
    group_size: int = 128
    residual_length: int = 128


@dataclass
class KIVIFusedConfig(KIVIConfig):
    """akv/baselines.py:406-423."""


def _check_shape(D: int, bits: int, gs: int):
    if bits not in (2, 4, 8):
        raise NotImplementedError(f"the MI355X KIVI tier packs 2, 4 or 8 bits, got {bits}")
    if D not in (64, 128) or gs not in (32, 64, 128):
        raise NotImplementedError("the MI355X KIVI tier takes head_dim 64 or 128 and group_size 32, 64 or 128")


def quantize_rows(x: torch.Tensor, bits: int, group_size: int):
    """KIVICache._quantize_tensor (akv/baselines.py:345-370) for x (B, H, n, D):
    packed codes (B * H, n, pD * bits / 8) uint8 and fp32 scales / zeros
    (B * H, n, G), one launch."""
    nat.require_device(x)
    B, H, n, D = x.shape
    _check_shape(D, bits, group_size)
    xf = nat.dev_contig(x.float())
    pD = padded_dim(D, group_size)
    G = pD // group_size
    codes = torch.empty(1, B * H, n, pD * bits // 8, dtype=torch.uint8, device=x.device)
    sc = torch.empty(1, B * H, n, G, dtype=torch.float32, device=x.device)
    ze = torch.empty_like(sc)
    if n:
        a = nat.QuantArgs()
        a.abi_version = nat.ABI_VERSION
        a.B, a.H, a.D = 1, B * H, D
        a.in_dtype = nat.DT_F32
        a.layout = nat.QUANT_ARENA
        a.k = xf.data_ptr()
        a.n_src = a.n_sel = n
        a.bits_k = a.bits_v = bits
        a.block_t = 32
        a.group_v = group_size
        a.k_codes, a.k_scale, a.k_zero = codes.data_ptr(), sc.data_ptr(), ze.data_ptr()
        nat.check(nat.load().akv_quant_pack(ctypes.byref(a), nat.stream_of(xf)), "KIVI quantize")
    return codes[0], sc[0], ze[0]


def dequantize_rows(codes: torch.Tensor, sc: torch.Tensor, ze: torch.Tensor, bits: int, group_size: int,
                    D: int, n: Optional[int] = None) -> torch.Tensor:
    """KIVICache._dequantize_tensor (akv/baselines.py:372-380): (R, n, D) float16 of
    fp32 codes * s + z, for contiguous codes (R, S, pD * bits / 8) and fp32 meta
    (R, S, G) of which the first n <= S tokens of each row are read (n = S unless
    given), in one launch."""
    R, S = codes.shape[0], codes.shape[1]
    n = S if n is None else n
    out = torch.empty(R, n, D, dtype=torch.float16, device=codes.device)
    if R * n == 0:
        return out
    keep = []
    desc = legacy_desc(codes, sc, ze, codes, sc, ze, bits, group_size, S, D, warm_heads=R, sym=0, keep=keep)
    desc.n_warm = n
    desc.token_stride = S
    a = nat.DequantArgs()
    a.abi_version = nat.ABI_VERSION
    a.B, a.Hkv, a.D = 1, R, D
    a.out_dtype = nat.DT_F16
    a.warm = desc
    a.k_out = out.data_ptr()
    nat.check(nat.load().akv_dequant_unpack(ctypes.byref(a), nat.stream_of(out)), "KIVI dequantize")
    return out


class _Tier:
    """One layer's quantized K or V: packed codes and fp32 (and, for the fused
    attention, fp16) scales / zeros per (batch * head, token), tokens in order."""

    def __init__(self, B: int, H: int, D: int, bits: int, gs: int, device, keep_f16: bool):
        self.B, self.H, self.rows, self.D, self.bits, self.gs = B, H, B * H, D, bits, gs
        pD = padded_dim(D, gs)
        self.row_bytes, self.G = pD * bits // 8, pD // gs
        self.n, self.cap, self.keep_f16 = 0, 0, keep_f16
        self.device = device
        self.codes = self.sc = self.ze = self.sc16 = self.ze16 = None

    def _grow(self, need: int):
        cap = max(64, self.cap)
        while cap < need:
            cap *= 2
        def grow(t, shape, dtype):
            new = torch.zeros(shape, dtype=dtype, device=self.device)
            if t is not None and self.n:
                new[:, : self.n] = t[:, : self.n]
            return new
        R, G = self.rows, self.G
        self.codes = grow(self.codes, (R, cap, self.row_bytes), torch.uint8)
        self.sc = grow(self.sc, (R, cap, G), torch.float32)
        self.ze = grow(self.ze, (R, cap, G), torch.float32)
        if self.keep_f16:
            self.sc16 = grow(self.sc16, (R, cap, G), torch.float16)
            self.ze16 = grow(self.ze16, (R, cap, G), torch.float16)
        self.cap = cap

    def append(self, codes, sc, ze):
        n = codes.shape[1]
        if self.n + n > self.cap:
            self._grow(self.n + n)
        s = slice(self.n, self.n + n)
        self.codes[:, s] = codes
        self.sc[:, s] = sc
        self.ze[:, s] = ze
        if self.keep_f16:
            self.sc16[:, s] = sc
            self.ze16[:, s] = ze
        self.n += n

    def __getitem__(self, key: str):
        """The reference's quant dict entries over the tier ('data', 'scales', 'zeros':
        rows in (batch, head, token) order; 'shape', 'bits', 'group_size')."""
        n = self.n
        if key == "data":
            return self.codes[:, :n].reshape(self.rows * n, self.row_bytes)
        if key in ("scales", "zeros"):
            return (self.sc if key == "scales" else self.ze)[:, :n].reshape(self.rows * n, self.G)
        return {"shape": (self.B, self.H, n, self.D), "bits": self.bits, "group_size": self.gs}[key]

    def dequantize(self) -> torch.Tensor:
        """(B, H, n, D) float16, one launch over the tier in place."""
        return dequantize_rows(self.codes, self.sc, self.ze, self.bits, self.gs, self.D,
                               n=self.n).view(self.B, self.H, self.n, self.D)

    def nbytes(self) -> int:
        n = self.n
        return self.rows * n * (self.row_bytes + 2 * 4 * self.G)


class KIVICache:
    """akv/baselines.py:249-403: every overflow re-quantizes the merged history and
    every update dequantizes the whole quantized tier."""

    _keep_f16 = False

    def __init__(self, config: Optional[KIVIConfig] = None):
        self.config = config or KIVIConfig()
        self._quant_keys: dict = {}      # layer -> _Tier
        self._quant_values: dict = {}
        self._residual_keys: dict = {}
        self._residual_values: dict = {}
        self._seq_lens: dict = {}

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int,
               attention_weights: Optional[torch.Tensor] = None):
        """akv/baselines.py:268-289: (B, H, N, D) in, the layer's full K / V out."""
        cfg = self.config
        nat.require_device(key_states, value_states)
        if layer_idx not in self._residual_keys:
            self._residual_keys[layer_idx] = key_states
            self._residual_values[layer_idx] = value_states
            self._seq_lens[layer_idx] = key_states.shape[2]
        else:
            self._residual_keys[layer_idx] = torch.cat([self._residual_keys[layer_idx], key_states], dim=2)
            self._residual_values[layer_idx] = torch.cat([self._residual_values[layer_idx], value_states], dim=2)
            self._seq_lens[layer_idx] += key_states.shape[2]
        if self._residual_keys[layer_idx].shape[2] > cfg.residual_length:
            self._quantize_overflow(layer_idx)
        return self._get_full_kv(layer_idx)

    def _new_tier(self, x: torch.Tensor, bits: int) -> "_Tier":
        B, H, _, D = x.shape
        return _Tier(B, H, D, bits, self.config.group_size, x.device, self._keep_f16)

    def _quantize_overflow(self, layer_idx: int):
        """akv/baselines.py:291-322: quantize the overflow; merge by dequantizing the
        old tier, concatenating and quantizing the whole again."""
        cfg = self.config
        res_k, res_v = self._residual_keys[layer_idx], self._residual_values[layer_idx]
        n_q = res_k.shape[2] - cfg.residual_length
        tk, tv = res_k[:, :, :n_q], res_v[:, :, :n_q]
        if layer_idx in self._quant_keys:
            tk = torch.cat([self._quant_keys[layer_idx].dequantize(), tk], dim=2)
            tv = torch.cat([self._quant_values[layer_idx].dequantize(), tv], dim=2)
        kt, vt = self._new_tier(tk, cfg.key_bits), self._new_tier(tv, cfg.value_bits)
        kt.append(*quantize_rows(tk, cfg.key_bits, cfg.group_size))
        vt.append(*quantize_rows(tv, cfg.value_bits, cfg.group_size))
        self._quant_keys[layer_idx], self._quant_values[layer_idx] = kt, vt
        self._residual_keys[layer_idx] = res_k[:, :, n_q:].contiguous()
        self._residual_values[layer_idx] = res_v[:, :, n_q:].contiguous()

    def _get_full_kv(self, layer_idx: int):
        """akv/baselines.py:324-343."""
        rk, rv = self._residual_keys[layer_idx], self._residual_values[layer_idx]
        if layer_idx in self._quant_keys:
            return (torch.cat([self._quant_keys[layer_idx].dequantize(), rk], dim=2),
                    torch.cat([self._quant_values[layer_idx].dequantize(), rv], dim=2))
        return rk, rv

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self._seq_lens.get(layer_idx, 0)

    def reset(self):
        self._quant_keys.clear()
        self._quant_values.clear()
        self._residual_keys.clear()
        self._residual_values.clear()
        self._seq_lens.clear()

    def memory_bytes(self) -> int:
        """akv/baselines.py:392-403: quantized tiers (codes as stored here, packed) plus
        the residual windows."""
        total = sum(t.nbytes() for t in self._quant_keys.values()) + sum(t.nbytes() for t in self._quant_values.values())
        total += sum(k.nbytes for k in self._residual_keys.values()) + sum(v.nbytes for v in self._residual_values.values())
        return int(total)

    def __len__(self):
        return self.get_seq_length()


class KIVIFusedCache(KIVICache):
    """akv/baselines.py:426-510: incremental quantization of each overflow chunk and a
    float16 working copy extended by that chunk's dequant only."""

    _keep_f16 = True

    def __init__(self, config: Optional[KIVIFusedConfig] = None):
        super().__init__(config or KIVIFusedConfig())
        self._dequant_keys_cache: dict = {}
        self._dequant_values_cache: dict = {}
        self._ws: dict = {}  # per-device decode workspace of fused_attention

    def _quantize_overflow(self, layer_idx: int):
        """akv/baselines.py:455-496."""
        cfg = self.config
        res_k, res_v = self._residual_keys[layer_idx], self._residual_values[layer_idx]
        n_q = res_k.shape[2] - cfg.residual_length
        tk, tv = res_k[:, :, :n_q], res_v[:, :, :n_q]
        B, H, _, D = res_k.shape
        if layer_idx not in self._quant_keys:
            self._quant_keys[layer_idx] = self._new_tier(tk, cfg.key_bits)
            self._quant_values[layer_idx] = self._new_tier(tv, cfg.value_bits)
        kq = quantize_rows(tk, cfg.key_bits, cfg.group_size)
        vq = quantize_rows(tv, cfg.value_bits, cfg.group_size)
        self._quant_keys[layer_idx].append(*kq)
        self._quant_values[layer_idx].append(*vq)
        nk = dequantize_rows(*kq, cfg.key_bits, cfg.group_size, D).view(B, H, n_q, D)
        nv = dequantize_rows(*vq, cfg.value_bits, cfg.group_size, D).view(B, H, n_q, D)
        if layer_idx in self._dequant_keys_cache:
            self._dequant_keys_cache[layer_idx] = torch.cat([self._dequant_keys_cache[layer_idx], nk], dim=2)
            self._dequant_values_cache[layer_idx] = torch.cat([self._dequant_values_cache[layer_idx], nv], dim=2)
        else:
            self._dequant_keys_cache[layer_idx], self._dequant_values_cache[layer_idx] = nk, nv
        self._residual_keys[layer_idx] = res_k[:, :, n_q:].contiguous()
        self._residual_values[layer_idx] = res_v[:, :, n_q:].contiguous()

    def _get_full_kv(self, layer_idx: int):
        """akv/baselines.py:498-510."""
        rk, rv = self._residual_keys[layer_idx], self._residual_values[layer_idx]
        if layer_idx in self._dequant_keys_cache:
            return (torch.cat([self._dequant_keys_cache[layer_idx], rk], dim=2),
                    torch.cat([self._dequant_values_cache[layer_idx], rv], dim=2))
        return rk, rv

    def fused_attention(self, query: torch.Tensor, layer_idx: int, sm_scale: Optional[float] = None) -> torch.Tensor:
        """softmax(q K^T * sm_scale) V over the layer's quantized tier (in place) and its
        residual window, query (B, Hq, M, D) with Hq a multiple of the cache's heads;
        float16 out.  One decode launch."""
        cfg = self.config
        if cfg.key_bits != cfg.value_bits:
            raise NotImplementedError("fused_attention reads one code width for K and V")
        nat.require_device(query)
        rk, rv = self._residual_keys[layer_idx], self._residual_values[layer_idx]
        if rk.dtype != torch.float16:
            raise TypeError("fused_attention takes a float16 cache")
        B, H, n_res, D = rk.shape
        q = nat.dev_contig(query.to(torch.float16))
        _, Hq, M, _ = q.shape
        rk, rv = nat.dev_contig(rk), nat.dev_contig(rv)
        kt, vt = self._quant_keys.get(layer_idx), self._quant_values.get(layer_idx)
        out = torch.empty_like(q)
        a = nat.DecodeArgs()
        a.abi_version = nat.ABI_VERSION
        a.B, a.Hq, a.Hkv, a.M, a.D = B, Hq, H, M, D
        a.q_dtype = nat.DT_F16
        a.q = q.data_ptr()
        if n_res:
            a.k_hot, a.v_hot = rk.data_ptr(), rv.data_ptr()
        a.n_hot = n_res
        a.hot_first = 0
        a.sm_scale = D ** -0.5 if sm_scale is None else float(sm_scale)
        if kt is not None and kt.n:
            w = a.warm
            w.kind = nat.WARM_LEGACY
            w.bits_k = w.bits_v = cfg.key_bits
            w.n_warm = kt.n
            w.token_stride = kt.cap
            w.k_codes, w.v_codes = kt.codes.data_ptr(), vt.codes.data_ptr()
            w.k_scale, w.k_zero = kt.sc16.data_ptr(), kt.ze16.data_ptr()
            w.v_scale, w.v_zero = vt.sc16.data_ptr(), vt.ze16.data_ptr()
            w.group_size = cfg.group_size
            w.meta_dtype = nat.DT_F16
            w.warm_heads = B * H
            w.legacy_sym = 0
        else:
            a.warm.kind = nat.WARM_NONE
        a.out = out.data_ptr()
        lib = nat.load()
        nbytes = lib.akv_decode_workspace_bytes(ctypes.byref(a))
        if nbytes < 0:
            nat.check(lib.akv_decode_attn(ctypes.byref(a), None), "KIVIFusedCache.fused_attention")
        # one workspace per device, shared by every layer, batch size and query length
        ws = self._ws.setdefault(q.device, nat.DecodeWorkspace()).get(
            nbytes, lib.akv_decode_counter_bytes(ctypes.byref(a)), q.device)
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
        nat.check(lib.akv_decode_attn(ctypes.byref(a), nat.stream_of(q)), "KIVIFusedCache.fused_attention")
        return out

    def reset(self):
        super().reset()
        self._dequant_keys_cache.clear()
        self._dequant_values_cache.clear()


def create_baseline(name: str, **kwargs):
    """akv/baselines.py:1023-1054 for the KIVI baselines ('kivi', 'kivi_fused' and its
    synonyms); the other baselines of the reference are not part of this build."""
    key = name.lower().replace("-", "").replace("_", "")
    if key == "kivi":
        return KIVICache(KIVIConfig(**kwargs))
    if key in ("kivifused", "fusedkivi", "kiviincremental"):
        return KIVIFusedCache(KIVIFusedConfig(**kwargs))
    if key in ("full", "h2o", "snapkv", "scissorhands", "scissors", "streamingllm", "streaming", "pyramidkv",
               "pyramid"):
        raise NotImplementedError(f"baseline {name!r} is not part of the MI355X build (KIVI baselines only)")
    raise ValueError(f"Unknown baseline: {key}. Choose from: full, h2o, kivi, kivi_fused, snapkv, "
                     f"scissorhands, streamingllm, pyramidkv")
