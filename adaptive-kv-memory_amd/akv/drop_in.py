"""The drop-in cache: AKVCache (presets, protected layers, per-layer update)
and AKVLayer (hot fp16 tier + packed warm tier, akv/drop_in.py:169-1200).

``_PRESETS`` and the preset resolution of ``AKVCache.__init__`` follow
akv/drop_in.py:89-124 and :910-964.  ``select_demote_indices`` is
akv/drop_in.py:392-413 (first 4 and last min(16, hot_budget // 4) hot tokens
protected, lowest scores first, indices returned in ascending order).
``AKVLayer.update`` keeps each demotion event packed (codes + scale / zero) and
serves the chronological view from one dequant launch; the reference keeps a
float16 working copy of the same values (_quantize_per_head at
akv/drop_in.py:315-374 quantizes and immediately dequantizes).
``AKVCache.demote`` quantizes a chosen token set into a warm tier of 32-token
K blocks, for callers that drive the tiers themselves.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _native as nat
from .warm_tier import WarmTier, packed_row_bytes, quantize_kv

_PRESETS = {
    "quality": {
        "warm_bits": 4,
        "hot_budget": 256,
        "description": "Near-lossless 4-bit. +1-2% PPL.",
    },
    "balanced": {
        "warm_bits": 3,
        "hot_budget": 128,
        "description": "Block-affine 3-bit. +3.3% PPL, 5x compression.",
    },
    "compact": {
        "warm_bits": 2,
        "hot_budget": 64,
        "description": "Block-affine 2-bit. +11% PPL, 8x compression.",
    },
    "k4v2": {
        "warm_bits": 4,
        "warm_key_bits": 4,
        "warm_value_bits": 2,
        "hot_budget": 128,
        "description": "Asymmetric K4/V2. Keys preserved, values aggressively compressed.",
    },
    "k4v3": {
        "warm_bits": 4,
        "warm_key_bits": 4,
        "warm_value_bits": 3,
        "hot_budget": 128,
        "description": "Asymmetric K4/V3. Near-quality keys with balanced value compression.",
    },
}


def select_demote_indices(importance: Optional[torch.Tensor], n_demote: int, hot_len: int,
                          hot_budget: int, device=None) -> torch.Tensor:
    """akv/drop_in.py:392-413 on the device (importance (hot_len,) or (B, hot_len)).

    With no scores, or scores of another length, the reference falls back to FIFO
    (``arange(n_demote)``, akv/drop_in.py:401-403); that index lands on ``device``
    (else on the scores' device), where the gather that consumes it runs."""
    if importance is None or importance.shape[-1] != hot_len:
        dev = device if device is not None else (importance.device if importance is not None else None)
        if dev is None:
            raise ValueError("select_demote_indices: no scores and no device for the FIFO fallback")
        return torch.arange(n_demote, device=dev)
    nat.require_device(importance)
    if not 0 <= n_demote <= hot_len:
        raise ValueError(f"n_demote {n_demote} outside [0, {hot_len}]")
    protect_initial = 4
    protect_recent = min(16, hot_budget // 4)
    scores = nat.dev_contig(importance, torch.float32)
    rows = scores.numel() // hot_len if hot_len else 0
    idx = torch.empty(importance.shape[:-1] + (n_demote,), dtype=torch.int64, device=importance.device)
    lib = nat.load()
    nat.check(lib.akv_select_demote(scores.data_ptr(), rows, hot_len, n_demote, protect_initial, protect_recent,
                                    idx.data_ptr(), nat.stream_of(scores)), "select_demote_indices")
    return idx


def quantize_per_head(k: torch.Tensor, v: torch.Tensor, key_bits: int = 3, value_bits: int = 3,
                      per_head_bits: Optional[list] = None, group_size: int = 64,
                      outlier_fraction: float = 0.0) -> tuple[torch.Tensor, torch.Tensor, int]:
    """AKVLayer._quantize_per_head (akv/drop_in.py:315-374) on the device.

    k, v (B, H, n, D): one AffineQuantizer call per batch element over the n tokens
    (K per channel, V per token, outliers shared by the heads) -- or, when
    ``per_head_bits`` names a width for each head, one call per (batch element, head)
    with a quantizer of that width for K and V (the reference's pool keyed by bits;
    a head-count mismatch falls back to the global widths).  Returns the dequantized
    K, V (fp16, bit-exact with the reference) and the measured packed bytes of the
    event (packed_layout.measure_packed_bytes).  The reference squeezes a batch of
    one; here each batch element is its own call."""
    from .affine_quantizer import AffineQuantConfig, AffineQuantizer
    from .packed_layout import measure_packed_bytes
    nat.require_device(k, v)
    B, H, n, D = k.shape
    out_k = torch.empty(B, H, n, D, dtype=torch.float16, device=k.device)
    out_v = torch.empty_like(out_k)
    packed = 0
    if not per_head_bits or len(per_head_bits) != H:
        qz = AffineQuantizer(AffineQuantConfig(key_bits=key_bits, value_bits=value_bits, group_size=group_size,
                                               outlier_fraction=outlier_fraction))
        for b in range(B):
            qk, qv = qz.quantize_keys(k[b]), qz.quantize_values(v[b])
            packed += measure_packed_bytes(qk, key_bits) + measure_packed_bytes(qv, value_bits)
            out_k[b] = qz.dequantize_keys(qk)
            out_v[b] = qz.dequantize_values(qv)
        return out_k, out_v, packed
    pool = {}
    for bits in set(per_head_bits):
        pool[bits] = AffineQuantizer(AffineQuantConfig(key_bits=bits, value_bits=bits, group_size=group_size,
                                                       outlier_fraction=outlier_fraction))
    for b in range(B):
        for h, bits in enumerate(per_head_bits):
            qz = pool[bits]
            qk, qv = qz.quantize_keys(k[b, h:h + 1]), qz.quantize_values(v[b, h:h + 1])
            packed += measure_packed_bytes(qk, bits) + measure_packed_bytes(qv, bits)
            out_k[b, h] = qz.dequantize_keys(qk)[0]
            out_v[b, h] = qz.dequantize_values(qv)[0]
    return out_k, out_v, packed


class _EventTier:
    """The packed warm tier of one AKVLayer: demotion events appended in order.

    Per (batch, head) the codes, V scale / zero and outlier values of every warm
    token (``cap`` token rows), and per event the K scale / zero rows (``ecap``)
    and per batch element its outlier channels; ``blk`` maps each warm token to
    its event and ``pos`` to its chronological position.  Capacities double as
    tokens arrive."""

    def __init__(self, B, H, D, bits_k, bits_v, n_out, dev):
        self.B, self.H, self.D, self.bits_k, self.bits_v, self.n_out = B, H, D, bits_k, bits_v, n_out
        self.dev = dev
        self.n = 0
        self.n_events = 0
        self.cap = self.ecap = 0
        self.t = {}
        self._grow(256, 16)

    def _alloc(self, cap, ecap):
        B, H, D, n_out, dev = self.B, self.H, self.D, self.n_out, self.dev
        f16, u8 = torch.float16, torch.uint8
        t = {
            "kc": torch.empty(B, H, cap, packed_row_bytes(D, self.bits_k), dtype=u8, device=dev),
            "vc": torch.empty(B, H, cap, packed_row_bytes(D, self.bits_v), dtype=u8, device=dev),
            "vs": torch.empty(B, H, cap, 1, dtype=f16, device=dev),
            "vz": torch.empty(B, H, cap, 1, dtype=f16, device=dev),
            "ks": torch.empty(B, H, ecap, D, dtype=f16, device=dev),
            "kz": torch.empty(B, H, ecap, D, dtype=f16, device=dev),
            "blk": torch.empty(cap, dtype=torch.int32, device=dev),
            "pos": torch.empty(cap, dtype=torch.int64, device=dev),
        }
        if n_out:
            t["kod"] = torch.empty(B, H, cap, n_out, dtype=f16, device=dev)
            t["vod"] = torch.empty(B, H, cap, n_out, dtype=f16, device=dev)
            t["koi"] = torch.empty(B, ecap, n_out, dtype=torch.int64, device=dev)
            t["voi"] = torch.empty(B, ecap, n_out, dtype=torch.int64, device=dev)
        return t

    _TOKEN_AXIS = {"kc": 2, "vc": 2, "vs": 2, "vz": 2, "kod": 2, "vod": 2, "blk": 0, "pos": 0}

    def _grow(self, cap, ecap):
        t = self._alloc(cap, ecap)
        for name, old in self.t.items():
            if name in self._TOKEN_AXIS:
                t[name].narrow(self._TOKEN_AXIS[name], 0, self.n).copy_(old.narrow(self._TOKEN_AXIS[name], 0, self.n))
            else:
                ax = 2 if name in ("ks", "kz") else 1
                t[name].narrow(ax, 0, self.n_events).copy_(old.narrow(ax, 0, self.n_events))
        self.t, self.cap, self.ecap = t, cap, ecap

    def append(self, w: WarmTier, positions: torch.Tensor):
        """One demotion event: ``w`` holds its n tokens as a single K block."""
        n = w.n_warm
        if self.n + n > self.cap or self.n_events + 1 > self.ecap:
            self._grow(max(self.cap, 2 * (self.n + n)), max(self.ecap, 2 * (self.n_events + 1)))
        t, a, e = self.t, self.n, self.n_events
        t["kc"][:, :, a:a + n] = w.k_codes
        t["vc"][:, :, a:a + n] = w.v_codes
        t["vs"][:, :, a:a + n] = w.v_scale
        t["vz"][:, :, a:a + n] = w.v_zero
        t["ks"][:, :, e:e + 1] = w.k_scale
        t["kz"][:, :, e:e + 1] = w.k_zero
        if self.n_out:
            t["kod"][:, :, a:a + n] = w.k_odata
            t["vod"][:, :, a:a + n] = w.v_odata
            t["koi"][:, e:e + 1] = w.k_oidx
            t["voi"][:, e:e + 1] = w.v_oidx
        t["blk"][a:a + n] = e
        t["pos"][a:a + n] = positions
        self.n += n
        self.n_events += 1

    def resident_bytes(self) -> int:
        """Bytes of the used extents (codes, meta, outliers, event map, positions)."""
        total = 0
        for name, x in self.t.items():
            if name in self._TOKEN_AXIS:
                total += x.narrow(self._TOKEN_AXIS[name], 0, self.n).nbytes
            else:
                total += x.narrow(2 if name in ("ks", "kz") else 1, 0, self.n_events).nbytes
        return total

    def dequantize_into(self, out_k: torch.Tensor, out_v: Optional[torch.Tensor], slots: bool = True):
        """Dequantize every warm token into out_k / out_v (B, H, rows, D): at its
        chronological position when ``slots``, else at its warm-tier index (keys only
        when ``out_v`` is None)."""
        if self.n == 0:
            return
        t = self.t
        d = nat.WarmDesc()
        d.kind = nat.WARM_AFFINE
        d.bits_k, d.bits_v = self.bits_k, self.bits_v
        d.n_warm = self.n
        d.token_stride = self.cap
        d.block_t = 1
        d.group_v = self.D
        d.n_out = self.n_out
        d.k_codes, d.v_codes = t["kc"].data_ptr(), t["vc"].data_ptr()
        d.k_scale, d.k_zero = t["ks"].data_ptr(), t["kz"].data_ptr()
        d.v_scale, d.v_zero = t["vs"].data_ptr(), t["vz"].data_ptr()
        if self.n_out:
            d.k_oidx, d.v_oidx = t["koi"].data_ptr(), t["voi"].data_ptr()
            d.k_odata, d.v_odata = t["kod"].data_ptr(), t["vod"].data_ptr()
        a = nat.DequantArgs()
        a.abi_version = nat.ABI_VERSION
        a.B, a.Hkv, a.D = self.B, self.H, self.D
        a.out_dtype = nat.dtype_code(out_k.dtype)
        a.warm = d
        a.k_out = out_k.data_ptr()
        a.v_out = out_v.data_ptr() if out_v is not None else None
        a.block_of_token = t["blk"].data_ptr()
        a.n_blocks = self.ecap
        if slots:
            a.out_slot = t["pos"].data_ptr()
        a.out_tokens = out_k.shape[2]
        nat.check(nat.load().akv_dequant_unpack(ctypes.byref(a), nat.stream_of(out_k)), "AKVLayer warm view")

    def take(self, idx: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """The float16 values of warm tokens ``idx`` (warm-tier order), (B, H, n, D)."""
        n = idx.numel()
        sub = _EventTier.__new__(_EventTier)
        sub.__dict__.update({k: v for k, v in self.__dict__.items() if k != "t"})
        sub.t = {}
        for name, x in self.t.items():
            if name in self._TOKEN_AXIS:
                sub.t[name] = x.narrow(self._TOKEN_AXIS[name], 0, self.n).index_select(self._TOKEN_AXIS[name], idx)
            else:
                sub.t[name] = x
        sub.n, sub.cap = n, n
        k = torch.empty(self.B, self.H, n, self.D, dtype=torch.float16, device=self.dev)
        v = torch.empty_like(k)
        sub.dequantize_into(k, v, slots=False)
        return k, v

    def keep(self, keep_mask: torch.Tensor):
        """Drop the warm tokens where ``keep_mask`` is False (their events' K meta rows stay)."""
        kept = keep_mask.nonzero().flatten()
        for name, x in self.t.items():
            if name in self._TOKEN_AXIS:
                ax = self._TOKEN_AXIS[name]
                x.narrow(ax, 0, kept.numel()).copy_(x.narrow(ax, 0, self.n).index_select(ax, kept))
        self.n = kept.numel()

    def index_batch(self, beam_idx: torch.Tensor):
        for name in list(self.t):
            if name not in ("blk", "pos"):
                self.t[name] = self.t[name].index_select(0, beam_idx.to(self.dev))
        self.B = self.t["kc"].shape[0]


class _HeadBitsTier:
    """The packed warm tier when each head has its own code width (a calibration's
    ``per_head_bits``, akv/drop_in.py:315-374): one ``_EventTier`` per width over that
    width's heads, each (batch element, head) its own row -- the reference quantizes
    every head with its own AffineQuantizer of that width (the pool keyed by bits), so
    keys are per channel over the event's tokens of that head and the outlier channels
    are chosen per head.  Same interface as ``_EventTier``."""

    def __init__(self, B, H, D, per_head_bits, dev):
        self.B, self.H, self.D, self.dev = B, H, D, dev
        self.n = 0
        self.groups = []  # [bits, head indices on the device, _EventTier or None]
        for bits in sorted(set(per_head_bits)):
            heads = [h for h, b in enumerate(per_head_bits) if b == bits]
            self.groups.append([bits, torch.tensor(heads, dtype=torch.long, device=dev), None])

    def demote(self, hk, hv, idx, outlier_fraction, positions) -> int:
        """Quantize hot tokens ``idx`` of every head with its width as one event; returns
        the measured packed bytes (codes + scale + zero of K and V, per head)."""
        B, _, _, D = hk.shape
        n = idx.numel()
        packed = 0
        for g in self.groups:
            bits, heads, tier = g
            hs = heads.numel()
            k = hk.index_select(1, heads).index_select(2, idx).reshape(B * hs, 1, n, D)
            v = hv.index_select(1, heads).index_select(2, idx).reshape(B * hs, 1, n, D)
            w = quantize_kv(k, v, bits, bits, block_t=max(n, 1), group_v=D, outlier_fraction=outlier_fraction)
            if tier is None:
                g[2] = tier = _EventTier(B * hs, 1, D, bits, bits, w.n_out, self.dev)
            tier.append(w, positions)
            packed += (w.k_codes.nbytes + w.k_scale.nbytes + w.k_zero.nbytes
                       + w.v_codes.nbytes + w.v_scale.nbytes + w.v_zero.nbytes)
        self.n += n
        return packed

    def resident_bytes(self) -> int:
        return sum(g[2].resident_bytes() for g in self.groups if g[2] is not None)

    def dequantize_into(self, out_k: torch.Tensor, out_v: Optional[torch.Tensor], slots: bool = True):
        rows = out_k.shape[2]
        for bits, heads, tier in self.groups:
            hs = heads.numel()
            tk = torch.empty(self.B * hs, 1, rows, self.D, dtype=out_k.dtype, device=out_k.device)
            tv = torch.empty_like(tk) if out_v is not None else None
            tier.dequantize_into(tk, tv, slots)
            out_k.index_copy_(1, heads, tk.view(self.B, hs, rows, self.D))
            if out_v is not None:
                out_v.index_copy_(1, heads, tv.view(self.B, hs, rows, self.D))

    def take(self, idx: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        n = idx.numel()
        k = torch.empty(self.B, self.H, n, self.D, dtype=torch.float16, device=self.dev)
        v = torch.empty_like(k)
        for bits, heads, tier in self.groups:
            tk, tv = tier.take(idx)
            k.index_copy_(1, heads, tk.view(self.B, heads.numel(), n, self.D))
            v.index_copy_(1, heads, tv.view(self.B, heads.numel(), n, self.D))
        return k, v

    def keep(self, keep_mask: torch.Tensor):
        for g in self.groups:
            g[2].keep(keep_mask)
        self.n = int(keep_mask.sum())

    def index_batch(self, beam_idx: torch.Tensor):
        beam_idx = beam_idx.to(self.dev)
        for g in self.groups:
            hs = g[1].numel()
            rows = (beam_idx.unsqueeze(1) * hs + torch.arange(hs, device=self.dev)).flatten()
            g[2].index_batch(rows)
        self.B = beam_idx.numel()


class AKVLayer:
    """One layer of the drop-in cache (akv/drop_in.py:169-873) with the warm tier
    kept packed on the device.

    ``update`` follows akv/drop_in.py:591-787: new tokens join the hot tier with
    their positions; the importance vector decays by 0.3 and appends ones
    (:375-389); past the (adaptive) budget the lowest-importance unprotected
    tokens are chosen on the device (``select_demote_indices``), gathered and
    quantized as one demotion event (one ``akv_quant_pack`` launch: keys per
    channel over the event's tokens, values per token over all channels,
    outliers per event and batch element, the reference's AffineQuantizer), and
    the event's codes and scale / zero rows are appended to the packed tier --
    no float16 working copy is kept.  The returned view is chronological: one
    ``akv_dequant_unpack`` launch writes every warm token at its position and the
    hot tokens are scattered in beside it (float16, or float32 when the hot
    tokens are float32 / bfloat16, as the reference's torch.cat promotes).  The
    measured packed bytes count codes + scale + zero per event
    (packed_layout.measure_packed_bytes).

    Promotion (:415-589): with the proxy on, the EMA of |cos| between the mean
    new key and each warm token's key (dequantized, averaged over batch and
    heads) is kept per warm token; warm tokens above ``promotion_threshold`` --
    by the attention weights' warm columns when ``cache_kwargs`` carries them,
    else by the proxy -- return to the front of the hot tier with their float16
    values and importance 2.0, at most max(1, hot_budget // 8) per step, and
    leave the packed tier.

    Each batch element is its own quantizer call over (H, n, D) -- the
    reference's call on ``k.squeeze(0)`` at batch 1.  With ``per_head_bits`` naming
    a width for every head (a calibration's), each (batch element, head) is its own
    call at its width (``_HeadBitsTier``); of another head count, the global widths
    apply, as in the reference."""

    def __init__(self, warm_bits: int = 3, hot_budget: int = 128, group_size: int = 64, protect: bool = False,
                 enable_promotion: bool = True, promotion_threshold: float = 0.05,
                 per_head_bits: Optional[list] = None,
                 enable_promotion_proxy: bool = True, proxy_decay: float = 0.7, adaptive_hot_frac: float = 0.0,
                 warm_key_bits: Optional[int] = None, warm_value_bits: Optional[int] = None,
                 outlier_fraction: float = 0.0):
        self.warm_bits = warm_bits
        self.hot_budget = hot_budget
        self.group_size = group_size
        self.protect = protect
        self.enable_promotion = enable_promotion
        self.promotion_threshold = promotion_threshold
        self.enable_promotion_proxy = enable_promotion_proxy
        self.proxy_decay = proxy_decay
        self.adaptive_hot_frac = adaptive_hot_frac
        self.warm_key_bits = warm_key_bits or warm_bits
        self.warm_value_bits = warm_value_bits or warm_bits
        self.outlier_fraction = outlier_fraction
        self.per_head_bits = list(per_head_bits) if per_head_bits is not None else None
        self._hot_keys: Optional[torch.Tensor] = None
        self._hot_values: Optional[torch.Tensor] = None
        self._hot_positions: Optional[torch.Tensor] = None   # (N_hot,) int64, host
        self._warm: Optional[_EventTier] = None
        self._warm_positions: Optional[torch.Tensor] = None  # (N_warm,) int64, host
        self._warm_len = 0
        self._total_len = 0
        self._warm_bytes_packed = 0
        self._importance: Optional[torch.Tensor] = None      # (N_hot,) float32, device
        self._proxy_score: Optional[torch.Tensor] = None     # (N_warm,) float32, device
        self._decay = 0.3
        self._step = 0
        self.keys = self.values = None

    def get_seq_length(self) -> int:
        return self._total_len

    def _append_hot(self, k, v, pos):
        if self._hot_keys is None:
            self._hot_keys, self._hot_values, self._hot_positions = k, v, pos
        else:
            self._hot_keys = torch.cat([self._hot_keys, k], dim=2)
            self._hot_values = torch.cat([self._hot_values, v], dim=2)
            self._hot_positions = torch.cat([self._hot_positions, pos])

    def _update_importance(self, n_new: int, hot_len: int, device):
        """akv/drop_in.py:375-389 (recency decay, on the device)."""
        if self._importance is None or self._importance.shape[0] != hot_len - n_new:
            self._importance = torch.ones(hot_len, dtype=torch.float32, device=device)
        else:
            self._importance = torch.cat([self._importance * self._decay,
                                          torch.ones(n_new, dtype=torch.float32, device=device)])

    def _update_proxy_score(self, key_states: torch.Tensor):
        """akv/drop_in.py:486-525 over the packed tier: only its keys are dequantized (one
        launch, warm-tier order, no copy of the packed arrays)."""
        if self._warm is None or self._warm.n == 0:
            self._proxy_score = None
            return
        probe = key_states.detach().float().mean(dim=(0, 1, 2))
        probe = probe / (probe.norm() + 1e-6)
        w = self._warm
        wk = torch.empty(w.B, w.H, w.n, w.D, dtype=torch.float16, device=w.dev)
        w.dequantize_into(wk, None, slots=False)
        wk_flat = wk.float().mean(dim=(0, 1))
        wk_norm = wk_flat / (wk_flat.norm(dim=-1, keepdim=True) + 1e-6)
        sim = wk_norm @ probe
        if self._proxy_score is None or self._proxy_score.shape[0] != sim.shape[0]:
            self._proxy_score = sim.abs()
        else:
            d = self.proxy_decay
            self._proxy_score = d * self._proxy_score + (1 - d) * sim.abs()

    def _promote(self, scores: torch.Tensor, use_proxy: bool):
        """akv/drop_in.py:433-484 / :543-589: move the warm tokens above the threshold
        (at most max(1, hot_budget // 8), the top ones) to the front of the hot tier."""
        warm_len = self._warm.n
        mask = scores > self.promotion_threshold
        n = int(mask.sum().item())
        if n == 0:
            return
        cap = max(1, self.hot_budget // 8)
        if n > cap:
            _, top = scores.topk(cap)
            mask = torch.zeros_like(mask)
            mask[top] = True
            n = cap
        idx = mask.nonzero().flatten()
        pk, pv = self._warm.take(idx)
        idx_host = idx.cpu()
        positions = self._warm_positions[idx_host]
        keep = ~mask
        self._warm.keep(keep)
        self._warm_positions = self._warm_positions[keep.cpu()]
        if use_proxy:
            self._proxy_score = self._proxy_score[keep]
        self._warm_bytes_packed = int(self._warm_bytes_packed * (max(0, warm_len - n) / warm_len))
        self._warm_len -= n
        self._hot_keys = torch.cat([pk, self._hot_keys], dim=2)
        self._hot_values = torch.cat([pv, self._hot_values], dim=2)
        self._hot_positions = torch.cat([positions, self._hot_positions])
        if self._importance is not None:
            self._importance = torch.cat([torch.full((n,), 2.0, device=self._importance.device), self._importance])

    def _demote(self, n_demote: int, hot_len: int):
        hk, hv = self._hot_keys, self._hot_values
        dev = hk.device
        B, H, _, D = hk.shape
        idx = select_demote_indices(self._importance, n_demote, hot_len, self.hot_budget, device=dev)
        idx_host = idx.cpu()
        positions = self._hot_positions[idx_host]
        if self.per_head_bits and len(self.per_head_bits) == H:
            if self._warm is None:
                self._warm = _HeadBitsTier(B, H, D, self.per_head_bits, dev)
            self._warm_bytes_packed += self._warm.demote(hk, hv, idx, self.outlier_fraction, positions.to(dev))
        else:
            w = quantize_kv(hk, hv, self.warm_key_bits, self.warm_value_bits, block_t=max(n_demote, 1), group_v=D,
                            outlier_fraction=self.outlier_fraction, sel=idx.unsqueeze(0).expand(B, n_demote))
            if self._warm is None:
                self._warm = _EventTier(B, H, D, self.warm_key_bits, self.warm_value_bits, w.n_out, dev)
            self._warm.append(w, positions.to(dev))
            # measure_packed_bytes per batch element: packed codes + fp16 scale and zero, K and V
            self._warm_bytes_packed += (w.k_codes.nbytes + w.k_scale.nbytes + w.k_zero.nbytes
                                        + w.v_codes.nbytes + w.v_scale.nbytes + w.v_zero.nbytes)
        self._warm_positions = positions if self._warm_positions is None else torch.cat([self._warm_positions,
                                                                                         positions])
        self._warm_len += n_demote
        if self._proxy_score is not None:  # new warm tokens start with no evidence
            self._proxy_score = torch.cat([self._proxy_score,
                                           torch.zeros(n_demote, dtype=self._proxy_score.dtype, device=dev)])
        keep = torch.ones(hot_len, dtype=torch.bool)
        keep[idx_host] = False
        keep_dev = keep.to(dev)
        self._hot_keys = hk[:, :, keep_dev]
        self._hot_values = hv[:, :, keep_dev]
        self._hot_positions = self._hot_positions[keep]
        self._importance = self._importance[keep_dev]

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor,
               cache_kwargs: Optional[dict] = None) -> tuple[torch.Tensor, torch.Tensor]:
        """Append new KV, demote past the budget, return the chronological view."""
        nat.require_device(key_states, value_states)
        B, H, N, D = key_states.shape
        new_positions = torch.arange(self._total_len, self._total_len + N, dtype=torch.long)
        if self.protect:
            self._append_hot(key_states, value_states, new_positions)
            self._total_len += N
            self.keys, self.values = self._hot_keys, self._hot_values
            return self._hot_keys, self._hot_values
        self._append_hot(key_states, value_states, new_positions)
        self._total_len += N
        self._step += 1
        hot_len = self._hot_keys.shape[2]
        self._update_importance(N, hot_len, key_states.device)
        if self.enable_promotion_proxy:
            self._update_proxy_score(key_states)
        if self.enable_promotion and cache_kwargs and "attention_weights" in cache_kwargs:
            aw = cache_kwargs["attention_weights"]
            if self._warm is not None and self._warm.n and aw.dim() == 4 and aw.shape[-1] >= self._warm.n + hot_len:
                self._promote(aw[:, :, :, : self._warm.n].float().mean(dim=(0, 1, 2)), use_proxy=False)
            hot_len = self._hot_keys.shape[2]
        elif self.enable_promotion and self.enable_promotion_proxy:
            if (self._proxy_score is not None and self._warm is not None and self._warm.n
                    and self._proxy_score.shape[0] == self._warm.n):
                self._promote(self._proxy_score, use_proxy=True)
            hot_len = self._hot_keys.shape[2]
        budget = self.hot_budget
        if self.adaptive_hot_frac > 0.0:
            budget = max(self.hot_budget, int(self.adaptive_hot_frac * self._total_len))
        if hot_len > budget:
            self._demote(hot_len - budget, hot_len)
        if self._warm is None:
            self.keys, self.values = self._hot_keys, self._hot_values
            return self._hot_keys, self._hot_values
        hk, hv = self._hot_keys, self._hot_values
        out_dt = torch.float16 if hk.dtype == torch.float16 else torch.float32
        fk = torch.empty(B, H, self._total_len, D, dtype=out_dt, device=hk.device)
        fv = torch.empty_like(fk)
        self._warm.dequantize_into(fk, fv)
        hp = self._hot_positions.to(hk.device)
        fk.index_copy_(2, hp, hk.to(out_dt))
        fv.index_copy_(2, hp, hv.to(out_dt))
        self.keys, self.values = fk, fv
        return fk, fv

    def crop(self, max_length: int):
        """Keep positions 0 .. max_length-1 (the cache's ``crop``): hot tokens at or past
        it leave the hot tier with their importance, warm ones leave the packed tier with
        their proxy scores, and the length becomes max_length."""
        if self._total_len <= max_length:
            return
        if self._hot_keys is not None:
            keep = self._hot_positions < max_length
            if not bool(keep.all()):
                kd = keep.to(self._hot_keys.device)
                self._hot_keys = self._hot_keys[:, :, kd]
                self._hot_values = self._hot_values[:, :, kd]
                self._hot_positions = self._hot_positions[keep]
                if self._importance is not None and self._importance.shape[0] == keep.shape[0]:
                    self._importance = self._importance[kd]
        if self._warm is not None and self._warm_positions is not None:
            wkeep = self._warm_positions < max_length
            n_drop = int((~wkeep).sum())
            if n_drop:
                warm_len = int(wkeep.shape[0])
                self._warm.keep(wkeep.to(self._warm.dev))
                self._warm_positions = self._warm_positions[wkeep]
                if self._proxy_score is not None and self._proxy_score.shape[0] == warm_len:
                    self._proxy_score = self._proxy_score[wkeep.to(self._proxy_score.device)]
                self._warm_bytes_packed = int(self._warm_bytes_packed * ((warm_len - n_drop) / warm_len))
                self._warm_len -= n_drop
        self._total_len = max_length

    def warm_view(self) -> tuple[Optional[torch.Tensor], Optional[torch.Tensor]]:
        """The dequantized warm tier in demotion order (the reference's working copy)."""
        if self._warm is None:
            return None, None
        w = self._warm
        k = torch.empty(w.B, w.H, w.n, w.D, dtype=torch.float16, device=w.dev)
        v = torch.empty_like(k)
        w.dequantize_into(k, v, slots=False)
        return k, v

    def memory_usage_bytes(self) -> dict:
        """akv/drop_in.py:789-873; ``warm_bytes_live`` is what the packed tier holds
        resident (codes, meta, outlier values, event and position maps)."""
        H, D = 1, 128
        hot_bytes = 0
        if self._hot_keys is not None:
            hot_bytes = self._hot_keys.nbytes + self._hot_values.nbytes
            H, D = self._hot_keys.shape[1], self._hot_keys.shape[3]
        warm_live = self._warm.resident_bytes() if self._warm is not None else 0
        packed = int(self._warm_bytes_packed)
        formula = 0
        if self._warm_len > 0:
            groups = (D + self.group_size - 1) // self.group_size
            formula = self._warm_len * ((H * D * self.warm_bits + 7) // 8 + groups * H * 4) * 2
        total = hot_bytes + packed
        fp16_equiv = self._total_len * H * D * 2 * 2
        return {"hot_bytes": hot_bytes, "warm_bytes": packed, "warm_bytes_live": warm_live,
                "warm_bytes_packed": packed, "warm_bytes_formula": formula, "total_bytes": total,
                "fp16_equivalent_bytes": fp16_equiv, "savings_ratio": fp16_equiv / max(total, 1)}


class AKVCache:
    """The drop-in cache (akv/drop_in.py:885-1200): preset resolution, protected
    layers, lazily created ``AKVLayer``s driven by ``update`` (the method an HF
    model calls per layer), and ``demote`` (the warm-tier hot path with 32-token
    K blocks, for callers that manage the tiers themselves), with the reference's other
    cache methods (length queries, iteration, the legacy tuple form, crop, the beam
    helpers, reset, for_model, from_calibration).  Subclassing HF's ``DynamicCache`` is
    not part of this build."""

    def __init__(self, preset: Optional[str] = None, warm_bits: Optional[int] = None,
                 warm_key_bits: Optional[int] = None, warm_value_bits: Optional[int] = None,
                 hot_budget: Optional[int] = None, group_size: int = 64, outlier_fraction: float = 0.0,
                 protect_first: int = 0, protect_last: int = 0, protect_layers: Optional[list] = None,
                 num_hidden_layers: Optional[int] = None, enable_promotion: bool = True,
                 promotion_threshold: float = 0.05, enable_promotion_proxy: bool = True,
                 proxy_decay: float = 0.7, adaptive_hot_frac: float = 0.0,
                 block_t: int = 32, group_v: int = 32):
        if preset is not None:
            if preset not in _PRESETS:
                raise ValueError(f"Unknown preset {preset!r}. Choose from: {sorted(_PRESETS.keys())}")
            if warm_bits is not None or hot_budget is not None:
                raise ValueError(
                    "preset= is mutually exclusive with warm_bits/hot_budget. "
                    "Pick a preset OR pass explicit params.")
            p = _PRESETS[preset]
            self.warm_bits = p["warm_bits"]
            self.hot_budget = p["hot_budget"]
        else:
            self.warm_bits = warm_bits or 3
            self.hot_budget = hot_budget or 128
        if preset and "warm_key_bits" in _PRESETS.get(preset, {}):
            self.warm_key_bits = _PRESETS[preset]["warm_key_bits"]
            self.warm_value_bits = _PRESETS[preset]["warm_value_bits"]
        else:
            self.warm_key_bits = warm_key_bits or self.warm_bits
            self.warm_value_bits = warm_value_bits or self.warm_bits
        self.preset = preset
        self.group_size = group_size
        self.outlier_fraction = outlier_fraction
        self.num_hidden_layers = num_hidden_layers
        self.enable_promotion = enable_promotion
        self.promotion_threshold = promotion_threshold
        self.enable_promotion_proxy = enable_promotion_proxy
        self.proxy_decay = proxy_decay
        self.adaptive_hot_frac = adaptive_hot_frac
        self._protect_first = protect_first
        self._protect_last = protect_last
        self._protect_explicit = list(protect_layers) if protect_layers else []
        self.block_t = block_t
        self.group_v = group_v
        # protected layers (akv/drop_in.py:971-998)
        if protect_last > 0 and num_hidden_layers is None:
            raise ValueError("protect_last requires num_hidden_layers. "
                             "Use AKVCache.for_model(model, ...) or pass num_hidden_layers=.")
        self._protected_set: set = set(range(protect_first))
        if num_hidden_layers is not None:
            for i in range(protect_last):
                self._protected_set.add(num_hidden_layers - 1 - i)
            for p in self._protect_explicit:
                self._protected_set.add(p if p >= 0 else num_hidden_layers + p)
        else:
            for p in self._protect_explicit:
                if p < 0:
                    raise ValueError("Negative protect_layers indices require num_hidden_layers. "
                                     "Use AKVCache.for_model(model, ...).")
                self._protected_set.add(p)
        self.layers: list = []
        self._seen_tokens = 0
        self._calibration_per_head_bits: dict = {}

    def _is_protected(self, layer_idx: int) -> bool:
        return layer_idx in self._protected_set

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int,
               cache_kwargs: Optional[dict] = None) -> tuple[torch.Tensor, torch.Tensor]:
        """akv/drop_in.py:1066-1096: create layers lazily, count tokens on layer 0, delegate."""
        while len(self.layers) <= layer_idx:
            idx = len(self.layers)
            self.layers.append(AKVLayer(
                warm_bits=self.warm_bits, hot_budget=self.hot_budget, group_size=self.group_size,
                protect=self._is_protected(idx), enable_promotion=self.enable_promotion,
                promotion_threshold=self.promotion_threshold, enable_promotion_proxy=self.enable_promotion_proxy,
                proxy_decay=self.proxy_decay, adaptive_hot_frac=self.adaptive_hot_frac,
                warm_key_bits=self.warm_key_bits, warm_value_bits=self.warm_value_bits,
                outlier_fraction=self.outlier_fraction,
                per_head_bits=self._calibration_per_head_bits.get(idx) if self._calibration_per_head_bits else None))
        if layer_idx == 0:
            self._seen_tokens += key_states.shape[2]
        return self.layers[layer_idx].update(key_states, value_states, cache_kwargs)

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self.layers[layer_idx].get_seq_length() if layer_idx < len(self.layers) else 0

    def get_usable_length(self, max_length: int, layer_idx: int = 0) -> int:
        return self.get_seq_length(layer_idx)

    def get_max_length(self) -> Optional[int]:
        return None

    @property
    def seen_tokens(self) -> int:
        return self._seen_tokens

    @seen_tokens.setter
    def seen_tokens(self, value: int):
        self._seen_tokens = value

    def reorder_cache(self, beam_idx: torch.Tensor):
        """akv/drop_in.py:1119-1128: reorder the batch axis of both tiers."""
        for layer in self.layers:
            if layer._hot_keys is not None:
                layer._hot_keys = layer._hot_keys.index_select(0, beam_idx)
                layer._hot_values = layer._hot_values.index_select(0, beam_idx)
            if layer._warm is not None:
                layer._warm.index_batch(beam_idx)

    def memory_usage(self) -> dict:
        """akv/drop_in.py:1130-1160."""
        keys = ("hot_bytes", "warm_bytes", "warm_bytes_live", "warm_bytes_packed", "warm_bytes_formula",
                "total_bytes", "fp16_equivalent_bytes")
        totals = {k: 0 for k in keys}
        for layer in self.layers:
            stats = layer.memory_usage_bytes()
            for k in keys:
                totals[k] += stats.get(k, 0)
        totals["savings_ratio"] = totals["fp16_equivalent_bytes"] / max(totals["total_bytes"], 1)
        totals["num_layers"] = len(self.layers)
        return totals

    def memory_report(self) -> dict:
        """akv/drop_in.py:1162-1184."""
        stats = self.memory_usage()
        return {"compressed_bytes": stats["total_bytes"], "fp16_equiv_bytes": stats["fp16_equivalent_bytes"],
                "savings_ratio": round(stats["savings_ratio"], 2), "key_bits": self.warm_key_bits,
                "value_bits": self.warm_value_bits, "num_layers": stats["num_layers"],
                "seq_length": self.get_seq_length(0)}

    def __len__(self) -> int:
        return len(self.layers)

    def __getitem__(self, layer_idx: int):
        """akv/drop_in.py:1188-1198: (warm working copy in demotion order, then hot)."""
        if layer_idx < len(self.layers):
            layer = self.layers[layer_idx]
            if layer._hot_keys is not None:
                wk, wv = layer.warm_view()
                if wk is None:
                    return layer._hot_keys, layer._hot_values
                return (torch.cat([wk, layer._hot_keys], dim=2), torch.cat([wv, layer._hot_values], dim=2))
        return torch.tensor([]), torch.tensor([])

    def __iter__(self):
        for i in range(len(self.layers)):
            yield self[i]

    def to_legacy_cache(self):
        """akv/drop_in.py:1203-1205: ((keys, values) per layer) as ``__getitem__`` gives them."""
        return tuple(self[i] for i in range(len(self.layers)))

    @classmethod
    def from_legacy_cache(cls, past_key_values=None) -> "AKVCache":
        """akv/drop_in.py:1273-1280: a default cache fed layer by layer through ``update``."""
        cache = cls()
        if past_key_values is not None:
            for layer_idx, (k, v) in enumerate(past_key_values):
                cache.update(k, v, layer_idx)
        return cache

    @property
    def key_cache(self) -> list:
        """akv/drop_in.py:1214-1221: each layer's keys as ``__getitem__`` gives them."""
        return [self[i][0] for i in range(len(self.layers))]

    @property
    def value_cache(self) -> list:
        """akv/drop_in.py:1223-1229."""
        return [self[i][1] for i in range(len(self.layers))]

    def crop(self, max_length: int):
        """akv/drop_in.py:1231-1243 (speculative-decoding rewind): every layer keeps the
        positions before ``max_length`` (a negative value counts back from the current
        length, as transformers' caches take it).  The reference trims the hot tier from
        its end, where the newest tokens are; a token past max_length that was already
        demoted leaves the packed tier too here, so every layer's view stays whole."""
        for layer in self.layers:
            n = max_length if max_length >= 0 else max(0, layer.get_seq_length() + max_length)
            layer.crop(n)

    def batch_select_indices(self, indices: torch.Tensor) -> "AKVCache":
        """akv/drop_in.py:1256-1265 (beam search): keep / reorder batch elements."""
        self.reorder_cache(indices)
        return self

    def batch_repeat_interleave(self, repeats: int) -> "AKVCache":
        """akv/drop_in.py:1245-1254 (beam expansion): each batch element ``repeats`` times
        in a row, in both tiers."""
        for layer in self.layers:
            if layer._hot_keys is None:
                continue
            idx = torch.arange(layer._hot_keys.shape[0], device=layer._hot_keys.device).repeat_interleave(repeats)
            layer._hot_keys = layer._hot_keys.index_select(0, idx)
            layer._hot_values = layer._hot_values.index_select(0, idx)
            if layer._warm is not None:
                layer._warm.index_batch(idx)
        return self

    def reset(self):
        """akv/drop_in.py:1267-1270: empty (every layer dropped, no tokens seen)."""
        self.layers.clear()
        self._seen_tokens = 0

    @classmethod
    def for_model(cls, model, **kwargs) -> "AKVCache":
        """akv/drop_in.py:1012-1053: a cache sized from ``model.config``
        (num_hidden_layers, or n_layer), the other arguments as given.  The reference
        also applies per-family defaults from its model-adapter registry (preset and
        protected layers) when the caller leaves them out; that registry is not part of
        this build, so pass them explicitly."""
        config = getattr(model, "config", None)
        if config is None:
            raise ValueError("model has no .config attribute")
        n_layers = getattr(config, "num_hidden_layers", None) or getattr(config, "n_layer", None)
        if n_layers is None:
            raise ValueError("Could not find num_hidden_layers in model.config. Pass num_hidden_layers= explicitly.")
        return cls(num_hidden_layers=n_layers, **kwargs)

    @classmethod
    def from_calibration(cls, calibration_path, **overrides) -> "AKVCache":
        """akv/drop_in.py:1282-1315: a cache from a calibration report (JSON, the
        reference's CalibrationReport fields): its protected layers and layer count, its
        average width when within [2, 4] bits (else its preset), and its per-(layer, head)
        widths; ``overrides`` win."""
        import json
        with open(calibration_path) as f:
            rep = json.load(f)
        kwargs = dict(protect_first=rep["recommended_protect_first"], protect_last=rep["recommended_protect_last"],
                      num_hidden_layers=rep["num_layers"])
        avg = float(rep["recommended_average_bits"])
        if 2.0 <= avg <= 4.0:
            kwargs["warm_bits"] = int(round(avg))
        else:
            kwargs["preset"] = rep["recommended_preset"]
        kwargs.update(overrides)
        cache = cls(**kwargs)
        cache._calibration_per_head_bits = {int(k): list(v) for k, v in rep.get("per_head_bits", {}).items()}
        return cache

    def demote(self, keys: torch.Tensor, values: torch.Tensor, importance: Optional[torch.Tensor],
               n_demote: int) -> tuple[WarmTier, torch.Tensor]:
        """Pick ``n_demote`` hot tokens per sequence (lowest importance, protected
        ends kept) and quantize them into a packed warm tier.

        keys / values: (B, H, hot_len, D) on the device; importance: (B, hot_len)
        or (hot_len,).  Returns (warm tier, selected indices (B, n_demote))."""
        B, H, hot_len, D = keys.shape
        idx = select_demote_indices(importance, n_demote, hot_len, self.hot_budget, device=keys.device)
        if idx.dim() == 1:
            idx = idx.unsqueeze(0).expand(B, -1)
        warm = quantize_kv(keys, values, self.warm_key_bits, self.warm_value_bits, self.block_t,
                           self.group_v, self.outlier_fraction, sel=idx)
        return warm, idx


def recommend_preset(model, tokenizer=None, sample_text: Optional[str] = None) -> dict:
    """akv/drop_in.py:1321-1366: a preset suggestion from ``model.config`` by a rough
    size estimate, layers x kv-heads x head_dim^2 x 4 (the reference's heuristic and
    its thresholds: above 5e9 balanced 3-bit, above 1e9 quality 4-bit with a 256-token
    hot window, else quality 4-bit with 512 and two protected layers at each end)."""
    config = getattr(model, "config", None)
    if config is None:
        return {"preset": "balanced", "reason": "No config found, using default"}
    n_layers = getattr(config, "num_hidden_layers", 32)
    n_heads = getattr(config, "num_key_value_heads", getattr(config, "num_attention_heads", 32))
    head_dim = getattr(config, "head_dim", getattr(config, "hidden_size", 4096) // getattr(config, "num_attention_heads", 32))
    est = n_layers * n_heads * head_dim * head_dim * 4
    if est > 5e9:
        return {"preset": "balanced", "warm_bits": 3, "hot_budget": 128, "protect_first": 2, "protect_last": 2,
                "reason": f"Large model ({est / 1e9:.0f}B est.) \u2014 robust to 3-bit"}
    if est > 1e9:
        return {"preset": "quality", "warm_bits": 4, "hot_budget": 256, "protect_first": 1, "protect_last": 1,
                "reason": f"Medium model ({est / 1e9:.1f}B est.) \u2014 use 4-bit for safety"}
    return {"preset": "quality", "warm_bits": 4, "hot_budget": 512, "protect_first": 2, "protect_last": 2,
            "reason": f"Small model ({est / 1e9:.1f}B est.) \u2014 protect more layers"}
