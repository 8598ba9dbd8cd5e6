"""Oracle restatement of ``AKVLayer.update`` (akv/drop_in.py:591-787), its
promotion paths (akv/drop_in.py:415-589) and ``memory_usage_bytes``' packed-byte
counter.

Per call with (B, H, N, D) keys / values:
  * positions [total, total + N) are appended to the hot positions and the
    tokens to the hot tier (akv/drop_in.py:600-644);
  * importance: ones(hot_len) when the old vector does not have hot_len - N
    entries, else old * 0.3 (float32) followed by N ones (:375-389);
  * effective budget max(hot_budget, int(adaptive_hot_frac * total)) when the
    fraction is positive (:664-670);
  * with the proxy on: EMA (decay proxy_decay) of |cos| between the mean new
    key and each warm token's key averaged over batch and heads, reset when the
    warm length changed underneath it (:486-525); promotion from attention
    weights (mean over batch, heads and queries of the first warm_len columns)
    or else from the proxy: warm tokens above promotion_threshold, at most
    max(1, hot_budget // 8) (the top ones), move to the front of the hot tier
    with importance 2.0 and their float16 values; the byte counter scales by the
    kept fraction (:415-484, :527-589);
  * over budget: n = hot_len - budget tokens chosen by _select_demote_indices
    (oracle.selection), quantized as ONE demotion event -- AffineQuantizer keys
    per channel over the event's tokens, values per token, outliers per event
    -- and dequantized to the float16 working copy appended to the warm tier;
    the measured packed bytes of the event (codes + scale + zero, K and V) are
    added up (:673-735); the chosen tokens leave the hot tier and the
    importance vector (:737-750);
  * the returned view is cat(warm, hot) (dtype promoted as torch.cat does:
    float16 with float16 stays float16, float16 with float32 / bfloat16 gives
    float32) sorted by position (:762-787); protected layers keep every token
    hot and return the hot tier.
Each batch element is one AffineQuantizer call over (H, n, D): the reference
calls it once on ``k.squeeze(0)``, which is that call at batch 1.  With
``per_head_bits`` of H entries each (batch element, head) is one call at that
head's width (akv/drop_in.py:315-374).

This module is test infrastructure: only the tests, the smoke check and the
benchmark's CPU-baseline leg use it, as the checker.

Pinning: the quantizer and dequantizer it calls are pinned in
tests/test_oracle_pinning.py and the selection in oracle/selection.py; the
state machine is checked against the reference's own cache-ordering tests
(tests/test_cache_ordering.py: position coverage after prefill with and
without demotion, chronological view, decode appends at total_len,
independent layers), the no-demotion identity of tests/test_bit_exact.py (the
view is the concatenated input, bit for bit) and the packed-byte properties of
tests/test_packed_bytes.py:95-127, restated in tests/test_oracle_layer.py,
plus closed forms for the importance recurrence and the byte counter.
"""
from __future__ import annotations

import numpy as np

from . import affine as oaff
from . import selection as osel
from .fp import F16, to_dtype


def _cat_dtype(a_dt: str, b_dt: str) -> str:
    return a_dt if a_dt == b_dt else "float32"


class AKVLayerOracle:
    """State of one AKVLayer; arrays hold values of ``dt`` (bf16 as float32 holding bf16 values)."""

    def __init__(self, warm_bits=3, hot_budget=128, protect=False, adaptive_hot_frac=0.0,
                 warm_key_bits=None, warm_value_bits=None, outlier_fraction=0.0, enable_promotion=False,
                 promotion_threshold=0.05, enable_promotion_proxy=False, proxy_decay=0.7, per_head_bits=None):
        self.enable_promotion = enable_promotion
        self.promotion_threshold = promotion_threshold
        self.enable_promotion_proxy = enable_promotion_proxy
        self.proxy_decay = proxy_decay
        self.proxy = None
        self.promoted_total = 0  # tokens promoted so far (bookkeeping for the checks)
        self.warm_bits = warm_bits
        self.hot_budget = hot_budget
        self.protect = protect
        self.adaptive_hot_frac = adaptive_hot_frac
        self.warm_key_bits = warm_key_bits or warm_bits
        self.warm_value_bits = warm_value_bits or warm_bits
        self.outlier_fraction = outlier_fraction
        self.per_head_bits = list(per_head_bits) if per_head_bits is not None else None
        self.hot_k = self.hot_v = None
        self.hot_pos = None
        self.warm_k = self.warm_v = None
        self.warm_pos = None
        self.importance = None
        self.total_len = 0
        self.step = 0
        self.warm_len = 0
        self.warm_bytes_packed = 0
        self.dt = None
        self.events = []  # (positions, per-batch (qk, qv) dicts) of each demotion event

    def _append_hot(self, k, v, pos):
        if self.hot_k is None:
            self.hot_k, self.hot_v, self.hot_pos = k, v, pos
        else:
            self.hot_k = np.concatenate([self.hot_k, k], axis=2)
            self.hot_v = np.concatenate([self.hot_v, v], axis=2)
            self.hot_pos = np.concatenate([self.hot_pos, pos])

    # ---- promotion (akv/drop_in.py:415-589)
    def _update_proxy(self, k):
        """EMA of |cos| between the mean new key and each warm token's key averaged
        over batch and heads (akv/drop_in.py:486-525), in float32."""
        if self.warm_k is None or self.warm_k.shape[2] == 0:
            self.proxy = None
            return
        probe = np.asarray(k, np.float32).mean(axis=(0, 1, 2), dtype=np.float32)
        probe = (probe / (np.float32(np.linalg.norm(probe)) + np.float32(1e-6))).astype(np.float32)
        wk = self.warm_k.astype(np.float32).mean(axis=(0, 1), dtype=np.float32)
        wn = (wk / (np.linalg.norm(wk, axis=-1, keepdims=True).astype(np.float32) + np.float32(1e-6))).astype(np.float32)
        sim = np.abs((wn @ probe).astype(np.float32))
        if self.proxy is None or self.proxy.shape[0] != sim.shape[0]:
            self.proxy = sim
        else:
            d = np.float32(self.proxy_decay)
            self.proxy = (d * self.proxy + (np.float32(1.0) - d) * sim).astype(np.float32)

    def _promote(self, mask_scores: np.ndarray, use_proxy: bool):
        """Promote warm tokens whose score exceeds the threshold, at most
        max(1, hot_budget // 8) of them (the top ones), to the front of the hot tier
        with importance 2.0; the packed-byte counter scales by the kept fraction."""
        warm_len = self.warm_k.shape[2]
        mask = mask_scores > np.float32(self.promotion_threshold)
        n = int(mask.sum())
        if n == 0:
            return
        cap = max(1, self.hot_budget // 8)
        if n > cap:
            top = np.argsort(-mask_scores, kind="stable")[:cap]
            mask = np.zeros(warm_len, bool)
            mask[top] = True
            n = cap
        idx = np.nonzero(mask)[0]
        self.promoted_total += n
        pk, pv, ppos = self.warm_k[:, :, idx], self.warm_v[:, :, idx], self.warm_pos[idx]
        keep = ~mask
        self.warm_k, self.warm_v, self.warm_pos = self.warm_k[:, :, keep], self.warm_v[:, :, keep], self.warm_pos[keep]
        if use_proxy:
            self.proxy = self.proxy[keep]
        self.warm_bytes_packed = int(self.warm_bytes_packed * (max(0, warm_len - n) / warm_len))
        self.warm_len -= n
        hot_dt = _cat_dtype(F16, self.hot_dt)
        self.hot_k = np.concatenate([to_dtype(pk.astype(np.float32), hot_dt),
                                     to_dtype(self.hot_k.astype(np.float32), hot_dt)], axis=2)
        self.hot_v = np.concatenate([to_dtype(pv.astype(np.float32), hot_dt),
                                     to_dtype(self.hot_v.astype(np.float32), hot_dt)], axis=2)
        self.hot_dt = hot_dt
        self.hot_pos = np.concatenate([ppos, self.hot_pos])
        self.importance = np.concatenate([np.full(n, 2.0, np.float32), self.importance])

    def update(self, k: np.ndarray, v: np.ndarray, dt: str = None, attention_weights=None):
        """k, v (B, H, N, D); returns the (full_k, full_v) view and its dtype name."""
        dt = dt or (F16 if k.dtype == np.float16 else "float32")
        self.dt = dt
        if self.hot_k is None:
            self.hot_dt = dt
        elif self.hot_dt != dt:
            self.hot_dt = _cat_dtype(self.hot_dt, dt)
        B, H, N, D = k.shape
        pos = np.arange(self.total_len, self.total_len + N, dtype=np.int64)
        if self.protect:
            self._append_hot(k, v, pos)
            self.total_len += N
            return self.hot_k, self.hot_v, dt
        self._append_hot(k, v, pos)
        self.total_len += N
        self.step += 1
        hot_len = self.hot_k.shape[2]
        if self.importance is None or self.importance.shape[0] != hot_len - N:
            self.importance = np.ones(hot_len, np.float32)
        else:
            self.importance = np.concatenate([(self.importance * np.float32(0.3)).astype(np.float32),
                                              np.ones(N, np.float32)])
        if self.enable_promotion_proxy:
            self._update_proxy(k)
        if self.enable_promotion and attention_weights is not None:
            if self.warm_k is not None and self.warm_k.shape[2] and attention_weights.shape[-1] >= self.warm_k.shape[2] + hot_len:
                aw = np.asarray(attention_weights, np.float32)[..., : self.warm_k.shape[2]]
                self._promote(aw.mean(axis=(0, 1, 2), dtype=np.float32), use_proxy=False)
            hot_len = self.hot_k.shape[2]
        elif self.enable_promotion and self.enable_promotion_proxy:
            if self.proxy is not None and self.warm_k is not None and self.warm_k.shape[2] \
                    and self.proxy.shape[0] == self.warm_k.shape[2]:
                self._promote(self.proxy, use_proxy=True)
            hot_len = self.hot_k.shape[2]
        budget = self.hot_budget
        if self.adaptive_hot_frac > 0.0:
            budget = max(self.hot_budget, int(self.adaptive_hot_frac * self.total_len))
        if hot_len > budget:
            n = hot_len - budget
            idx = osel.select_demote_indices(self.importance, n, hot_len, self.hot_budget)
            dk, dv = self.hot_k[:, :, idx], self.hot_v[:, :, idx]
            dt = self.hot_dt  # the quantizer runs in the hot tier's dtype
            wk = np.zeros((B, H, n, D), np.float16)
            wv = np.zeros((B, H, n, D), np.float16)
            per_b = []
            for b in range(B):
                if self.per_head_bits and len(self.per_head_bits) == H:
                    # one quantizer call per head at its width (akv/drop_in.py:349-374)
                    heads = []
                    for h, bits in enumerate(self.per_head_bits):
                        qk = oaff.quantize_keys(dk[b, h:h + 1], bits, self.outlier_fraction, dt=dt)
                        qv = oaff.quantize_values(dv[b, h:h + 1], bits, self.outlier_fraction, dt=dt)
                        wk[b, h] = oaff.dequantize_keys(qk)[0]
                        wv[b, h] = oaff.dequantize_values(qv)[0]
                        self.warm_bytes_packed += packed_bytes(qk) + packed_bytes(qv)
                        heads.append((qk, qv))
                    per_b.append(heads)
                    continue
                qk = oaff.quantize_keys(dk[b], self.warm_key_bits, self.outlier_fraction, dt=dt)
                qv = oaff.quantize_values(dv[b], self.warm_value_bits, self.outlier_fraction, dt=dt)
                wk[b] = oaff.dequantize_keys(qk)
                wv[b] = oaff.dequantize_values(qv)
                self.warm_bytes_packed += packed_bytes(qk) + packed_bytes(qv)
                per_b.append((qk, qv))
            self.events.append((self.hot_pos[idx].copy(), per_b))
            if self.warm_k is None:
                self.warm_k, self.warm_v, self.warm_pos = wk, wv, self.hot_pos[idx].copy()
            else:
                self.warm_k = np.concatenate([self.warm_k, wk], axis=2)
                self.warm_v = np.concatenate([self.warm_v, wv], axis=2)
                self.warm_pos = np.concatenate([self.warm_pos, self.hot_pos[idx]])
            self.warm_len += n
            if self.proxy is not None:
                self.proxy = np.concatenate([self.proxy, np.zeros(n, np.float32)])
            keep = np.ones(hot_len, bool)
            keep[idx] = False
            self.hot_k, self.hot_v = self.hot_k[:, :, keep], self.hot_v[:, :, keep]
            self.hot_pos = self.hot_pos[keep]
            self.importance = self.importance[keep]
        if self.warm_k is None:
            return self.hot_k, self.hot_v, dt
        out_dt = _cat_dtype(F16, self.hot_dt)
        fk = np.concatenate([to_dtype(self.warm_k.astype(np.float32), out_dt),
                             to_dtype(self.hot_k.astype(np.float32), out_dt)], axis=2)
        fv = np.concatenate([to_dtype(self.warm_v.astype(np.float32), out_dt),
                             to_dtype(self.hot_v.astype(np.float32), out_dt)], axis=2)
        order = np.argsort(np.concatenate([self.warm_pos, self.hot_pos]), kind="stable")
        return fk[:, :, order], fv[:, :, order], out_dt


def packed_bytes(q: dict) -> int:
    """measure_packed_bytes of an AffineQuantizer dict (akv/packed_layout.py:501-543):
    the packed codes as stored plus the scale and zero tensors at float16."""
    return int(q["codes"].size * q["codes"].itemsize + 2 * q["scale"].size * 2)

