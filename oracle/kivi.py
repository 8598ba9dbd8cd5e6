"""Oracle restatement of the KIVI baselines (akv/baselines.py:236-535).

``kivi_quantize`` (``KIVICache._quantize_tensor``, :345-370): x (B, H, n, D) as
float32 rows of the last axis, zero-padded to a multiple of the group size; per
(row, group) min / max; scale = (max - min) / maxv clamped at 1e-10; code =
round-half-even((x - min) / scale) clamped to [0, maxv]; every op in float32.
Returns unpacked codes (rows, G, gs) uint8 and float32 scales / zeros (rows, G).
``kivi_dequantize`` (``_dequantize_tensor``, :372-380): float32 code * scale +
zero (two roundings), the padding dropped, cast to float16.

``KIVIOracle`` follows ``KIVICache.update`` (:268-289), ``_quantize_overflow``
(naive: :291-322, the merged history re-quantized; fused: :455-496, each overflow
chunk quantized once and its dequant appended to a float16 working copy) and
``_get_full_kv`` (:324-343 / :498-510).

This module is test infrastructure: only the tests, the smoke check and the
benchmark's CPU-baseline leg use it, as the checker.

Pinning (tests/test_oracle_kivi.py): the codes against a float64 nearest-level
brute force (the chosen level's error is the least, within float32 rounding of the
quotient); KATs for the round-half-even ties, a constant group (scale clamped at
1e-10, codes 0, dequant = the constant) and the zero padding of a head_dim that is
not a multiple of the group size; the dequant against its closed form in float64
for every code; and the reference's own KIVI tests restated on the oracle (fused vs
naive within 0.5 at 4 bits, memory of the same order, incremental growth).
"""
from __future__ import annotations

import numpy as np

from .fp import F16, to_dtype


def kivi_quantize(x: np.ndarray, bits: int, group_size: int):
    a = np.asarray(x, dtype=np.float32)
    D = a.shape[-1]
    flat = a.reshape(-1, D)
    if D % group_size:
        flat = np.concatenate([flat, np.zeros((flat.shape[0], group_size - D % group_size), np.float32)], axis=1)
    g = flat.reshape(flat.shape[0], -1, group_size)
    gmin = g.min(axis=-1, keepdims=True)
    gmax = g.max(axis=-1, keepdims=True)
    maxv = np.float32((1 << bits) - 1)
    with np.errstate(divide="ignore", invalid="ignore"):
        sc = ((gmax - gmin).astype(np.float32) / maxv).astype(np.float32)
        sc = np.where(np.isnan(sc), sc, np.maximum(sc, np.float32(1e-10))).astype(np.float32)
        q = ((g - gmin).astype(np.float32) / sc).astype(np.float32)
    codes = np.clip(np.rint(q), 0, maxv)
    codes = np.where(np.isnan(codes), 0, codes).astype(np.uint8)
    return codes, sc[..., 0], gmin[..., 0]


def kivi_dequantize(codes: np.ndarray, sc: np.ndarray, ze: np.ndarray, shape) -> np.ndarray:
    d = (codes.astype(np.float32) * np.asarray(sc, np.float32)[..., None]).astype(np.float32)
    d = (d + np.asarray(ze, np.float32)[..., None]).astype(np.float32)
    D = shape[-1]
    flat = d.reshape(d.shape[0], -1)[:, :D]
    return to_dtype(flat.reshape(shape), F16)


class KIVIOracle:
    """Per-layer state of ``KIVICache`` (fused=False) or ``KIVIFusedCache`` (fused=True);
    K / V as float32 arrays holding float16 values."""

    def __init__(self, key_bits=2, value_bits=2, group_size=128, residual_length=128, fused=True):
        self.kb, self.vb, self.gs, self.res_len, self.fused = key_bits, value_bits, group_size, residual_length, fused
        self.res_k, self.res_v, self.q_k, self.q_v, self.dq_k, self.dq_v, self.seq = {}, {}, {}, {}, {}, {}, {}

    def _q(self, x, bits):
        codes, sc, ze = kivi_quantize(x, bits, self.gs)
        return {"codes": codes, "scales": sc, "zeros": ze, "shape": x.shape}

    def _dq(self, d):
        return kivi_dequantize(d["codes"], d["scales"], d["zeros"], d["shape"]).astype(np.float32)

    def update(self, k, v, layer):
        k = to_dtype(np.asarray(k, np.float32), F16).astype(np.float32)
        v = to_dtype(np.asarray(v, np.float32), F16).astype(np.float32)
        if layer not in self.res_k:
            self.res_k[layer], self.res_v[layer], self.seq[layer] = k, v, k.shape[2]
        else:
            self.res_k[layer] = np.concatenate([self.res_k[layer], k], axis=2)
            self.res_v[layer] = np.concatenate([self.res_v[layer], v], axis=2)
            self.seq[layer] += k.shape[2]
        if self.res_k[layer].shape[2] > self.res_len:
            self._overflow(layer)
        return self.get_full_kv(layer)

    def _overflow(self, layer):
        rk, rv = self.res_k[layer], self.res_v[layer]
        n_q = rk.shape[2] - self.res_len
        tk, tv = rk[:, :, :n_q], rv[:, :, :n_q]
        if self.fused:
            qk, qv = self._q(tk, self.kb), self._q(tv, self.vb)
            nk, nv = self._dq(qk), self._dq(qv)
            if layer in self.q_k:
                self.q_k[layer].append(qk)
                self.q_v[layer].append(qv)
                self.dq_k[layer] = np.concatenate([self.dq_k[layer], nk], axis=2)
                self.dq_v[layer] = np.concatenate([self.dq_v[layer], nv], axis=2)
            else:
                self.q_k[layer], self.q_v[layer] = [qk], [qv]
                self.dq_k[layer], self.dq_v[layer] = nk, nv
        else:
            if layer in self.q_k:
                tk = np.concatenate([self._dq(self.q_k[layer][0]), tk], axis=2)
                tv = np.concatenate([self._dq(self.q_v[layer][0]), tv], axis=2)
            self.q_k[layer], self.q_v[layer] = [self._q(tk, self.kb)], [self._q(tv, self.vb)]
        self.res_k[layer], self.res_v[layer] = rk[:, :, n_q:], rv[:, :, n_q:]

    def quantized_rows(self, layer, values=False):
        """The layer's quantized tier as (codes (B*H, n, pD) uint8, scales, zeros
        (B*H, n, G)) in (batch, head, token) order."""
        chunks = (self.q_v if values else self.q_k)[layer]
        outs = []
        for d in chunks:
            B, H, n, _ = d["shape"]
            G = d["scales"].shape[-1]
            outs.append((d["codes"].reshape(B * H, n, -1), d["scales"].reshape(B * H, n, G),
                         d["zeros"].reshape(B * H, n, G)))
        return tuple(np.concatenate([o[i] for o in outs], axis=1) for i in range(3))

    def get_full_kv(self, layer):
        rk, rv = self.res_k[layer], self.res_v[layer]
        if layer not in self.q_k:
            return rk, rv
        if self.fused:
            wk, wv = self.dq_k[layer], self.dq_v[layer]
        else:
            wk, wv = self._dq(self.q_k[layer][0]), self._dq(self.q_v[layer][0])
        return np.concatenate([wk, rk], axis=2), np.concatenate([wv, rv], axis=2)

    def memory_bytes(self, packed=True):
        """Codes (bit-packed when `packed`, else one byte each as the reference keeps
        them) + float32 scales / zeros + the residual windows at float16."""
        total = 0
        for store, bits in ((self.q_k, self.kb), (self.q_v, self.vb)):
            for chunks in store.values():
                for d in chunks:
                    n_codes = d["codes"].size
                    total += (n_codes * bits // 8 if packed else n_codes) + 8 * d["scales"].size
        for r in list(self.res_k.values()) + list(self.res_v.values()):
            total += r.size * 2
        return total
