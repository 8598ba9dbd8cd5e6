"""Oracle restatement of ``akv/affine_quantizer.py`` and its block/group form.

Reference semantics (akv/affine_quantizer.py:63-189), applied in the input
dtype with per-op rounding (see ``oracle.fp``):

  K (per channel, min/max over tokens):
    [outliers] n_out = max(1, int(D*f)); rank channels by
               k.float().norm(dim=1).mean(dim=0), take the top n_out, keep
               k[..., idx] as fp16, zero those channels          (:75-85)
    mn, mx = amin/amax over tokens                                 (:88-89)
    scale = (mx - mn) / maxv ; scale = clamp(scale, min=1e-8)      (:91-92)
    zero  = mn                                                     (:93)
    codes = round_half_even((k - zero) / scale).clamp(0, maxv).to(u8)  (:95)
    scale, zero stored as fp16; codes bit-packed                   (:97-109)
  V: the same with min/max over channels (per token)               (:131-176)
  dequant: unpack -> codes.half() * scale (fp16 round) + zero (fp16 round),
           then outlier channels overwritten                       (:112-124, :178-189)

``clamp(min=1e-8)`` is a no-op in fp16 (1e-8 rounds to 0), so a constant
channel has scale 0, (k-zero)/scale = 0/0 = NaN and NaN.to(uint8) = 0.

Block/group form used by the warm tier: K is quantized with the call above
on each block of T tokens of one (batch, head-group) -- ``quantize_keys`` on a
(Hkv, T, D) slice, so outliers are chosen per (batch, block) and shared by
the heads; V keeps the per-token rule but takes min/max over each group of G
channels (G = D is exactly ``quantize_values``).  T = N and G = D reproduce
AffineQuantizer call for call.

Pinning: closed forms checked against float64 brute force that enumerates
every quantization level and picks the nearest (ties to even) from the
fp16-rounded intermediates; the scale==0 / NaN path and clamp are checked on
constant and single-token blocks; the block form at T=N, G=D is checked
against the single-call form.  Channel ranking under exact or near ties
(fp32 summation order inside norm/mean) is parity unpinned.
"""
from __future__ import annotations

import numpy as np

from . import bitpack
from .fp import F16, F32, BF16, op, scalar_in, to_dtype, to_u8


def _dt_of(x: np.ndarray, dt):
    if dt is not None:
        return dt
    if x.dtype == np.float16:
        return F16
    if x.dtype == np.float32:
        return F32
    raise ValueError("oracle quantizer takes float16 or float32 arrays (pass dt='bfloat16' for bf16 values)")


def _store(x: np.ndarray, dt: str) -> np.ndarray:
    return to_dtype(x, dt)


def _quant_core(x, axis, bits, dt):
    """min/max along ``axis`` (keepdims) -> (codes u8, scale, zero) in dt."""
    maxv = (1 << bits) - 1
    mn = np.min(x, axis=axis, keepdims=True)
    mx = np.max(x, axis=axis, keepdims=True)
    scale = op(np.subtract, mx, mn, dt)
    scale = op(np.divide, scale, np.float32(maxv), dt)
    lo = scalar_in(1e-8, dt)
    s32 = scale.astype(np.float32)
    s32 = np.where(np.isnan(s32), s32, np.maximum(s32, lo))
    scale = _store(s32, dt)
    zero = mn
    with np.errstate(divide="ignore", invalid="ignore"):
        q = op(np.divide, op(np.subtract, x, zero, dt), scale, dt)
    q = np.rint(q.astype(np.float32))
    q = np.clip(q, 0.0, float(maxv))
    return to_u8(q), scale, zero


def _outliers(x: np.ndarray, frac: float, token_axis: int, head_axis: int):
    """Channel ranking of akv/affine_quantizer.py:76-80 (ties: lowest index first)."""
    D = x.shape[-1]
    n_out = max(1, int(D * frac))
    xf = x.astype(np.float32)
    norms = np.sqrt(np.sum(xf * xf, axis=token_axis, dtype=np.float32), dtype=np.float32)
    h_ax = head_axis if head_axis < token_axis else head_axis - 1
    cn = np.mean(norms, axis=h_ax, dtype=np.float32)
    order = np.argsort(-cn, axis=-1, kind="stable")
    return order[..., :n_out].astype(np.int64)


def quantize_keys(k: np.ndarray, bits: int, outlier_fraction: float = 0.0,
                  packed: bool = True, dt=None, outlier_idx=None) -> dict:
    """akv/affine_quantizer.py:63-110 on k (H, N, D).  ``outlier_idx`` (tests only)
    imposes the outlier channels instead of ranking them."""
    dt = _dt_of(k, dt)
    k = np.array(k, copy=True)
    res = {}
    if outlier_fraction > 0:
        idx = (_outliers(k, outlier_fraction, token_axis=1, head_axis=0) if outlier_idx is None
               else np.asarray(outlier_idx, dtype=np.int64))
        res["outlier_idx"] = idx
        res["outlier_data"] = to_dtype(k[..., idx], F16)
        k[..., idx] = 0
    codes, scale, zero = _quant_core(k, 1, bits, dt)
    res["scale"] = to_dtype(scale, F16)
    res["zero"] = to_dtype(zero, F16)
    res["orig_dim"] = codes.shape[-1]
    res["bits"] = bits
    res["codes"] = bitpack.pack(codes, bits) if packed else codes
    return res


def quantize_values(v: np.ndarray, bits: int, outlier_fraction: float = 0.0,
                    packed: bool = True, dt=None, outlier_idx=None) -> dict:
    """akv/affine_quantizer.py:131-176 on v (H, N, D).  ``outlier_idx`` (tests only)
    imposes the outlier channels instead of ranking them."""
    dt = _dt_of(v, dt)
    v = np.array(v, copy=True)
    res = {}
    if outlier_fraction > 0:
        idx = (_outliers(v, outlier_fraction, token_axis=1, head_axis=0) if outlier_idx is None
               else np.asarray(outlier_idx, dtype=np.int64))
        res["outlier_idx"] = idx
        res["outlier_data"] = to_dtype(v[..., idx], F16)
        v[..., idx] = 0
    codes, scale, zero = _quant_core(v, 2, bits, dt)
    res["scale"] = to_dtype(scale, F16)
    res["zero"] = to_dtype(zero, F16)
    res["orig_dim"] = codes.shape[-1]
    res["bits"] = bits
    res["codes"] = bitpack.pack(codes, bits) if packed else codes
    return res


def _dequant_f16(codes_u8: np.ndarray, scale: np.ndarray, zero: np.ndarray) -> np.ndarray:
    """codes.half() * scale + zero with two fp16 roundings (akv/affine_quantizer.py:117-120)."""
    c = codes_u8.astype(np.float16)
    return (c * scale.astype(np.float16)) + zero.astype(np.float16)


def dequantize_keys(qk: dict, packed: bool = True) -> np.ndarray:
    """akv/affine_quantizer.py:112-124."""
    codes = qk["codes"]
    if packed and qk["bits"] in (2, 3, 4):
        codes = bitpack.unpack(codes, qk["bits"], qk["orig_dim"])
    out = _dequant_f16(codes, qk["scale"], qk["zero"])
    if "outlier_idx" in qk:
        out[..., qk["outlier_idx"]] = qk["outlier_data"]
    return out


dequantize_values = dequantize_keys  # akv/affine_quantizer.py:178-189 is the same arithmetic


# ---------------------------------------------------------------------------
# Warm-tier block/group form: (B, H, N, D) in, kernel layout out.
# ---------------------------------------------------------------------------

def quantize_kv_blocked(k: np.ndarray, v: np.ndarray, bits_k: int, bits_v: int,
                        T: int = 32, G: int = 32, outlier_fraction: float = 0.0,
                        dt=None) -> dict:
    """K: ``quantize_keys`` per (batch, T-token block) on the (H, T, D) slice.
    V: per token over each G-channel group, outliers per (batch, block).

    Returns the warm-tier arrays:
      k_codes (B,H,N,Pk) u8, k_scale/k_zero (B,H,nblk,D) f16,
      v_codes (B,H,N,Pv) u8, v_scale/v_zero (B,H,N,D//G) f16,
      and with outliers k_oidx/v_oidx (B,nblk,n_out) i64,
      k_odata/v_odata (B,H,N,n_out) f16.
    """
    dt = _dt_of(k, dt)
    B, H, N, D = k.shape
    if D % G:
        raise ValueError("D must be a multiple of G")
    nblk = (N + T - 1) // T
    k_codes = np.zeros((B, H, N, D), np.uint8)
    v_codes = np.zeros((B, H, N, D), np.uint8)
    k_scale = np.zeros((B, H, nblk, D), np.float16)
    k_zero = np.zeros((B, H, nblk, D), np.float16)
    v_scale = np.zeros((B, H, N, D // G), np.float16)
    v_zero = np.zeros((B, H, N, D // G), np.float16)
    out = {}
    n_out = max(1, int(D * outlier_fraction)) if outlier_fraction > 0 else 0
    if n_out:
        out["k_oidx"] = np.zeros((B, nblk, n_out), np.int64)
        out["v_oidx"] = np.zeros((B, nblk, n_out), np.int64)
        out["k_odata"] = np.zeros((B, H, N, n_out), np.float16)
        out["v_odata"] = np.zeros((B, H, N, n_out), np.float16)
    # full blocks vectorised, then the ragged tail block
    nfull = N // T
    spans = []
    if nfull:
        spans.append((0, nfull * T, nfull))
    if N % T:
        spans.append((nfull * T, N, 1))
    for (t0, t1, nb) in spans:
        L = (t1 - t0) // nb
        b0 = t0 // T
        kb = np.array(k[:, :, t0:t1, :].reshape(B, H, nb, L, D), copy=True)
        vb = np.array(v[:, :, t0:t1, :].reshape(B, H, nb, L, D), copy=True)
        if n_out:
            for (x, key) in ((kb, "k"), (vb, "v")):
                idx = _outliers(x, outlier_fraction, token_axis=3, head_axis=1)  # (B, nb, n_out)
                out[key + "_oidx"][:, b0:b0 + nb] = idx
                gi = idx[:, None, :, None, :]  # (B,1,nb,1,n_out)
                gathered = np.take_along_axis(x, np.broadcast_to(gi, (B, H, nb, L, n_out)), axis=4)
                out[key + "_odata"][:, :, t0:t1] = to_dtype(gathered, F16).reshape(B, H, t1 - t0, n_out)
                np.put_along_axis(x, np.broadcast_to(gi, (B, H, nb, L, n_out)), 0, axis=4)
        ck, sk, zk = _quant_core(kb, 3, bits_k, dt)  # min/max over tokens of the block
        k_codes[:, :, t0:t1] = ck.reshape(B, H, t1 - t0, D)
        k_scale[:, :, b0:b0 + nb] = to_dtype(sk, F16)[:, :, :, 0, :]
        k_zero[:, :, b0:b0 + nb] = to_dtype(zk, F16)[:, :, :, 0, :]
        vg = vb.reshape(B, H, nb, L, D // G, G)
        cv, sv, zv = _quant_core(vg, 5, bits_v, dt)  # min/max over each channel group
        v_codes[:, :, t0:t1] = cv.reshape(B, H, t1 - t0, D)
        v_scale[:, :, t0:t1] = to_dtype(sv, F16).reshape(B, H, t1 - t0, D // G)
        v_zero[:, :, t0:t1] = to_dtype(zv, F16).reshape(B, H, t1 - t0, D // G)
    out.update(
        k_codes=bitpack.pack(k_codes, bits_k), k_scale=k_scale, k_zero=k_zero,
        v_codes=bitpack.pack(v_codes, bits_v), v_scale=v_scale, v_zero=v_zero,
        bits_k=bits_k, bits_v=bits_v, T=T, G=G, D=D, N=N, n_out=n_out,
    )
    return out


def dequant_kv_blocked(w: dict):
    """fp16 K and V (B, H, N, D) from the warm-tier arrays (same arithmetic as
    ``dequantize_keys`` / ``dequantize_values``)."""
    D, N, T, G = w["D"], w["N"], w["T"], w["G"]
    ck = bitpack.unpack(w["k_codes"], w["bits_k"], D)
    cv = bitpack.unpack(w["v_codes"], w["bits_v"], D)
    blk = np.arange(N) // T
    ks = w["k_scale"][:, :, blk, :]
    kz = w["k_zero"][:, :, blk, :]
    kd = _dequant_f16(ck, ks, kz)
    grp = np.arange(D) // G
    vs = w["v_scale"][..., grp]
    vz = w["v_zero"][..., grp]
    vd = _dequant_f16(cv, vs, vz)
    if w.get("n_out", 0):
        B, H = kd.shape[:2]
        for (x, key) in ((kd, "k"), (vd, "v")):
            idx = w[key + "_oidx"][:, blk, :]  # (B, N, n_out)
            gi = np.broadcast_to(idx[:, None], (B, H, N, idx.shape[-1]))
            np.put_along_axis(x, gi, w[key + "_odata"], axis=3)
    return kd, vd
