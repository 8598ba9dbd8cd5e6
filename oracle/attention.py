"""Oracle restatement of the reference's fp32 dequant-attention.

``triton_kernels._fused_decode_attention_dispatch`` (akv/triton_kernels.py:350-387)
is the fp32 oracle: dequantize the warm tier, expand it to (B, H), concatenate
with the hot tier (hot first), then
    attn = softmax(query.float() @ keys.float().T * sm_scale) ; out = attn @ values.float()
and cast to the query dtype.  ``fused_mixed_precision_attention`` returns the
same attention weights as ``(out, attn)`` (akv/triton_ops.py:554-601, fp32 on
the device path).  The per-(batch, kv-head) warm tier with grouped-query heads
is the same computation with HF ``repeat_kv`` semantics (query head h uses kv
head h // (Hq // Hkv)); it is evaluated here group by group without
materialising the repeat.

Pinning: checked against a float64 brute-force loop over (b, h, m, n) on tiny
shapes, the row-sum-to-one invariant (tests/test_triton_ops.py:134-155) and
the no-warm reduction to plain attention (akv/triton_kernels.py:326-329).
"""
from __future__ import annotations

import math

import numpy as np


def attention_fp32(q, k, v, sm_scale=None, return_weights=True):
    """q (B,Hq,M,D); k, v (B,Hkv,N,D) (any float dtype; cast to fp32).

    Returns (out fp32 (B,Hq,M,D), attn fp32 (B,Hq,M,N) or None)."""
    q = np.asarray(q).astype(np.float32)
    k = np.asarray(k).astype(np.float32)
    v = np.asarray(v).astype(np.float32)
    B, Hq, M, D = q.shape
    Hkv, N = k.shape[1], k.shape[2]
    if Hq % Hkv:
        raise ValueError("Hq must be a multiple of Hkv")
    g = Hq // Hkv
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    qg = q.reshape(B, Hkv, g * M, D)
    s = np.matmul(qg, np.swapaxes(k, -1, -2)).astype(np.float32) * np.float32(sm_scale)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s, dtype=np.float32)
    p /= p.sum(axis=-1, keepdims=True, dtype=np.float32)
    out = np.matmul(p, v).astype(np.float32).reshape(B, Hq, M, D)
    attn = p.reshape(B, Hq, M, N) if return_weights else None
    return out, attn


def mixed_attention_fp32(q, k_hot, v_hot, k_warm, v_warm, sm_scale=None, hot_first=True,
                         return_weights=True):
    """Hot fp16 tier + dequantized warm tier (already fp16/dtype values).

    ``k_warm``/``v_warm`` are (B,Hkv,Nw,D), or (Nw,D) for the reference's
    broadcast warm tier (akv/triton_kernels.py:376-377 ``expand(B, H)``)."""
    B, Hkv = k_hot.shape[0], k_hot.shape[1]
    if k_warm is not None and np.asarray(k_warm).ndim == 2:
        k_warm = np.broadcast_to(np.asarray(k_warm)[None, None], (B, Hkv) + np.asarray(k_warm).shape)
        v_warm = np.broadcast_to(np.asarray(v_warm)[None, None], (B, Hkv) + np.asarray(v_warm).shape)
    if k_warm is None:
        k, v = k_hot, v_hot
    elif hot_first:
        k = np.concatenate([np.asarray(k_hot), np.asarray(k_warm).astype(np.asarray(k_hot).dtype)], axis=2)
        v = np.concatenate([np.asarray(v_hot), np.asarray(v_warm).astype(np.asarray(v_hot).dtype)], axis=2)
    else:
        k = np.concatenate([np.asarray(k_warm).astype(np.asarray(k_hot).dtype), np.asarray(k_hot)], axis=2)
        v = np.concatenate([np.asarray(v_warm).astype(np.asarray(v_hot).dtype), np.asarray(v_hot)], axis=2)
    return attention_fp32(q, k, v, sm_scale, return_weights)


def prefill_causal_fp32(q, k_cache, v_cache, k_chunk, v_chunk, sm_scale=None, positions=None):
    """Chunked prefill with the chunk's own causal self-attention (no counterpart in the
    reference, whose attention over a prompt chunk is the model's): query row m attends to
    every cached token and to chunk tokens 0..positions[m] (positions defaults to 0..M-1,
    the chunk's own order).  q (B,Hq,M,D); k_cache, v_cache (B,Hkv,N,D), N may be 0;
    k_chunk, v_chunk (B,Hkv,Mc,D).  fp32 as ``attention_fp32``; returns out (B,Hq,M,D).

    Pinning: ``prefill_causal_f64_bruteforce`` on tiny shapes; a row whose position is the
    chunk's last token sees every token (``attention_fp32`` over cache + chunk); a lone
    query at position 0 with an empty cache returns chunk value 0."""
    q = np.asarray(q).astype(np.float32)
    kc, vc = np.asarray(k_chunk).astype(np.float32), np.asarray(v_chunk).astype(np.float32)
    B, Hq, M, D = q.shape
    Hkv, Mc = kc.shape[1], kc.shape[2]
    g = Hq // Hkv
    pos = np.arange(M) if positions is None else np.asarray(positions)
    k = kc if k_cache is None else np.concatenate([np.asarray(k_cache).astype(np.float32), kc], axis=2)
    v = vc if v_cache is None else np.concatenate([np.asarray(v_cache).astype(np.float32), vc], axis=2)
    N = k.shape[2] - Mc
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    qg = q.reshape(B, Hkv, g * M, D)
    s = np.matmul(qg, np.swapaxes(k, -1, -2)).astype(np.float32) * np.float32(sm_scale)
    rowpos = np.tile(pos, g)  # row h_local * M + m has chunk position pos[m]
    masked = np.arange(Mc)[None, :] > rowpos[:, None]
    s[..., N:][:, :, masked] = -np.inf
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s, dtype=np.float32)
    p /= p.sum(axis=-1, keepdims=True, dtype=np.float32)
    return np.matmul(p, v).astype(np.float32).reshape(B, Hq, M, D)


def prefill_causal_f64_bruteforce(q, k_cache, v_cache, k_chunk, v_chunk, sm_scale=None):
    """Loop-level float64 form of ``prefill_causal_fp32`` for tiny shapes."""
    q = np.asarray(q, np.float64)
    kc, vc = np.asarray(k_chunk, np.float64), np.asarray(v_chunk, np.float64)
    kk = np.asarray(k_cache, np.float64) if k_cache is not None else kc[:, :, :0]
    vv = np.asarray(v_cache, np.float64) if v_cache is not None else vc[:, :, :0]
    B, Hq, M, D = q.shape
    g = Hq // kc.shape[1]
    sm = 1.0 / math.sqrt(D) if sm_scale is None else sm_scale
    out = np.zeros((B, Hq, M, D))
    for b in range(B):
        for h in range(Hq):
            kh = h // g
            for m in range(M):
                keys = [kk[b, kh, n] for n in range(kk.shape[2])] + [kc[b, kh, j] for j in range(m + 1)]
                vals = [vv[b, kh, n] for n in range(vv.shape[2])] + [vc[b, kh, j] for j in range(m + 1)]
                s = [sum(q[b, h, m, d] * key[d] for d in range(D)) * sm for key in keys]
                mx = max(s)
                e = [math.exp(x - mx) for x in s]
                tot = sum(e)
                for val, ei in zip(vals, e):
                    out[b, h, m] += ei / tot * val
    return out


def attention_f64_bruteforce(q, k, v, sm_scale=None):
    """Loop-level float64 reference for tiny shapes (pins ``attention_fp32``)."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    B, Hq, M, D = q.shape
    Hkv, N = k.shape[1], k.shape[2]
    g = Hq // Hkv
    sm = 1.0 / math.sqrt(D) if sm_scale is None else sm_scale
    out = np.zeros((B, Hq, M, D))
    attn = np.zeros((B, Hq, M, N))
    for b in range(B):
        for h in range(Hq):
            kh = h // g
            for m in range(M):
                s = [sum(q[b, h, m, d] * k[b, kh, n, d] for d in range(D)) * sm for n in range(N)]
                mx = max(s)
                e = [math.exp(x - mx) for x in s]
                tot = sum(e)
                for n in range(N):
                    attn[b, h, m, n] = e[n] / tot
                    out[b, h, m] += attn[b, h, m, n] * v[b, kh, n]
    return out, attn
