"""Decode over the legacy per-token-group warm tier (the layout of the reference's
public legacy ops, akv/triton_ops.py:657-713 and akv/fused_attention.py:281-317, and
of PackedKVArena) against the oracle's fp32 dequant-attention.

Head_dim 128 with 2 / 4 bits, groups of 32 / 64 / 128 and fp16 scales runs the
LDS-streamed kernel; 8 bits, head_dim 64 and bf16 / fp32 scales run the general
split kernel.  Covered: the asymmetric branch and the symmetric one (all zero-points
0, detected on the device, or forced), one warm tier shared by every batch element and
head, one per kv head or one per (batch, kv head), grouped-query heads, ragged lengths, a token stride above the
warm length (an arena's capacity), hot tokens before or after the warm ones, and
scales large enough that -1024 s overflows fp16 (the exact slow path)."""
import numpy as np
import pytest
import torch

from gpu_util import announce, assert_close_attn, to_dev
from oracle import attention as oatt
from oracle import legacy as oleg

pytestmark = pytest.mark.gpu


def _tier(rng, rows, N, D, bits, gs, sym, scale=1.0, dt=np.float16):
    """rows x N tokens quantized per (token, group) with KVQuantizer's arithmetic:
    packed codes (rows * N, pD * bits / 8), scales / zeros (rows * N, G), and the
    oracle's dequantized (rows, N, D) float32."""
    x = (rng.standard_normal((rows * N, D)) * scale).astype(np.float16)
    qt = oleg.kvq_quantize(x, bits, gs, sym)
    G = qt["scales"].shape[-1]
    s, z = qt["scales"].reshape(-1, G), qt["zeros"].reshape(-1, G)
    deq = oleg.dequantize_packed(qt["data"], s, z, bits, gs, rows * N, D).astype(np.float32)
    return qt["data"].reshape(rows * N, -1), s.astype(dt), z.astype(dt), deq.reshape(rows, N, D)


def _run(q, kh, vh, parts, bits, gs, N, D, warm_heads, Hkv, hot_first, sym=-1, token_stride=0):
    from akv._legacy import legacy_desc
    from akv.warm_tier import run_decode
    keep = []
    (kp, ks, kz), (vp, vs, vz) = parts
    desc = legacy_desc(to_dev(kp), to_dev(ks), to_dev(kz), to_dev(vp), to_dev(vs), to_dev(vz), bits, gs,
                       token_stride or N, D, warm_heads=warm_heads, sym=sym, keep=keep)
    desc.n_warm = N
    desc.token_stride = token_stride
    out, _ = run_decode(to_dev(q), to_dev(kh) if kh is not None else None, to_dev(vh) if vh is not None else None,
                        desc, Hkv, None, hot_first, keep=keep)
    torch.cuda.synchronize()
    return out


def _ref(q, kh, vh, kd, vd, hot_first, warm_heads, B, Hkv):
    """Oracle attention with the warm tier -- (N, D) shared, or (Hkv, N, D) per head --
    broadcast to (B, Hkv)."""
    if warm_heads == 1:
        kd, vd = np.broadcast_to(kd, (B, Hkv) + kd.shape), np.broadcast_to(vd, (B, Hkv) + vd.shape)
    else:
        kd, vd = np.broadcast_to(kd[None], (B,) + kd.shape), np.broadcast_to(vd[None], (B,) + vd.shape)
    D = q.shape[-1]
    if kh is None:
        kh = vh = np.zeros((B, Hkv, 0, D), np.float16)
    ref, _ = oatt.mixed_attention_fp32(q, kh, vh, kd.astype(np.float16), vd.astype(np.float16),
                                       hot_first=hot_first, return_weights=False)
    return ref


def _ref_full(q, kh, vh, kd, vd, hot_first, B, Hkv):
    """Oracle attention with a warm tier per (batch, kv head): kd, vd (B, Hkv, N, D)."""
    if kh is None:
        kh = vh = np.zeros((B, Hkv, 0, q.shape[-1]), np.float16)
    ref, _ = oatt.mixed_attention_fp32(q, kh, vh, kd.astype(np.float16), vd.astype(np.float16),
                                       hot_first=hot_first, return_weights=False)
    return ref


CASES = [  # bits, gs, sym, warm tier ("one" shared / "per" kv head / "bh" per batch and kv head), B, Hq, Hkv, M, N, Nh, hot_first
    (4, 64, False, "per", 1, 32, 32, 1, 1000, 200, False),
    (4, 32, False, "one", 2, 8, 2, 1, 300, 40, True),
    (4, 128, True, "one", 2, 4, 4, 1, 517, 0, True),
    (2, 32, False, "per", 1, 8, 8, 1, 333, 16, False),
    (2, 64, True, "per", 3, 16, 4, 2, 250, 33, True),
    (2, 128, False, "one", 1, 12, 2, 1, 4096, 512, False),
    (4, 128, False, "bh", 3, 8, 4, 1, 203, 64, False),
    (2, 64, True, "bh", 2, 12, 2, 3, 450, 17, True),
]


@pytest.mark.parametrize("bits,gs,sym,wh,B,Hq,Hkv,M,N,Nh,hot_first", CASES)
def test_legacy_decode_matches_oracle(bits, gs, sym, wh, B, Hq, Hkv, M, N, Nh, hot_first):
    announce(f"legacy decode bits={bits} gs={gs} sym={sym} warm={wh} B={B} Hq={Hq} Hkv={Hkv} M={M} N={N} Nh={Nh}")
    rng = np.random.default_rng(bits * 100 + gs + N)
    D = 128
    rows = {"one": 1, "per": Hkv, "bh": B * Hkv}[wh]
    kp, ks, kz, kd = _tier(rng, rows, N, D, bits, gs, sym)
    vp, vs, vz, vd = _tier(rng, rows, N, D, bits, gs, sym)
    q = rng.standard_normal((B, Hq, M, D)).astype(np.float16)
    kh = rng.standard_normal((B, Hkv, Nh, D)).astype(np.float16) if Nh else None
    vh = rng.standard_normal((B, Hkv, Nh, D)).astype(np.float16) if Nh else None
    out = _run(q, kh, vh, ((kp, ks, kz), (vp, vs, vz)), bits, gs, N, D, rows, Hkv, hot_first)
    if wh == "bh":  # (B * Hkv, N, D) -> (B, Hkv, N, D)
        ref = _ref_full(q, kh, vh, kd.reshape(B, Hkv, N, D), vd.reshape(B, Hkv, N, D), hot_first, B, Hkv)
    else:
        ref = _ref(q, kh, vh, kd if rows > 1 else kd[0], vd if rows > 1 else vd[0], hot_first, rows, B, Hkv)
    assert_close_attn(out, ref)


@pytest.mark.parametrize("sym", [0, 1])
def test_forced_branch_and_token_stride(sym):
    """legacy_sym forced (no detection kernel) and a per-head token stride above the
    warm length: the first N rows of each head's `cap` rows are the tier."""
    announce(f"legacy decode forced sym={sym}, token stride")
    rng = np.random.default_rng(11 + sym)
    B, H, D, N, cap, bits, gs = 1, 8, 128, 700, 1024, 4, 64
    kp, ks, kz, kd = _tier(rng, H, cap, D, bits, gs, bool(sym))
    vp, vs, vz, vd = _tier(rng, H, cap, D, bits, gs, bool(sym))
    q = rng.standard_normal((B, H, 1, D)).astype(np.float16)
    kh = rng.standard_normal((B, H, 64, D)).astype(np.float16)
    vh = rng.standard_normal((B, H, 64, D)).astype(np.float16)
    out = _run(q, kh, vh, ((kp, ks, kz), (vp, vs, vz)), bits, gs, N, D, H, H, False, sym=sym, token_stride=cap)
    assert_close_attn(out, _ref(q, kh, vh, kd[:, :N], vd[:, :N], False, H, B, H))


def test_overflowing_scales_take_the_exact_path():
    """Scales of 64 and more (|-1024 s| overflows fp16) in one unit of K and of V."""
    announce("legacy decode with scales >= 64")
    rng = np.random.default_rng(21)
    B, H, D, N, bits, gs = 1, 4, 128, 96, 4, 32
    kp, ks, kz, _ = _tier(rng, H, N, D, bits, gs, False)
    vp, vs, vz, _ = _tier(rng, H, N, D, bits, gs, False)
    ks[40:50] = np.float16(80.0)
    vs[70:75] = np.float16(96.0)
    kz[40:50] = np.float16(-500.0)
    kd = oleg.dequantize_packed(kp, ks, kz, bits, gs, H * N, D).astype(np.float32).reshape(H, N, D)
    vd = oleg.dequantize_packed(vp, vs, vz, bits, gs, H * N, D).astype(np.float32).reshape(H, N, D)
    q = (rng.standard_normal((B, H, 1, D)) * 0.01).astype(np.float16)  # keeps the logits of the large keys modest
    out = _run(q, None, None, ((kp, ks, kz), (vp, vs, vz)), bits, gs, N, D, H, H, True)
    ref = _ref(q, None, None, kd, vd, True, H, B, H)
    # values up to ~1400: the attention tolerance scaled to the output's magnitude
    assert_close_attn(out, ref, max_abs=2e-3 * 1500, mean_abs=1e-3 * 1500)


@pytest.mark.parametrize("dt,bits,D", [(np.float32, 4, 128), (np.float16, 8, 128), (np.float16, 4, 64)])
def test_general_kernel_cases(dt, bits, D):
    """fp32 scales, 8-bit codes and head_dim 64 stay on the general split kernel."""
    announce(f"legacy decode general kernel dt={dt.__name__} bits={bits} D={D}")
    rng = np.random.default_rng(31 + bits + D)
    B, H, N, gs = 2, 4, 210, 32
    kp, ks, kz, kd = _tier(rng, 1, N, D, bits, gs, False, dt=dt)
    vp, vs, vz, vd = _tier(rng, 1, N, D, bits, gs, False, dt=dt)
    q = rng.standard_normal((B, H, 1, D)).astype(np.float16)
    kh = rng.standard_normal((B, H, 20, D)).astype(np.float16)
    vh = rng.standard_normal((B, H, 20, D)).astype(np.float16)
    out = _run(q, kh, vh, ((kp, ks, kz), (vp, vs, vz)), bits, gs, N, D, 1, H, True)
    assert_close_attn(out, _ref(q, kh, vh, kd[0], vd[0], True, 1, B, H))
