"""Cache-side entry points against the oracle: AKVCache.demote (FIFO with no
scores, and per-sequence scores), quantize_per_head (global quantizer, per-head
bit pools, head-count fallback) with its measured packed bytes, the compat
fused_quantize_evict through KVQuantizer, and AffineQuantizer at 8 bits."""
import numpy as np
import pytest
import torch

from gpu_util import announce, bits_equal, to_dev
from oracle import affine as oaff
from oracle import legacy as oleg
from oracle import selection as osel

pytestmark = pytest.mark.gpu


def _kv(shape, seed):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal(shape).astype(np.float32)
    v = rng.standard_normal(shape).astype(np.float32)
    k[..., 5] *= 10.0
    return k.astype(np.float16), v.astype(np.float16)


def _check_tier(warm, ref):
    for name in ("k_codes", "k_scale", "k_zero", "v_codes", "v_scale", "v_zero"):
        bits_equal(getattr(warm, name), ref[name])


@pytest.mark.parametrize("with_scores", [False, True])
def test_demote_matches_oracle(with_scores):
    import akv
    announce(f"AKVCache.demote scores={with_scores}")
    B, H, hot_len, D, n = 2, 2, 150, 128, 22
    k, v = _kv((B, H, hot_len, D), 31)
    cache = akv.AKVCache(preset="balanced")
    if with_scores:
        imp = np.random.default_rng(32).random((B, hot_len)).astype(np.float32)
        warm, idx = cache.demote(to_dev(k), to_dev(v), to_dev(imp), n)
        sel = np.stack([osel.select_demote_indices(imp[b], n, hot_len, cache.hot_budget) for b in range(B)])
    else:
        warm, idx = cache.demote(to_dev(k), to_dev(v), None, n)
        sel = np.tile(np.arange(n), (B, 1))
    assert idx.device.type == "cuda"
    np.testing.assert_array_equal(idx.cpu().numpy(), sel)
    kg = np.stack([k[b][:, sel[b]] for b in range(B)])
    vg = np.stack([v[b][:, sel[b]] for b in range(B)])
    ref = oaff.quantize_kv_blocked(kg, vg, cache.warm_key_bits, cache.warm_value_bits, cache.block_t, cache.group_v)
    _check_tier(warm, ref)


def _measure(q, bits):
    """measured bytes of an oracle quantizer dict: packed codes + scale + zero (fp16)."""
    return q["codes"].nbytes + q["scale"].nbytes + q["zero"].nbytes


@pytest.mark.parametrize("per_head_bits,of", [(None, 0.0), ([2, 3, 4, 3], 0.0), ([2, 4, 4, 2], 0.02), ([2, 3], 0.0)])
def test_quantize_per_head(per_head_bits, of):
    from akv.drop_in import quantize_per_head
    announce(f"quantize_per_head bits={per_head_bits} of={of}")
    B, H, n, D = 2, 4, 37, 128
    k, v = _kv((B, H, n, D), 41)
    dk, dv, nbytes = quantize_per_head(to_dev(k), to_dev(v), 3, 3, per_head_bits, 64, of)
    exp_k = np.empty_like(k)
    exp_v = np.empty_like(v)
    exp_bytes = 0
    for b in range(B):
        if per_head_bits and len(per_head_bits) == H:
            for h, bits in enumerate(per_head_bits):
                qk = oaff.quantize_keys(k[b, h:h + 1], bits, of)
                qv = oaff.quantize_values(v[b, h:h + 1], bits, of)
                exp_k[b, h] = oaff.dequantize_keys(qk)[0]
                exp_v[b, h] = oaff.dequantize_values(qv)[0]
                exp_bytes += _measure(qk, bits) + _measure(qv, bits)
        else:  # global widths (also the head-count mismatch fallback)
            qk = oaff.quantize_keys(k[b], 3, of)
            qv = oaff.quantize_values(v[b], 3, of)
            exp_k[b] = oaff.dequantize_keys(qk)
            exp_v[b] = oaff.dequantize_values(qv)
            exp_bytes += _measure(qk, 3) + _measure(qv, 3)
    bits_equal(dk, exp_k)
    bits_equal(dv, exp_v)
    assert nbytes == exp_bytes


def test_compat_fused_quantize_evict():
    import akv
    from akv.fused_attention import fused_quantize_evict
    announce("compat fused_quantize_evict(KVQuantizer)")
    k, v = _kv((1, 2, 40, 64), 51)
    mask = np.random.default_rng(52).random(40) < 0.4
    qz = akv.KVQuantizer(akv.QuantConfig(bits=4, group_size=32))
    qk, qv = fused_quantize_evict(to_dev(k), to_dev(v), None, to_dev(mask), qz)
    for got, src in ((qk, k), (qv, v)):
        ref = oleg.kvq_quantize(src[:, :, mask], 4, 32)
        np.testing.assert_array_equal(got.data.cpu().numpy().reshape(-1), ref["data"].reshape(-1))
        bits_equal(got.scales.reshape(ref["scales"].shape), ref["scales"])
        bits_equal(got.zeros.reshape(ref["zeros"].shape), ref["zeros"])
    assert fused_quantize_evict(to_dev(k), to_dev(v), None, to_dev(np.zeros(40, bool)), qz) == (None, None)


@pytest.mark.parametrize("packed", [True, False])
def test_affine_quantizer_8bit_passthrough(packed):
    import akv
    announce(f"AffineQuantizer 8-bit packed={packed}")
    k, v = _kv((3, 29, 128), 61)
    qz = akv.AffineQuantizer(akv.AffineQuantConfig(key_bits=8, value_bits=8, packed=packed))
    qk, qv = qz.quantize_keys(to_dev(k)), qz.quantize_values(to_dev(v))
    rk, rv = oaff.quantize_keys(k, 8, packed=packed), oaff.quantize_values(v, 8, packed=packed)
    for got, ref in ((qk, rk), (qv, rv)):
        np.testing.assert_array_equal(got["codes"].cpu().numpy(), ref["codes"])
        bits_equal(got["scale"], ref["scale"])
        bits_equal(got["zero"], ref["zero"])
        assert got["bits"] == 8 and got["codes"].shape[-1] == 128
    bits_equal(qz.dequantize_keys(qk), oaff.dequantize_keys(rk, packed=packed))
    bits_equal(qz.dequantize_values(qv), oaff.dequantize_values(rv, packed=packed))
