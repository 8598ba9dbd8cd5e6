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


def _filled_cache(B=2, seed=31):
    """A cache that has demoted: a 40-token prefill and three one-token steps at a hot
    budget of 16 (promotion off, so the tiers only change by demotion)."""
    import akv
    cache = akv.AKVCache(warm_bits=3, hot_budget=16, enable_promotion=False, enable_promotion_proxy=False)
    k, v = _kv((B, 2, 40, 128), seed)
    views = [cache.update(to_dev(k), to_dev(v), 0)]
    for step in range(3):
        k1, v1 = _kv((B, 2, 1, 128), seed + 1 + step)
        views.append(cache.update(to_dev(k1), to_dev(v1), 0))
    return cache, views[-1]


def test_crop_rewinds_both_tiers():
    """crop(n) keeps positions 0..n-1: the next step's view starts with the old view's
    first n rows (bit for bit) and holds n + 1 tokens; crop below the warm tier's positions
    drops warm tokens too; a negative length counts back from the current one."""
    announce("AKVCache.crop")
    cache, view = _filled_cache()
    fk, fv = view
    assert cache.get_seq_length() == 43 and cache.layers[0]._warm.n > 0
    cache.crop(38)
    assert cache.get_seq_length() == 38
    k1, v1 = _kv((2, 2, 1, 128), 99)
    gk, gv = cache.update(to_dev(k1), to_dev(v1), 0)
    assert gk.shape[2] == 39
    assert torch.equal(gk[:, :, :38], fk[:, :, :38]) and torch.equal(gv[:, :, :38], fv[:, :, :38])
    assert torch.equal(gk[:, :, 38:], to_dev(k1))
    cache.crop(10)  # below positions already in the packed tier
    layer = cache.layers[0]
    assert cache.get_seq_length() == 10 and bool((layer._warm_positions < 10).all())
    assert layer._warm.n == layer._warm_positions.numel() and layer._hot_keys.shape[2] + layer._warm.n == 10
    gk, _ = cache.update(to_dev(k1), to_dev(v1), 0)
    assert gk.shape[2] == 11 and torch.equal(gk[:, :, :10], fk[:, :, :10])
    cache.crop(-3)
    assert cache.get_seq_length() == 8


def test_batch_helpers_iteration_and_legacy_form():
    """batch_repeat_interleave / batch_select_indices reorder both tiers along the batch
    (checked through the chronological view of the next step), __iter__, key_cache /
    value_cache and to_legacy_cache give __getitem__'s tensors, from_legacy_cache feeds
    update, reset empties."""
    import akv
    announce("AKVCache batch helpers / iteration / legacy form")
    cache, view = _filled_cache()
    ref = [t.clone() for t in cache[0]]
    items = list(cache)
    assert len(items) == 1 and all(torch.equal(a, b) for a, b in zip(items[0], ref))
    assert torch.equal(cache.key_cache[0], ref[0]) and torch.equal(cache.value_cache[0], ref[1])
    legacy = cache.to_legacy_cache()
    assert torch.equal(legacy[0][0], ref[0])
    cache.batch_repeat_interleave(2)
    rep = cache[0]
    assert rep[0].shape[0] == 4
    for i, src in enumerate((0, 0, 1, 1)):
        assert torch.equal(rep[0][i], ref[0][src]) and torch.equal(rep[1][i], ref[1][src])
    cache.batch_select_indices(torch.tensor([3, 0], device="cuda"))
    sel = cache[0]
    assert torch.equal(sel[0][0], ref[0][1]) and torch.equal(sel[0][1], ref[0][0])
    cache.crop(42)  # one hot token fewer, so the next step demotes nothing and the old rows stay as they were
    k1, v1 = _kv((2, 2, 1, 128), 77)
    gk, _ = cache.update(to_dev(k1), to_dev(v1), 0)
    assert torch.equal(gk[0, :, :42], view[0][1, :, :42]) and torch.equal(gk[1, :, :42], view[0][0, :, :42])
    k, v = _kv((1, 2, 5, 128), 5)
    c2 = akv.AKVCache.from_legacy_cache(((to_dev(k), to_dev(v)), (to_dev(k), to_dev(v))))
    assert len(c2) == 2 and c2.get_seq_length(1) == 5 and torch.equal(c2[1][0], to_dev(k))
    c2.reset()
    assert len(c2) == 0
