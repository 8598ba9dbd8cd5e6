"""AKVLayer / AKVCache.update with the packed warm tier against the oracle's
restatement of the reference's update path (oracle/layer.py): every returned
view bit-exact over prefill + decode + chunk sequences (fp16 views; float32
views for bf16 / fp32 tokens), the measured packed bytes, the position
bookkeeping, protected layers, __getitem__'s demotion-order view and
reorder_cache."""
import numpy as np
import pytest
import torch

from gpu_util import announce, to_dev
from oracle.fp import BF16, F16, F32, to_dtype
from oracle.layer import AKVLayerOracle

pytestmark = pytest.mark.gpu

_DT = {torch.float16: F16, torch.bfloat16: BF16, torch.float32: F32}


def _tokens(rng, B, H, n, D, dtype):
    x = (rng.standard_normal((B, H, n, D)) * 1.3).astype(np.float32)
    x[..., 7] *= 8.0  # a loud channel (picked as the outlier when outliers are on)
    host = to_dtype(x, _DT[dtype]).astype(np.float32)
    t = torch.from_numpy(host).to(dtype).cuda()
    return t, (host.astype(np.float16) if dtype == torch.float16 else host)


def _same(got: torch.Tensor, want: np.ndarray, what: str):
    g = got.cpu()
    if g.dtype == torch.float16:
        gv, wv = g.numpy().view(np.uint16), np.asarray(want, np.float16).view(np.uint16)
    else:
        gv, wv = g.float().numpy().view(np.uint32), np.asarray(want, np.float32).view(np.uint32)
    assert gv.shape == wv.shape, f"{what}: shape {gv.shape} != {wv.shape}"
    bad = np.count_nonzero(gv != wv)
    assert bad == 0, f"{what}: {bad} of {gv.size} values differ"


def _run(layer, orc, B, H, D, dtype, chunks, seed):
    rng = np.random.default_rng(seed)
    for step, n in enumerate(chunks):
        announce(f"layer update step {step}: {n} tokens")
        k, kh = _tokens(rng, B, H, n, D, dtype)
        v, vh = _tokens(rng, B, H, n, D, dtype)
        fk, fv = layer.update(k, v)
        ok, ov, _ = orc.update(kh, vh, dt=_DT[dtype])
        _same(fk, ok, f"K view after step {step}")
        _same(fv, ov, f"V view after step {step}")
        assert layer._total_len == orc.total_len and layer._warm_len == orc.warm_len
        if orc.warm_pos is not None:
            assert layer._warm_positions.tolist() == orc.warm_pos.tolist()
        assert layer._hot_positions.tolist() == orc.hot_pos.tolist()
        assert layer._warm_bytes_packed == orc.warm_bytes_packed


@pytest.mark.parametrize("kb,vb,of,D", [(3, 3, 0.0, 128), (4, 2, 0.01, 128), (2, 2, 0.0, 64), (4, 4, 0.02, 128)])
def test_update_views_match_oracle(kb, vb, of, D):
    from akv.drop_in import AKVLayer
    announce(f"AKVLayer K{kb}/V{vb} outliers {of} D={D}")
    B, H = 2, 4
    layer = AKVLayer(warm_bits=kb, warm_key_bits=kb, warm_value_bits=vb, hot_budget=64, outlier_fraction=of,
                     enable_promotion=False)
    orc = AKVLayerOracle(warm_bits=kb, warm_key_bits=kb, warm_value_bits=vb, hot_budget=64, outlier_fraction=of)
    _run(layer, orc, B, H, D, torch.float16, [300] + [1] * 12 + [17, 1, 40], seed=kb * 10 + vb)
    stats = layer.memory_usage_bytes()
    assert 0 < stats["warm_bytes_packed"] < stats["fp16_equivalent_bytes"]
    assert stats["warm_bytes_packed"] <= stats["warm_bytes_live"]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_update_non_fp16_tokens(dtype):
    """bf16 / fp32 tokens: the demotion quantizes in that dtype, the view is float32
    (float16 warm values beside the exact hot tokens, as torch.cat promotes)."""
    from akv.drop_in import AKVLayer
    announce(f"AKVLayer {dtype} tokens")
    layer = AKVLayer(warm_bits=3, hot_budget=32, enable_promotion=False)
    orc = AKVLayerOracle(warm_bits=3, hot_budget=32)
    _run(layer, orc, 1, 2, 128, dtype, [100, 1, 1, 9], seed=4)


def test_adaptive_budget_and_protected_layers():
    from akv.drop_in import AKVCache
    announce("AKVCache.update: protected first layer, adaptive budget")
    B, H, D = 1, 2, 128
    cache = AKVCache(warm_bits=4, hot_budget=32, adaptive_hot_frac=0.25, protect_first=1, enable_promotion=False,
                     num_hidden_layers=3)
    orcs = [None] + [AKVLayerOracle(warm_bits=4, hot_budget=32, adaptive_hot_frac=0.25) for _ in range(2)]
    rng = np.random.default_rng(8)
    seen = []
    for step, n in enumerate([200, 1, 1, 30]):
        k, kh = _tokens(rng, B, H, n, D, torch.float16)
        v, vh = _tokens(rng, B, H, n, D, torch.float16)
        seen.append(kh)
        for li in range(3):
            fk, fv = cache.update(k, v, li)
            if li == 0:
                _same(fk, np.concatenate(seen, axis=2), "protected layer")
            else:
                ok, ov, _ = orcs[li].update(kh, vh)
                _same(fk, ok, f"layer {li} step {step}")
                _same(fv, ov, f"layer {li} step {step}")
    assert cache.seen_tokens == 232 and cache.get_seq_length(1) == 232
    assert cache.layers[1]._hot_keys.shape[2] == max(32, int(0.25 * 232))
    rep = cache.memory_report()
    assert rep["num_layers"] == 3 and rep["seq_length"] == 232 and rep["savings_ratio"] > 1.0
    # the aggregator's keys (tests/test_memory_alignment.py:140-165)
    stats = cache.memory_usage()
    assert set(stats) == {"hot_bytes", "warm_bytes", "warm_bytes_live", "warm_bytes_packed", "warm_bytes_formula",
                          "total_bytes", "fp16_equivalent_bytes", "savings_ratio", "num_layers"}
    assert 0 < stats["warm_bytes"] == stats["warm_bytes_packed"] <= stats["warm_bytes_live"]
    assert stats["total_bytes"] == stats["hot_bytes"] + stats["warm_bytes_packed"]


def test_getitem_and_reorder_cache():
    from akv.drop_in import AKVCache
    announce("AKVCache __getitem__ / reorder_cache")
    B, H, D = 2, 2, 128
    cache = AKVCache(warm_bits=3, hot_budget=16, enable_promotion=False)
    orc = AKVLayerOracle(warm_bits=3, hot_budget=16)
    rng = np.random.default_rng(5)
    k, kh = _tokens(rng, B, H, 80, D, torch.float16)
    v, vh = _tokens(rng, B, H, 80, D, torch.float16)
    cache.update(k, v, 0)
    orc.update(kh, vh)
    gk, gv = cache[0]
    _same(gk, np.concatenate([orc.warm_k, orc.hot_k], axis=2), "__getitem__ K (demotion order, then hot)")
    _same(gv, np.concatenate([orc.warm_v, orc.hot_v], axis=2), "__getitem__ V")
    cache.reorder_cache(torch.tensor([1, 0], device="cuda"))
    k2, kh2 = _tokens(rng, B, H, 1, D, torch.float16)
    fk, _ = cache.update(k2, k2, 0)
    ok, _, _ = orc.update(kh2[::-1].copy(), kh2[::-1].copy())
    _same(fk.flip(0), ok, "view after reorder_cache([1, 0])")


@pytest.mark.parametrize("of", [0.0, 0.02])
def test_per_head_bits_match_oracle(of):
    """Calibrated per-head widths: each (batch element, head) is quantized at its own
    width with its own outlier channels; views, positions, packed bytes and the warm
    view in demotion order match the oracle, through a promotion from attention
    weights and a reorder_cache."""
    from akv.drop_in import AKVCache, AKVLayer
    announce(f"AKVLayer per-head widths, outliers {of}")
    B, H, D, bits = 2, 4, 128, [2, 4, 3, 4]
    layer = AKVLayer(warm_bits=3, hot_budget=48, outlier_fraction=of, enable_promotion=True,
                     enable_promotion_proxy=False, per_head_bits=bits)
    orc = AKVLayerOracle(warm_bits=3, hot_budget=48, outlier_fraction=of, enable_promotion=True,
                         enable_promotion_proxy=False, per_head_bits=bits)
    _run(layer, orc, B, H, D, torch.float16, [200] + [1] * 5 + [30, 1], seed=31)
    wk, wv = layer.warm_view()
    _same(wk, orc.warm_k, "warm view K (demotion order)")
    _same(wv, orc.warm_v, "warm view V")
    # promotion from attention weights takes tokens out of every width's tier
    rng = np.random.default_rng(32)
    n_all = orc.warm_len + orc.hot_k.shape[2] + 1
    aw = np.full((B, H, 1, n_all), 0.001, np.float32)
    aw[..., [1, 7, 30]] = [0.3, 0.2, 0.5]
    k, kh = _tokens(rng, B, H, 1, D, torch.float16)
    v, vh = _tokens(rng, B, H, 1, D, torch.float16)
    fk, fv = layer.update(k, v, {"attention_weights": to_dev(aw)})
    ok, ov, _ = orc.update(kh, vh, attention_weights=aw)
    _same(fk, ok, "K view after the promotion")
    _same(fv, ov, "V view after the promotion")
    assert orc.promoted_total == 3 and layer._warm_bytes_packed == orc.warm_bytes_packed
    # another head count: the global widths apply (the reference's fallback)
    k = torch.zeros(1, 2, 4, 128, dtype=torch.float16, device="cuda")
    AKVLayer(hot_budget=2, enable_promotion=False, per_head_bits=[2, 4, 4]).update(k, k)
    # reorder_cache over the per-width tiers
    cache = AKVCache(warm_bits=3, hot_budget=16, enable_promotion=False)
    cache._calibration_per_head_bits = {0: [2, 4]}
    orc2 = AKVLayerOracle(warm_bits=3, hot_budget=16, per_head_bits=[2, 4])
    k, kh = _tokens(rng, 2, 2, 60, D, torch.float16)
    v, vh = _tokens(rng, 2, 2, 60, D, torch.float16)
    cache.update(k, v, 0)
    orc2.update(kh, vh)
    cache.reorder_cache(torch.tensor([1, 0], device="cuda"))
    k2, kh2 = _tokens(rng, 2, 2, 1, D, torch.float16)
    fk, _ = cache.update(k2, k2, 0)
    ok, _, _ = orc2.update(kh2[::-1].copy(), kh2[::-1].copy())
    _same(fk.flip(0), ok, "view after reorder_cache([1, 0]) with per-head widths")


def test_calibrated_widths_reach_their_layers(tmp_path):
    """tests/test_per_head_bits.py restated: a calibration report's widths reach the
    layers it names, one packed tier per distinct width; an uncalibrated layer keeps
    the global width; a layer whose head count differs from its calibration falls back
    to the global width and still demotes."""
    import json
    from akv.drop_in import AKVCache, AKVLayer, _HeadBitsTier
    announce("per-head widths from a calibration report")
    rep = {"model_name": "x", "model_type": "llama", "num_layers": 4, "num_kv_heads": 2, "head_dim": 64,
           "recommended_preset": "balanced", "recommended_protect_first": 0, "recommended_protect_last": 0,
           "recommended_average_bits": 3.0, "per_head_bits": {"0": [2, 3], "1": [4, 4]}}
    path = tmp_path / "calib.json"
    path.write_text(json.dumps(rep))
    cache = AKVCache.from_calibration(str(path), hot_budget=2, enable_promotion=False)
    g = torch.Generator().manual_seed(41)
    k = torch.randn(1, 2, 6, 64, generator=g).half().cuda()
    v = torch.randn(1, 2, 6, 64, generator=g).half().cuda()
    for li in range(3):
        cache.update(k, v, li)
    assert cache.layers[0].per_head_bits == [2, 3] and cache.layers[1].per_head_bits == [4, 4]
    assert cache.layers[2].per_head_bits is None
    assert [grp[0] for grp in cache.layers[0]._warm.groups] == [2, 3]
    assert [grp[0] for grp in cache.layers[1]._warm.groups] == [4]
    assert not isinstance(cache.layers[2]._warm, _HeadBitsTier)
    for li in range(3):
        layer = cache.layers[li]
        assert layer._warm_len == 4 and layer.get_seq_length() == 6
    # one more token through the per-width tiers: the view holds all seven
    fk0, _ = cache.layers[0].update(k[:, :, :1], v[:, :, :1])
    assert fk0.shape == (1, 2, 7, 64) and torch.isfinite(fk0).all()

    layer = AKVLayer(warm_bits=3, hot_budget=2, enable_promotion=False, per_head_bits=[2, 3, 4, 2])
    fk, fv = layer.update(k[:, :, :4], v[:, :, :4])
    assert layer._warm_len == 2 and not isinstance(layer._warm, _HeadBitsTier)
    assert fk.shape == fv.shape == (1, 2, 4, 64)


def test_promotion_from_attention_weights():
    """Warm columns of the attention weights above the threshold (6 of them, cap 4):
    the top 4 return to the front of the hot tier with their float16 values."""
    from akv.drop_in import AKVLayer
    announce("AKVLayer promotion from attention weights")
    B, H, D = 1, 2, 128
    layer = AKVLayer(warm_bits=3, hot_budget=32, enable_promotion=True, enable_promotion_proxy=False)
    orc = AKVLayerOracle(warm_bits=3, hot_budget=32, enable_promotion=True, enable_promotion_proxy=False)
    rng = np.random.default_rng(11)
    k, kh = _tokens(rng, B, H, 100, D, torch.float16)
    v, vh = _tokens(rng, B, H, 100, D, torch.float16)
    layer.update(k, v)
    orc.update(kh, vh)
    warm_len, hot_len = orc.warm_len, orc.hot_k.shape[2]
    aw = np.full((B, H, 1, warm_len + hot_len + 1), 0.001, np.float32)
    aw[..., [3, 10, 11, 20, 40, 50]] = [0.2, 0.5, 0.06, 0.3, 0.07, 0.4]
    for step in range(3):
        k, kh = _tokens(rng, B, H, 1, D, torch.float16)
        v, vh = _tokens(rng, B, H, 1, D, torch.float16)
        fk, fv = layer.update(k, v, {"attention_weights": to_dev(aw)} if step == 0 else None)
        ok, ov, _ = orc.update(kh, vh, attention_weights=aw if step == 0 else None)
        _same(fk, ok, f"K view after step {step}")
        _same(fv, ov, f"V view after step {step}")
        assert layer._hot_positions.tolist() == orc.hot_pos.tolist()
        assert layer._warm_positions.tolist() == orc.warm_pos.tolist()
        assert layer._warm_bytes_packed == orc.warm_bytes_packed
        np.testing.assert_array_equal(layer._importance.cpu().numpy(), orc.importance)


@pytest.mark.parametrize("threshold,decay", [(0.0, 0.0), (0.2, 0.7)])
def test_proxy_promotion_matches_oracle(threshold, decay):
    """The proxy (float32 reductions: within 2e-5 of the oracle's) and the
    promotions it drives, over a prefill and decode steps; views bit-exact."""
    from akv.drop_in import AKVLayer
    announce(f"AKVLayer proxy promotion threshold={threshold} decay={decay}")
    B, H, D = 2, 2, 128
    layer = AKVLayer(warm_bits=4, hot_budget=24, enable_promotion=True, enable_promotion_proxy=True,
                     promotion_threshold=threshold, proxy_decay=decay)
    orc = AKVLayerOracle(warm_bits=4, hot_budget=24, enable_promotion=True, enable_promotion_proxy=True,
                         promotion_threshold=threshold, proxy_decay=decay)
    rng = np.random.default_rng(12)
    for step, n in enumerate([120] + [1] * 10 + [5]):
        k, kh = _tokens(rng, B, H, n, D, torch.float16)
        v, vh = _tokens(rng, B, H, n, D, torch.float16)
        fk, fv = layer.update(k, v)
        ok, ov, _ = orc.update(kh, vh)
        if orc.proxy is not None:
            np.testing.assert_allclose(layer._proxy_score.cpu().numpy(), orc.proxy, rtol=2e-5, atol=2e-6)
        _same(fk, ok, f"K view after step {step}")
        _same(fv, ov, f"V view after step {step}")
        assert layer._hot_positions.tolist() == orc.hot_pos.tolist()
    assert orc.promoted_total > 0
