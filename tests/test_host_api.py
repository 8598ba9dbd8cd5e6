"""Host-side behaviour of the akv package that needs no GPU: presets, errors,
refusal of CPU tensors (there is no CPU path)."""
import pytest
import torch


def test_presets_table():
    import akv
    p = akv._PRESETS
    assert set(p) == {"quality", "balanced", "compact", "k4v2", "k4v3"}
    assert (p["quality"]["warm_bits"], p["quality"]["hot_budget"]) == (4, 256)
    assert (p["balanced"]["warm_bits"], p["balanced"]["hot_budget"]) == (3, 128)
    assert (p["compact"]["warm_bits"], p["compact"]["hot_budget"]) == (2, 64)
    assert (p["k4v2"]["warm_key_bits"], p["k4v2"]["warm_value_bits"]) == (4, 2)
    assert (p["k4v3"]["warm_key_bits"], p["k4v3"]["warm_value_bits"]) == (4, 3)


def test_preset_resolution_and_errors():
    import akv
    c = akv.AKVCache(preset="k4v2")
    assert (c.warm_bits, c.hot_budget, c.warm_key_bits, c.warm_value_bits) == (4, 128, 4, 2)
    c = akv.AKVCache(preset="balanced")
    assert (c.warm_key_bits, c.warm_value_bits, c.group_size, c.outlier_fraction) == (3, 3, 64, 0.0)
    c = akv.AKVCache(warm_bits=2, hot_budget=32, warm_value_bits=4)
    assert (c.warm_key_bits, c.warm_value_bits) == (2, 4)
    c = akv.AKVCache()
    assert (c.warm_bits, c.hot_budget) == (3, 128)
    with pytest.raises(ValueError, match="Unknown preset"):
        akv.AKVCache(preset="nope")
    with pytest.raises(ValueError, match="mutually exclusive"):
        akv.AKVCache(preset="quality", warm_bits=4)
    with pytest.raises(ValueError, match="mutually exclusive"):
        akv.AKVCache(preset="quality", hot_budget=8)


def test_cpu_tensors_are_refused():
    import akv
    k = torch.zeros(1, 1, 32, 128, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="ROCm devices only"):
        akv.quantize_kv(k, k)
    with pytest.raises(RuntimeError, match="ROCm devices only"):
        akv.pack(torch.zeros(2, 8, dtype=torch.uint8), 4)
    q = torch.zeros(1, 2, 1, 64, dtype=torch.float16)
    with pytest.raises(AssertionError):
        akv.fused_decode_attention(torch.zeros(1, 2, 2, 64, dtype=torch.float16), q, q)
    with pytest.raises(RuntimeError, match="ROCm devices only"):
        akv.fused_decode_attention(q, torch.zeros(1, 2, 4, 64, dtype=torch.float16),
                                   torch.zeros(1, 2, 4, 64, dtype=torch.float16))


def test_legacy_bits_and_config_errors():
    import akv
    with pytest.raises(ValueError):
        akv.QuantConfig(bits=3)
    with pytest.raises(ValueError):
        akv.QuantConfig(group_size=0)
    assert akv.HAS_TRITON is False


def test_workload_shapes():
    from akv import workloads as wl
    s = wl.QWEN_DECODE_32K
    assert (s.B, s.Hq, s.Hkv, s.N, s.n_hot, s.bits_k, s.layers, s.decay) == (8, 12, 2, 32768, 1024, 3, 28, 0.9)
    k, v = wl.make_kv(wl.DecodeShape("t", 1, 2, 2, 128, 4, 60, 3, 3, k_outlier_channels=2))
    assert k.dtype == torch.float16 and k.shape == (1, 2, 64, 128)
    # two channels per head scaled x10
    std = k.float().std(dim=2)[0]
    assert int((std > 5).sum()) == 4


def test_decode_workspace_tracks_the_last_counter_region():
    """A reused decode workspace: after a call only that call's counter prefix is known
    to be zero (its partials follow it), so a later call with a larger counter region
    must find it cleared again.  Runs on host memory; the 'call' is simulated by
    writing partial bytes after the counter prefix."""
    from akv._native import DecodeWorkspace
    ws = DecodeWorkspace()
    buf = ws.get(4096, 512, "cpu")
    assert int(buf[:512].sum()) == 0
    buf = ws.get(4096, 256, "cpu")  # a smaller region: no clearing needed
    buf[256:1024] = 7  # that call's partials land over the old counter tail
    buf = ws.get(4096, 512, "cpu")
    assert int(buf[:512].sum()) == 0, "the grown counter region was not cleared"
    buf[512:] = 3
    assert ws.get(4096, 512, "cpu") is buf and int(buf[:512].sum()) == 0
    assert ws.get(8192, 256, "cpu").numel() >= 8192  # grows when a call needs more bytes


def test_estimate_memory_savings_closed_form():
    """KVQuantizer.estimate_memory_savings (akv/quantizer.py:256-272) at 32 layers x 32
    heads x 4096 tokens x 128: fp16 K and V 2,147,483,648 B; 4-bit data 536,870,912 B;
    one group of 128 -> fp16 scale + zero per (layer, K/V, head, token) 33,554,432 B."""
    import akv
    q = akv.KVQuantizer(akv.QuantConfig(bits=4, group_size=128))
    s = q.estimate_memory_savings(num_layers=32, num_heads=32, seq_len=4096, head_dim=128, bits=4)
    assert s["original_mb"] == 2147.483648
    assert abs(s["quantized_mb"] - 570.425344) < 1e-9
    assert abs(s["savings_mb"] - (2147.483648 - 570.425344)) < 1e-9
    assert abs(s["compression_ratio"] - 2147483648 / 570425344) < 1e-12
    # 2 bits with groups of 32: 4 groups per row, data a quarter byte per value
    s = akv.KVQuantizer(akv.QuantConfig(bits=2, group_size=32)).estimate_memory_savings(1, 1, 10, 128)
    assert s["original_mb"] == 1 * 2 * 1 * 10 * 128 * 2 / 1e6
    assert abs(s["quantized_mb"] - (2 * 10 * 128 * 2 / 8 + 2 * 10 * 4 * 4) / 1e6) < 1e-12


def test_cache_length_queries_and_arena_config():
    """AKVCache.get_usable_length is the layer's sequence length and get_max_length is
    None (akv/drop_in.py:1104-1110); PackedKVConfig's derived sizes
    (akv/packed_layout.py:41-53): values per byte, packed head_dim, groups per row."""
    import akv
    from akv.packed_layout import PackedKVConfig
    cache = akv.AKVCache()
    assert cache.get_usable_length(4096) == 0 and cache.get_usable_length(16, layer_idx=3) == 0
    assert cache.get_max_length() is None
    for bits, pf in ((2, 4), (4, 2), (8, 1)):
        c = PackedKVConfig(head_dim=128, bits=bits, group_size=48, device="cpu")
        assert (c.pack_factor, c.packed_dim, c.num_groups) == (pf, 128 // pf, 3)


class _Cfg:
    def __init__(self, **kw):
        self.__dict__.update(kw)


class _Model:
    def __init__(self, **kw):
        self.config = _Cfg(**kw)


def test_recommend_preset_thresholds():
    """recommend_preset (akv/drop_in.py:1321-1366): layers x kv-heads x head_dim^2 x 4
    against 5e9 and 1e9 (so common models land in the last branch: Qwen2.5-1.5B is 3.7e6)."""
    import akv
    assert akv.recommend_preset(object())["preset"] == "balanced"
    big = akv.recommend_preset(_Model(num_hidden_layers=100, num_key_value_heads=128, head_dim=512))  # 1.3e10
    assert (big["preset"], big["warm_bits"], big["hot_budget"], big["protect_first"]) == ("balanced", 3, 128, 2)
    mid = akv.recommend_preset(_Model(num_hidden_layers=64, num_key_value_heads=64, head_dim=256))  # 1.07e9
    assert (mid["preset"], mid["warm_bits"], mid["hot_budget"], mid["protect_last"]) == ("quality", 4, 256, 1)
    small = akv.recommend_preset(_Model(num_hidden_layers=28, num_key_value_heads=2, hidden_size=1536,
                                        num_attention_heads=12))  # head_dim 128 from hidden / heads
    assert (small["preset"], small["hot_budget"], small["protect_first"]) == ("quality", 512, 2)


def test_for_model_and_from_calibration(tmp_path):
    import json
    import akv
    c = akv.AKVCache.for_model(_Model(num_hidden_layers=12), preset="compact", protect_last=2)
    assert c.num_hidden_layers == 12 and c._is_protected(11) and c._is_protected(10) and not c._is_protected(9)
    assert akv.AKVCache.for_model(_Model(n_layer=6)).num_hidden_layers == 6
    with pytest.raises(ValueError, match="no .config"):
        akv.AKVCache.for_model(object())
    with pytest.raises(ValueError, match="num_hidden_layers"):
        akv.AKVCache.for_model(_Model(hidden_size=64))
    rep = {"model_name": "m", "model_type": "llama", "num_layers": 8, "num_kv_heads": 2, "head_dim": 128,
           "kv_outlier_ratio": 3.0, "attention_entropy_mean": 1.0, "attention_sink_strength": 0.1,
           "recommended_preset": "quality", "recommended_protect_first": 1, "recommended_protect_last": 1,
           "recommended_average_bits": 2.6, "per_head_bits": {"0": [2, 4], "3": [3, 3]}, "sensitivities": []}
    path = tmp_path / "calib.json"
    path.write_text(json.dumps(rep))
    c = akv.AKVCache.from_calibration(str(path))
    assert c.warm_bits == 3 and c.num_hidden_layers == 8 and c._is_protected(0) and c._is_protected(7)
    assert c._calibration_per_head_bits == {0: [2, 4], 3: [3, 3]}
    rep["recommended_average_bits"] = 6.0
    path.write_text(json.dumps(rep))
    c = akv.AKVCache.from_calibration(str(path), protect_first=0)
    assert c.preset == "quality" and c.warm_bits == 4 and not c._is_protected(0)


def test_empty_cache_views_and_reset():
    import akv
    c = akv.AKVCache()
    assert list(c) == [] and c.to_legacy_cache() == () and c.key_cache == [] and c.value_cache == []
    c._seen_tokens = 5
    c.reset()
    assert len(c) == 0 and c.seen_tokens == 0


def test_layer_constructor_parameter_order():
    """AKVLayer's parameters in the reference's order (akv/drop_in.py:162-177), so
    positional calls bind as they do there."""
    import inspect
    import akv
    params = list(inspect.signature(akv.AKVLayer.__init__).parameters)[1:]
    assert params == ["warm_bits", "hot_budget", "group_size", "protect", "enable_promotion",
                      "promotion_threshold", "per_head_bits", "enable_promotion_proxy", "proxy_decay",
                      "adaptive_hot_frac", "warm_key_bits", "warm_value_bits", "outlier_fraction"]
