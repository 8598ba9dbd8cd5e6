"""The AKVLayer oracle (oracle/layer.py) against the reference's own cache
tests, restated: position coverage and chronological order
(tests/test_cache_ordering.py), the no-demotion identity (tests/test_bit_exact.py:
the view is the concatenated input, bit for bit), the measured packed bytes
(tests/test_packed_bytes.py:95-127), and closed forms of the importance
recurrence and of the byte counter."""
import numpy as np
import pytest

from oracle import affine as oaff
from oracle.layer import AKVLayerOracle, packed_bytes


def _pos_kv(N, heads=2, head_dim=8):
    """Position-encoded K (every channel of token i is i) as the reference's tests build it."""
    k = np.broadcast_to(np.arange(N, dtype=np.float32).reshape(1, 1, N, 1), (1, heads, N, head_dim))
    return k.astype(np.float16), k.astype(np.float16).copy()


def _layer(**kw):
    kw.setdefault("warm_bits", 3)
    return AKVLayerOracle(**kw)


def test_prefill_no_demote_keeps_positions_in_order():
    layer = _layer(hot_budget=256)
    k, v = _pos_kv(64)
    layer.update(k, v)
    assert layer.warm_pos is None and layer.hot_pos.tolist() == list(range(64))


@pytest.mark.parametrize("N,budget", [(256, 32), (100, 64), (37, 16)])
def test_prefill_with_demote_position_coverage_is_complete(N, budget):
    layer = _layer(hot_budget=budget)
    k, v = _pos_kv(N)
    fk, fv, _ = layer.update(k, v)
    warm, hot = layer.warm_pos.tolist(), layer.hot_pos.tolist()
    assert len(warm) + len(hot) == N and sorted(warm + hot) == list(range(N))
    assert len(hot) == budget and layer.warm_len == N - budget
    # the protected ends stay hot: the first 4 and the last min(16, budget // 4)
    assert set(range(4)) <= set(hot) and set(range(N - min(16, budget // 4), N)) <= set(hot)
    assert fk.shape == (1, 2, N, 8)


def test_full_view_is_chronologically_sorted():
    """Slot i of the view holds token i: hot slots carry the exact input, warm
    slots its per-event dequantized value (the position-encoded K survives 3-bit
    per-channel quantization of a demotion event only approximately)."""
    N = 256
    layer = _layer(hot_budget=32)
    k, v = _pos_kv(N)
    fk, _, _ = layer.update(k, v)
    hot = layer.hot_pos
    np.testing.assert_array_equal(fk[0, 0, hot, 0], k[0, 0, hot, 0])
    # one event: keys per channel over its 224 tokens -> step (max - min) / 7 per code
    warm = layer.warm_pos
    err = np.abs(fk[0, 0, warm, 0].astype(np.float32) - warm.astype(np.float32))
    step = (warm.max() - warm.min()) / 7.0
    assert err.max() <= step / 2 + 0.5


def test_decode_step_appends_at_correct_position():
    layer = _layer(hot_budget=256)
    k, v = _pos_kv(64)
    layer.update(k, v)
    z1 = np.zeros((1, 2, 1, 8), np.float16)
    layer.update(z1, z1)
    assert layer.hot_pos.tolist() == list(range(65))
    z16 = np.zeros((1, 2, 16, 8), np.float16)
    layer.update(z16, z16)
    assert layer.hot_pos.tolist() == list(range(81))


def test_multilayer_independence():
    layers = [_layer(hot_budget=32) for _ in range(3)]
    k, v = _pos_kv(128)
    for layer in layers:
        layer.update(k, v)
    for layer in layers:
        assert sorted(layer.warm_pos.tolist() + layer.hot_pos.tolist()) == list(range(128))


def test_no_demotion_view_is_the_input_bit_for_bit():
    rng = np.random.default_rng(0)
    layer = _layer(hot_budget=1024)
    parts = [rng.standard_normal((2, 4, n, 64)).astype(np.float16) for n in (100, 1, 1, 7)]
    for p in parts:
        fk, fv, dt = layer.update(p, p * np.float16(2))
    np.testing.assert_array_equal(fk.view(np.uint16), np.concatenate(parts, axis=2).view(np.uint16))
    assert dt == "float16"


def test_protected_layer_keeps_everything_hot():
    layer = _layer(hot_budget=4, protect=True)
    k, v = _pos_kv(50)
    fk, _, _ = layer.update(k, v)
    assert layer.warm_k is None and fk.shape[2] == 50


def test_importance_recurrence_closed_form():
    """After updates of n_1, n_2, ... tokens with no demotion, token j of update i
    scores 0.3^(#later updates) in float32 (ones on re-init)."""
    layer = _layer(hot_budget=10_000)
    z = lambda n: np.zeros((1, 1, n, 8), np.float16)
    sizes = [5, 1, 3, 1]
    for n in sizes:
        layer.update(z(n), z(n))
    want = []
    for i, n in enumerate(sizes):
        s = np.float32(1.0)
        for _ in sizes[i + 1:]:
            s = np.float32(s * np.float32(0.3))
        want += [s] * n
    np.testing.assert_array_equal(layer.importance, np.array(want, np.float32))


def test_measured_packed_bytes():
    """tests/test_packed_bytes.py:95-127 restated: two updates of 8 tokens into a
    budget of 4 demote 12 tokens; the measured bytes are positive, below the fp16
    cost, and equal the closed form of each event (codes + fp16 scale and zero)."""
    rng = np.random.default_rng(1)
    layer = _layer(warm_bits=4, hot_budget=4)
    k = rng.standard_normal((1, 2, 8, 64)).astype(np.float32)
    layer.update(k, k.copy())
    layer.update(k, k.copy())
    assert layer.warm_len == 12
    fp16_equiv = layer.total_len * 2 * 64 * 2 * 2
    assert 0 < layer.warm_bytes_packed < fp16_equiv
    want = 0
    for pos, per_b in layer.events:
        n = len(pos)
        # K: (H, n, 64) codes at 4 bits + (H, 1, 64) scale and zero; V: codes + (H, n, 1) scale and zero
        want += 2 * n * 32 + 2 * 2 * 64 * 2 + 2 * n * 32 + 2 * 2 * n * 2
        for qk, qv in per_b:
            assert packed_bytes(qk) + packed_bytes(qv) == 2 * n * 32 + 2 * 2 * 64 * 2 + 2 * n * 32 + 2 * 2 * n * 2
    assert layer.warm_bytes_packed == want


def test_event_working_copy_is_the_quantizer_round_trip():
    """The warm working copy of an event equals dequantize(quantize(.)) of the
    chosen tokens, batch element by batch element, with outliers."""
    rng = np.random.default_rng(2)
    layer = _layer(warm_bits=2, hot_budget=40, outlier_fraction=0.02)
    k = rng.standard_normal((2, 2, 100, 64)).astype(np.float16)
    v = rng.standard_normal((2, 2, 100, 64)).astype(np.float16)
    layer.update(k, v)
    pos = layer.warm_pos
    for b in range(2):
        qk = oaff.quantize_keys(k[b][:, pos], 2, 0.02)
        np.testing.assert_array_equal(layer.warm_k[b].view(np.uint16), oaff.dequantize_keys(qk).view(np.uint16))


# ---------------------------------------------------------------- promotion

def _step(layer, rng, H=4, D=8, n=1, direction=None, scale=1.0):
    if direction is None:
        k = (rng.standard_normal((1, H, n, D)) * scale).astype(np.float32)
    else:
        k = (np.broadcast_to(direction, (1, H, n, D)) + rng.standard_normal((1, H, n, D)) * 0.05).astype(np.float32)
    v = (rng.standard_normal((1, H, n, D)) * scale).astype(np.float32)
    return layer.update(k, v)


def test_proxy_fires_without_attention_weights():
    """tests/test_proxy_promotion.py:31-52 restated."""
    layer = _layer(hot_budget=8, enable_promotion=True, enable_promotion_proxy=True, promotion_threshold=0.0,
                   proxy_decay=0.0)
    rng = np.random.default_rng(0)
    for _ in range(16):
        _step(layer, rng)
    assert layer.warm_len > 0 and layer.proxy is not None and layer.proxy.shape[0] == layer.warm_len


def test_proxy_disabled_skips_path():
    layer = _layer(hot_budget=8, enable_promotion=True, enable_promotion_proxy=False)
    rng = np.random.default_rng(1)
    for _ in range(16):
        _step(layer, rng)
    assert layer.proxy is None


def test_proxy_ranks_similar_warm_slot_highest():
    """tests/test_proxy_promotion.py:72-133 restated."""
    layer = _layer(warm_bits=4, hot_budget=16, enable_promotion=False, enable_promotion_proxy=True, proxy_decay=0.0)
    rng = np.random.default_rng(7)
    H, D = 4, 16
    for _ in range(4):
        _step(layer, rng, H, D)
    target = rng.standard_normal(D).astype(np.float32)
    target /= np.linalg.norm(target)
    layer.update(np.broadcast_to(target, (1, H, 1, D)).astype(np.float32).copy(),
                 rng.standard_normal((1, H, 1, D)).astype(np.float32))
    for _ in range(40):
        _step(layer, rng, H, D)
    assert layer.warm_len > 0
    layer.update((np.broadcast_to(target, (1, H, 1, D)) + 0.01 * rng.standard_normal((1, H, 1, D))).astype(np.float32),
                 rng.standard_normal((1, H, 1, D)).astype(np.float32))
    wk = layer.warm_k.astype(np.float32).mean(axis=(0, 1))
    true = np.abs((wk / (np.linalg.norm(wk, axis=-1, keepdims=True) + 1e-6)) @ target)
    assert int(np.argmax(layer.proxy)) == int(np.argmax(true))


def test_proxy_score_resizes_on_demote():
    layer = _layer(hot_budget=4, enable_promotion=True, enable_promotion_proxy=True, promotion_threshold=10.0,
                   proxy_decay=0.5)
    rng = np.random.default_rng(2)
    for _ in range(8):
        _step(layer, rng, 2, 8)
    assert layer.warm_len > 0 and layer.proxy.shape[0] == layer.warm_len


def test_proxy_closed_form():
    """One proxy update against float64 evaluation of the same formula."""
    layer = _layer(hot_budget=8, enable_promotion=False, enable_promotion_proxy=True, proxy_decay=0.7)
    rng = np.random.default_rng(3)
    for _ in range(12):
        _step(layer, rng)
    prev = layer.proxy.copy()
    wk = layer.warm_k.astype(np.float64).mean(axis=(0, 1))
    k = rng.standard_normal((1, 4, 1, 8)).astype(np.float32)
    probe = k.astype(np.float64).mean(axis=(0, 1, 2))
    probe /= np.linalg.norm(probe) + 1e-6
    sim = np.abs((wk / (np.linalg.norm(wk, axis=-1, keepdims=True) + 1e-6)) @ probe)
    layer.update(k, k)  # no demotion changes the warm set before the proxy update (8 hot + 1 -> 1 demoted after)
    want = 0.7 * prev + 0.3 * sim
    np.testing.assert_allclose(layer.proxy[: len(want)], want, rtol=2e-6, atol=1e-7)


def test_promote_preserves_position_coverage():
    """tests/test_cache_ordering.py:98-124 restated: threshold 0 promotes every step."""
    N = 128
    layer = _layer(hot_budget=16, enable_promotion=True, enable_promotion_proxy=True, promotion_threshold=0.0)
    k, v = _pos_kv(N)
    layer.update(k.astype(np.float32), v.astype(np.float32))
    rng = np.random.default_rng(4)
    for _ in range(8):
        _step(layer, rng, 2, 8)
    warm, hot = layer.warm_pos.tolist(), layer.hot_pos.tolist()
    assert len(warm) + len(hot) == N + 8 and sorted(warm + hot) == list(range(N + 8))
    assert layer.promoted_total >= 8  # max(1, 16 // 8) = 2 per step once the proxy is live


def test_promotion_from_attention_weights():
    """Warm columns above the threshold move to the front of the hot tier with
    importance 2.0, at most max(1, budget // 8) of them (the top ones); the byte
    counter keeps the kept fraction."""
    layer = _layer(hot_budget=32, enable_promotion=True, enable_promotion_proxy=False, promotion_threshold=0.05)
    k, v = _pos_kv(100)
    layer.update(k, v)
    warm_len, hot_len = layer.warm_len, layer.hot_k.shape[2]
    aw = np.full((1, 2, 1, warm_len + hot_len + 1), 0.001, np.float32)
    aw[..., [3, 10, 11, 20, 40, 50]] = [0.2, 0.5, 0.06, 0.3, 0.07, 0.4]  # 6 above the threshold, cap 4
    bytes_before = layer.warm_bytes_packed
    wpos = layer.warm_pos.copy()
    z = np.zeros((1, 2, 1, 8), np.float16)
    layer.update(z, z, attention_weights=aw)
    top4 = sorted([10, 50, 20, 3])
    assert layer.hot_pos[:4].tolist() == wpos[top4].tolist()
    assert layer.warm_len == warm_len - 4 + 5  # 4 promoted, then 33 + 4 - 32 demoted back to the budget
    assert set(wpos[top4].tolist()) <= set(layer.hot_pos.tolist())
    assert layer.warm_bytes_packed >= int(bytes_before * (warm_len - 4) / warm_len)
