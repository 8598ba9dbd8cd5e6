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
