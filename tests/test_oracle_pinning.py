"""Pin each oracle function with checks that a plausible mistake would fail:
float64 / exact brute force, invariants, and special cases."""
import math
from fractions import Fraction

import numpy as np
import pytest

from oracle import affine as oaff
from oracle import attention as oatt
from oracle import bitpack as obp
from oracle import fp as ofp
from oracle import importance as oimp
from oracle import legacy as oleg
from oracle import selection as osel


# ---------------------------------------------------------------- fp helpers

def _rne_exact(x: Fraction, mant: int, emin: int) -> Fraction:
    if x == 0:
        return Fraction(0)
    s = -1 if x < 0 else 1
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, emin)
    ulp = Fraction(2) ** (e - mant)
    q = a / ulp
    n = q.numerator // q.denominator
    r = q - n
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and n % 2):
        n += 1
    return s * n * ulp


def test_numpy_fp16_ops_are_correctly_rounded():
    rng = np.random.default_rng(0)
    a = rng.standard_normal(3000).astype(np.float16)
    b = (rng.random(3000) * 3 + 0.01).astype(np.float16)
    for op in (np.add, np.subtract, np.multiply, np.divide):
        got = op(a, b)
        for x, y, g in zip(a[:400], b[:400], got[:400]):
            ex = {np.add: Fraction(float(x)) + Fraction(float(y)),
                  np.subtract: Fraction(float(x)) - Fraction(float(y)),
                  np.multiply: Fraction(float(x)) * Fraction(float(y)),
                  np.divide: Fraction(float(x)) / Fraction(float(y))}[op]
            assert Fraction(float(g)) == _rne_exact(ex, 10, -14)


def test_round_bf16_exact_and_ties():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(2000) * 10).astype(np.float32)
    got = ofp.round_bf16(x)
    for v, g in zip(x, got):
        assert Fraction(float(g)) == _rne_exact(Fraction(float(v)), 7, -126)
    # exact ties go to even
    t = np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8], np.float32)
    np.testing.assert_array_equal(ofp.round_bf16(t), np.array([1.0, 1.0 + 2 ** -6], np.float32))


def test_to_u8_matches_torch_table():
    # torch 2.10 on the CPU prints these for float -> uint8
    x = np.array([-1.0, 255.0, 256.0, np.nan, np.inf, -0.4, 7.9], np.float32)
    assert list(ofp.to_u8(x)) == [255, 255, 0, 0, 0, 0, 7]


# ------------------------------------------------------------------- bitpack

def _pack_bruteforce(codes, bits):
    """Bit-by-bit packer from the bit positions (independent of the oracle's shifts)."""
    out_bits = []
    if bits == 3:
        n = -(-len(codes) // 8) * 8
    elif bits == 4:
        n = -(-len(codes) // 2) * 2
    else:
        n = -(-len(codes) // 4) * 4
    c = list(codes) + [0] * (n - len(codes))
    for v in c:
        for k in range(bits - 1, -1, -1):
            out_bits.append((int(v) >> k) & 1)
    return [int("".join(map(str, out_bits[i:i + 8])), 2) for i in range(0, len(out_bits), 8)]


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_bitpack_bruteforce_and_roundtrip(bits):
    rng = np.random.default_rng(bits)
    for dim in (64, 128, 256, 8, 16, 24):
        codes = rng.integers(0, 1 << bits, (5, dim), dtype=np.uint8)
        p = obp.pack(codes, bits)
        for r in range(5):
            assert list(p[r]) == _pack_bruteforce(codes[r], bits)
        np.testing.assert_array_equal(obp.unpack(p, bits, dim), codes)
        assert p.shape[-1] == obp.packed_row_bytes(dim, bits)
    assert obp.pack(np.arange(8, dtype=np.uint8), 8) is not None


def test_bitpack_sizes_reference_tests():
    # tests/test_bitpack.py:13-55 and tests/test_packed_bytes.py:24-54 of the reference
    for dim in (64, 128, 256):
        assert obp.pack(np.zeros((2, 32, dim), np.uint8), 4).shape[-1] == dim // 2
        assert obp.pack(np.zeros((2, 32, dim), np.uint8), 3).shape[-1] == dim * 3 // 8
        assert obp.pack(np.zeros((2, 32, dim), np.uint8), 2).shape[-1] == dim // 4
    x = np.random.default_rng(0).integers(0, 16, (2, 32), dtype=np.uint8)
    p = obp.pack_uint4(x)
    np.testing.assert_array_equal((p >> 4) & 15, x[..., 0::2])
    np.testing.assert_array_equal(p & 15, x[..., 1::2])


# ------------------------------------------------------------------- affine

def _bruteforce_codes(x16: np.ndarray, bits: int):
    """Nearest level (ties to even) in float64 from the fp16-rounded intermediates."""
    maxv = (1 << bits) - 1
    mn, mx = float(x16.min()), float(x16.max())
    scale = float(np.float16(np.float16(mx - mn) / np.float16(maxv)))
    codes = []
    for v in x16.astype(np.float64):
        d = float(np.float16(v - mn))
        if scale == 0:
            codes.append(0 if d == 0 else maxv)
            continue
        q = float(np.float16(d / scale))
        best = None
        for lev in range(maxv + 1):  # enumerate every level
            dist = abs(q - lev)
            if best is None or dist < best[0] - 1e-12 or (abs(dist - best[0]) <= 1e-12 and lev % 2 == 0):
                best = (dist, lev)
        codes.append(best[1] if q <= maxv + 0.5 else maxv)
    return np.array(codes, np.uint8), scale


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_affine_codes_bruteforce(bits):
    rng = np.random.default_rng(bits + 10)
    for trial in range(60):
        x = (rng.standard_normal(12) * rng.choice([0.01, 1, 30])).astype(np.float16)
        q = oaff.quantize_keys(x.reshape(1, -1, 1), bits, packed=False)
        ref, scale = _bruteforce_codes(x, bits)
        np.testing.assert_array_equal(q["codes"].ravel(), ref)
        assert float(q["scale"].ravel()[0]) == scale


def test_affine_fp32_input_path():
    """fp32 input: fp32 arithmetic, scale clamp 1e-8 active, scale stored as fp16."""
    x = np.full((1, 4, 2), 2.0, np.float32)
    q = oaff.quantize_keys(x, 3, packed=False)
    assert np.all(q["codes"] == 0)
    assert np.all(q["scale"] == np.float16(1e-8))  # 1e-8 in fp16 is 0 -> clamp result rounds to 0
    x[0, :, 0] = [0.0, 1.0, 2.0, 3.5]
    q = oaff.quantize_keys(x, 3, packed=False)
    assert list(q["codes"][0, :, 0]) == [0, 2, 4, 7]


def test_blocked_equals_single_call():
    rng = np.random.default_rng(3)
    k = rng.standard_normal((1, 3, 64, 128)).astype(np.float16)
    v = rng.standard_normal((1, 3, 64, 128)).astype(np.float16)
    w = oaff.quantize_kv_blocked(k, v, 3, 4, T=64, G=128)
    qk = oaff.quantize_keys(k[0], 3)
    qv = oaff.quantize_values(v[0], 4)
    np.testing.assert_array_equal(w["k_codes"][0], qk["codes"])
    np.testing.assert_array_equal(w["k_scale"][0], qk["scale"])
    np.testing.assert_array_equal(w["v_codes"][0], qv["codes"])
    np.testing.assert_array_equal(w["v_scale"][0], qv["scale"])
    kd, vd = oaff.dequant_kv_blocked(w)
    np.testing.assert_array_equal(kd[0], oaff.dequantize_keys(qk))
    np.testing.assert_array_equal(vd[0], oaff.dequantize_values(qv))


def test_outlier_ranking_and_restore():
    rng = np.random.default_rng(4)
    k = rng.standard_normal((2, 16, 64)).astype(np.float16)
    k[:, :, 9] *= 20
    k[:, :, 33] *= 8
    q = oaff.quantize_keys(k, 2, outlier_fraction=2 / 64)
    assert list(q["outlier_idx"]) == [9, 33]
    d = oaff.dequantize_keys(q)
    np.testing.assert_array_equal(d[..., [9, 33]], k[..., [9, 33]])
    assert np.all(q["scale"][..., 9] == 0)  # channel zeroed before min/max


def test_group_v_changes_only_value_meta():
    rng = np.random.default_rng(5)
    k = rng.standard_normal((1, 2, 32, 128)).astype(np.float16)
    v = rng.standard_normal((1, 2, 32, 128)).astype(np.float16)
    a = oaff.quantize_kv_blocked(k, v, 3, 3, 32, 32)
    b = oaff.quantize_kv_blocked(k, v, 3, 3, 32, 128)
    np.testing.assert_array_equal(a["k_codes"], b["k_codes"])
    assert a["v_scale"].shape[-1] == 4 and b["v_scale"].shape[-1] == 1
    # per 32-channel groups reconstruct V at least as well as one group per token
    _, va = oaff.dequant_kv_blocked(a)
    _, vb = oaff.dequant_kv_blocked(b)
    assert np.abs(va.astype(np.float32) - v).mean() < np.abs(vb.astype(np.float32) - v).mean()


# ------------------------------------------------------------------- legacy

def test_dequantize_packed_closed_form_every_code():
    for bits in (2, 4, 8):
        maxv = (1 << bits) - 1
        codes = np.arange(maxv + 1, dtype=np.uint8)
        D = 32
        N = (maxv + 1 + D - 1) // D
        c = np.resize(codes, N * D).reshape(N, D)
        packed = oleg.kvq_pack(c, bits)
        s = np.array([[0.37], [1.5], [0.01], [2.0], [0.9], [3.0], [0.2], [0.1]][:N], np.float16)
        z = np.array([[-1.1], [0.3], [2.0], [-0.5], [0.7], [0.0], [1.0], [-2.0]][:N], np.float16)
        got = oleg.dequantize_packed(packed, s, z, bits, D, N, D, "float32")
        exp = c.astype(np.float64) * s.astype(np.float64) + z.astype(np.float64)
        np.testing.assert_allclose(got, exp, rtol=2e-7, atol=1e-7)


def test_symmetric_branch_and_wrap():
    x = np.array([[-3.0, 1.0, 2.0, 0.5] * 8], np.float32)  # min is -absmax -> round(-7.5) = -8 -> code 255
    qt = oleg.kvq_quantize(x, 4, 32, symmetric=True)
    assert np.all(qt["zeros"] == 0)
    u = oleg.kvq_unpack(qt["data"], 4, 32)
    assert u[0] == 15  # -1 wrapped to 255, low nibble kept by the packer
    d = oleg.kvq_dequantize(qt)
    assert np.isclose(d[0, 0], (15 - 7) * (3.0 / 7.5))


def test_legacy_8bit_mse_bound():
    # tests/test_triton_ops.py:40-50 of the reference
    x = np.random.default_rng(42).standard_normal((32, 64)).astype(np.float16)
    qt = oleg.kvq_quantize(x, 8, 32)
    rec = oleg.dequantize_packed(qt["data"], qt["scales"], qt["zeros"], 8, 32, 32, 64)
    assert ((x.astype(np.float32) - rec.astype(np.float32)) ** 2).mean() < 0.01


def test_quantize_evict_matches_value_rule():
    rng = np.random.default_rng(6)
    keys = rng.standard_normal((20, 64)).astype(np.float16)
    mask = rng.random(20) < 0.5
    kp, ks, kz, *_ = oleg.quantize_evict(keys, keys, mask, 4, 64)
    # same arithmetic as quantize_values on one group per token
    qv = oaff.quantize_values(keys[mask][None], 4, packed=True)
    np.testing.assert_array_equal(kp, qv["codes"][0])
    np.testing.assert_array_equal(ks, qv["scale"][0, :, 0:1].reshape(-1, 1)[:, 0:1].reshape(ks.shape))


# ---------------------------------------------------------------- attention

def test_attention_fp32_vs_f64_bruteforce():
    rng = np.random.default_rng(7)
    q = rng.standard_normal((2, 4, 2, 8)).astype(np.float16)
    k = rng.standard_normal((2, 2, 11, 8)).astype(np.float16)
    v = rng.standard_normal((2, 2, 11, 8)).astype(np.float16)
    out, attn = oatt.attention_fp32(q, k, v)
    ro, ra = oatt.attention_f64_bruteforce(q, k, v)
    np.testing.assert_allclose(out, ro, atol=2e-6)
    np.testing.assert_allclose(attn, ra, atol=1e-6)
    np.testing.assert_allclose(attn.sum(-1), 1.0, atol=1e-6)


def test_mixed_attention_orders_and_broadcast():
    rng = np.random.default_rng(8)
    q = rng.standard_normal((1, 2, 1, 16)).astype(np.float16)
    kh = rng.standard_normal((1, 2, 5, 16)).astype(np.float16)
    vh = rng.standard_normal((1, 2, 5, 16)).astype(np.float16)
    kw = rng.standard_normal((7, 16)).astype(np.float16)
    vw = rng.standard_normal((7, 16)).astype(np.float16)
    o1, a1 = oatt.mixed_attention_fp32(q, kh, vh, kw, vw, hot_first=True)
    o2, a2 = oatt.mixed_attention_fp32(q, kh, vh, kw, vw, hot_first=False)
    np.testing.assert_allclose(o1, o2, atol=1e-6)  # softmax is order invariant
    np.testing.assert_allclose(a1[..., :5], a2[..., 7:], atol=1e-7)
    o3, _ = oatt.mixed_attention_fp32(q, kh, vh, None, None)
    r3, _ = oatt.attention_fp32(q, kh, vh)
    np.testing.assert_allclose(o3, r3)


# --------------------------------------------------------------- importance

def test_importance_float64_closed_form():
    rng = np.random.default_rng(9)
    a = rng.random((3, 4, 5, 20)).astype(np.float32)
    s = rng.random(20).astype(np.float32)
    exp = s.astype(np.float64) * 0.7 + a.astype(np.float64).mean(axis=(0, 1)).sum(axis=0)
    np.testing.assert_allclose(oimp.fused_importance_update(a, s, 0.7), exp, rtol=1e-6)
    # truncate / pad
    assert oimp.fused_importance_update(a, np.zeros(10, np.float32), 1.0).shape == (10,)
    p = oimp.fused_importance_update(a, np.ones(25, np.float32), 0.5)
    np.testing.assert_allclose(p[20:], 0.5)


def test_scorer_growth_and_window():
    s = oimp.scorer_update(None, np.ones((1, 1, 1, 4), np.float32), decay=0.5)
    s = oimp.scorer_update(s, np.ones((1, 1, 1, 6), np.float32), decay=0.5)
    np.testing.assert_allclose(s, [1.5, 1.5, 1.5, 1.5, 1.0, 1.0])
    w = oimp.scorer_update(None, np.ones((1, 1, 40, 10), np.float32), "observation_window", 1.0,
                           observation_window=8, pooling_kernel=3)
    np.testing.assert_allclose(w[1:-1], 8.0)
    np.testing.assert_allclose(w[[0, -1]], 8.0 * 2 / 3)


# ---------------------------------------------------------------- selection

def test_select_demote_bruteforce():
    import itertools
    rng = np.random.default_rng(10)
    for trial in range(20):
        hot_len, n, budget = 14, 4, 16
        imp = rng.random(hot_len).astype(np.float32)
        got = osel.select_demote_indices(imp, n, hot_len, budget)
        protect = set(range(4)) | set(range(hot_len - min(16, budget // 4), hot_len))
        best = min((c for c in itertools.combinations(range(hot_len), n) if not set(c) & protect),
                   key=lambda c: sum(imp[list(c)]))
        assert list(got) == sorted(best)
    assert list(osel.select_demote_indices(np.zeros(5), 3, 9, 16)) == [0, 1, 2]


def test_scorer_policy_strategies_closed_forms():
    """HEAVY_HITTER / RECENCY_WEIGHTED / FIFO / HYBRID of akv/importance.py:130-150,
    element by element in float64."""
    rng = np.random.default_rng(21)
    a = rng.random((2, 3, 4, 9)).astype(np.float32)
    s0 = rng.random(6).astype(np.float32)  # shorter than kv_len: grows with zeros
    imp = a.astype(np.float64).mean(axis=(0, 1)).sum(axis=0)
    grown = np.concatenate([s0, np.zeros(3)]).astype(np.float64)
    hh = oimp.scorer_update(s0, a, "heavy_hitter")
    np.testing.assert_allclose(hh, [max(g, i) for g, i in zip(grown, imp)], rtol=1e-6)
    np.testing.assert_allclose(oimp.scorer_update(s0, a, "recency_weighted"), [i / 8 for i in range(9)], atol=1e-7)
    np.testing.assert_array_equal(oimp.scorer_update(s0, a, "fifo"), np.arange(9, dtype=np.float32))
    hy = oimp.scorer_update(s0, a, "hybrid", decay=0.9, attention_weight=0.7, recency_weight=0.3)
    ema = [g * 0.9 + i for g, i in zip(grown, imp)]
    m = max(max(ema), 1e-10)
    np.testing.assert_allclose(hy, [0.7 * e / m + 0.3 * (k / 8) for k, e in enumerate(ema)], rtol=1e-6)
    # a longer score vector keeps the entries past kv_len untouched
    long = np.full(12, 5.0, np.float32)
    np.testing.assert_array_equal(oimp.scorer_update(long, a, "fifo")[9:], 5.0)


def test_observation_window_float64_loop():
    """Window sum of the last W queries then avg_pool1d(ks, stride 1, pad ks//2, include pad)."""
    rng = np.random.default_rng(22)
    for M, N, W, ks in ((10, 40, 4, 7), (3, 30, 8, 5), (6, 12, 6, 4), (5, 6, 2, 7)):
        a = rng.random((2, 2, M, N)).astype(np.float32)
        got = oimp.scorer_update(None, a, "observation_window", 1.0, observation_window=W, pooling_kernel=ks)
        avg = a.astype(np.float64).mean(axis=(0, 1))
        w = min(W, M)
        ki = [sum(avg[q, n] for q in range(M - w, M)) for n in range(N)]
        if ks > 1 and N > ks:
            pad = ks // 2
            ki = [sum(ki[j] for j in range(n - pad, n - pad + ks) if 0 <= j < N) / ks for n in range(N)]
        np.testing.assert_allclose(got, ki, rtol=1e-5, atol=1e-7)


def test_eviction_candidates_bruteforce():
    """get_eviction_candidates (akv/importance.py:245-300): the unprotected subset of
    the requested size with the smallest score sum, over every subset of tie-free
    tiny inputs; FIFO takes the oldest unprotected; too few evictable -> fewer."""
    import itertools
    from oracle import importance as oimp
    rng = np.random.default_rng(21)
    for seq_len in (6, 9, 12):
        for initial, recent in ((2, 1), (1, 3), (0, 0)):
            s = rng.permutation(seq_len).astype(np.float32) + rng.random(seq_len).astype(np.float32) * 0.1
            free = [i for i in range(seq_len) if i >= min(initial, seq_len) and i < seq_len - min(recent, seq_len)]
            for k in range(0, len(free) + 2):
                got = oimp.eviction_candidates(s, seq_len, k, "importance", initial, recent)
                kk = min(k, len(free))
                best = min(itertools.combinations(free, kk), key=lambda c: sum(float(s[i]) for i in c)) if kk else ()
                assert got.tolist() == sorted(best)
                fifo = oimp.eviction_candidates(None, seq_len, k, "fifo", initial, recent)
                assert fifo.tolist() == free[:kk]
    assert oimp.eviction_candidates(None, 10, 3, "importance").size == 0
