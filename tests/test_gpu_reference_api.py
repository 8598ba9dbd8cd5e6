"""The reference's public ops (akv.triton_ops / triton_kernels / fused_attention)
on the device: the reference tests (tests/test_triton_ops.py) restated, plus
parity with the oracle on the same inputs."""
import math

import numpy as np
import pytest
import torch

from gpu_util import announce, assert_close_attn, to_dev
from oracle import attention as oatt
from oracle import importance as oimp
from oracle import legacy as oleg

pytestmark = pytest.mark.gpu


@pytest.fixture
def kv_data():
    rng = np.random.default_rng(42)
    B, H, N, D = 1, 4, 64, 64
    q = rng.standard_normal((B, H, 1, D)).astype(np.float16)
    k = rng.standard_normal((B, H, N, D)).astype(np.float16)
    v = rng.standard_normal((B, H, N, D)).astype(np.float16)
    return q, k, v


def _legacy(x, bits=4, gs=32):
    qt = oleg.kvq_quantize(x, bits, gs)
    G = qt["scales"].shape[-1]
    return qt, qt["scales"].reshape(-1, G), qt["zeros"].reshape(-1, G)


def test_fused_quantized_attention_shape_and_parity(kv_data):
    import akv
    announce("fused_quantized_attention")
    q, k, v = kv_data
    kq, ks, kz = _legacy(k)
    vq, vs, vz = _legacy(v)
    out = akv.fused_quantized_attention(to_dev(q), to_dev(kq["data"]), to_dev(ks), to_dev(kz),
                                        to_dev(vq["data"]), to_dev(vs), to_dev(vz), bits=4, group_size=32)
    assert out.shape == q.shape
    N = ks.shape[0]
    kd = oleg.dequantize_packed(kq["data"], ks, kz, 4, 32, N, 64)
    vd = oleg.dequantize_packed(vq["data"], vs, vz, 4, 32, N, 64)
    ref, _ = oatt.mixed_attention_fp32(q, np.zeros((1, 4, 0, 64), np.float16), np.zeros((1, 4, 0, 64), np.float16),
                                       kd, vd, hot_first=True, return_weights=False)
    assert_close_attn(out, ref)


@pytest.mark.parametrize("M", [1, 4])
def test_fused_mixed_precision_attention(kv_data, M):
    import akv
    announce(f"fused_mixed_precision_attention M={M}")
    q, k, v = kv_data
    if M > 1:
        q = np.random.default_rng(1).standard_normal((1, 4, M, 64)).astype(np.float16)
    n_hot = 32
    kh, vh = k[:, :, :n_hot], v[:, :, :n_hot]
    kw = k[:, :, n_hot:].reshape(-1, 64)[None, None]
    vw = v[:, :, n_hot:].reshape(-1, 64)[None, None]
    kq, ks, kz = _legacy(kw)
    vq, vs, vz = _legacy(vw)
    out, attn = akv.fused_mixed_precision_attention(
        to_dev(q), to_dev(kh), to_dev(vh), to_dev(kq["data"]), to_dev(ks), to_dev(kz),
        to_dev(vq["data"]), to_dev(vs), to_dev(vz), bits=4, group_size=32)
    assert out.shape == q.shape
    assert attn.dtype == torch.float32 and attn.shape == (1, 4, M, n_hot + ks.shape[0])
    sums = attn.sum(dim=-1)
    assert torch.allclose(sums, torch.ones_like(sums), atol=1e-3)
    Nw = ks.shape[0]
    kd = oleg.dequantize_packed(kq["data"], ks, kz, 4, 32, Nw, 64)
    vd = oleg.dequantize_packed(vq["data"], vs, vz, 4, 32, Nw, 64)
    ref, ref_attn = oatt.mixed_attention_fp32(q, kh, vh, kd, vd, hot_first=True)
    assert_close_attn(out, ref)
    np.testing.assert_allclose(attn.cpu().numpy(), ref_attn, atol=2e-6, rtol=1e-4)


def test_fused_decode_attention_legacy_parity():
    import akv
    announce("fused_decode_attention legacy warm")
    rng = np.random.default_rng(3)
    B, H, D, Nh, Nw = 2, 4, 128, 40, 300
    q = rng.standard_normal((B, H, 1, D)).astype(np.float16)
    kh = rng.standard_normal((B, H, Nh, D)).astype(np.float16)
    vh = rng.standard_normal((B, H, Nh, D)).astype(np.float16)
    for bits, gs in ((4, 128), (2, 32), (8, 64)):
        kw = rng.standard_normal((Nw, D)).astype(np.float16)
        vw = rng.standard_normal((Nw, D)).astype(np.float16)
        kq, ks, kz = _legacy(kw, bits, gs)
        vq, vs, vz = _legacy(vw, bits, gs)
        out = akv.fused_decode_attention(to_dev(q), to_dev(kh), to_dev(vh), to_dev(kq["data"]), to_dev(ks),
                                         to_dev(kz), to_dev(vq["data"]), to_dev(vs), to_dev(vz), bits=bits,
                                         group_size=gs)
        kd = oleg.dequantize_packed(kq["data"], ks, kz, bits, gs, Nw, D)
        vd = oleg.dequantize_packed(vq["data"], vs, vz, bits, gs, Nw, D)
        ref, _ = oatt.mixed_attention_fp32(q, kh, vh, kd, vd, hot_first=True, return_weights=False)
        assert_close_attn(out, ref)


def test_fused_decode_attention_errors_and_hot_only():
    import akv
    announce("fused_decode_attention errors / hot only")
    rng = np.random.default_rng(4)
    q = to_dev(rng.standard_normal((1, 2, 2, 64)).astype(np.float16))
    kh = rng.standard_normal((1, 2, 16, 64)).astype(np.float16)
    with pytest.raises(AssertionError):
        akv.fused_decode_attention(q, to_dev(kh), to_dev(kh))
    q1 = rng.standard_normal((1, 2, 1, 64)).astype(np.float16)
    out = akv.fused_decode_attention(to_dev(q1), to_dev(kh), to_dev(kh))
    ref, _ = oatt.attention_fp32(q1, kh, kh, return_weights=False)
    assert_close_attn(out, ref)
    z = to_dev(np.zeros((16, 2), np.float16))
    with pytest.raises(ValueError):
        akv.fused_decode_attention(to_dev(q1), to_dev(kh), to_dev(kh), to_dev(np.zeros(16 * 48, np.uint8)), z, z,
                                   to_dev(np.zeros(16 * 48, np.uint8)), z, z, bits=3, group_size=32)


def test_int4_per_head_ops():
    import akv
    announce("fused_int4_decode_attention / mixed_precision_decode_attention")
    rng = np.random.default_rng(5)
    B, H, N, D, gs = 2, 4, 200, 128, 32
    q = rng.standard_normal((B, H, 1, D)).astype(np.float16)
    kc = rng.integers(0, 256, (H, N, D // 2), dtype=np.uint8)
    vc = rng.integers(0, 256, (H, N, D // 2), dtype=np.uint8)
    ks = (rng.random((H, N, D // gs)) * 0.3 + 0.01).astype(np.float16)
    kz = (rng.standard_normal((H, N, D // gs)) - 1).astype(np.float16)
    vs = (rng.random((H, N, D // gs)) * 0.3 + 0.01).astype(np.float16)
    vz = (rng.standard_normal((H, N, D // gs)) - 1).astype(np.float16)
    out = akv.fused_int4_decode_attention(to_dev(q), to_dev(kc), to_dev(ks), to_dev(kz), to_dev(vc), to_dev(vs),
                                          to_dev(vz), group_size=gs)
    kd = oleg.dequant_int4_tile(kc, ks, kz, D, gs)
    vd = oleg.dequant_int4_tile(vc, vs, vz, D, gs)
    ref, _ = oatt.attention_fp32(q, np.broadcast_to(kd[None], (B, H, N, D)), np.broadcast_to(vd[None], (B, H, N, D)),
                                 return_weights=False)
    assert_close_attn(out, ref)
    kh = rng.standard_normal((B, H, 24, D)).astype(np.float16)
    vh = rng.standard_normal((B, H, 24, D)).astype(np.float16)
    out2 = akv.mixed_precision_decode_attention(to_dev(q), to_dev(kh), to_dev(vh), to_dev(kc), to_dev(ks),
                                                to_dev(kz), to_dev(vc), to_dev(vs), to_dev(vz), group_size=gs)
    ref2, _ = oatt.mixed_attention_fp32(q, kh, vh, np.broadcast_to(kd[None], (B, H, N, D)),
                                        np.broadcast_to(vd[None], (B, H, N, D)), hot_first=True, return_weights=False)
    assert_close_attn(out2, ref2)


def test_fused_importance_update_kats():
    import akv
    announce("fused_importance_update")
    rng = np.random.default_rng(42)
    attn = rng.random((1, 4, 1, 64)).astype(np.float32)
    attn /= attn.sum(-1, keepdims=True)
    scores = to_dev(np.zeros(64, np.float32))
    updated = akv.fused_importance_update(to_dev(attn), scores, decay=0.95)
    assert updated.shape == (64,) and updated.sum() > 0
    assert updated.data_ptr() == scores.data_ptr()  # in place
    s1 = to_dev(np.ones(32, np.float32))
    u1 = akv.fused_importance_update(to_dev(np.zeros((1, 1, 1, 32), np.float32)), s1, decay=0.5)
    assert torch.allclose(u1, torch.ones(32, device="cuda") * 0.5, atol=1e-5)
    # M > 1 sums over queries; pad / truncate to len(scores)
    a = rng.random((2, 3, 5, 40)).astype(np.float32)
    for n in (40, 30, 55):
        s0 = rng.random(n).astype(np.float32)
        got = akv.fused_importance_update(to_dev(a), to_dev(s0.copy()), decay=0.8)
        np.testing.assert_allclose(got.cpu().numpy(), oimp.fused_importance_update(a, s0, 0.8), rtol=1e-6, atol=1e-7)
    # non-dyadic weights over many (batch, head) rows and 3 queries (16 waves per key tile):
    # the per-query mean, then the sum over queries, as the reference associates it
    a = rng.random((8, 12, 3, 300)).astype(np.float32)
    a /= a.sum(-1, keepdims=True)
    s0 = rng.random(300).astype(np.float32)
    got = akv.fused_importance_update(to_dev(a), to_dev(s0.copy()), decay=0.9)
    np.testing.assert_allclose(got.cpu().numpy(), oimp.fused_importance_update(a, s0, 0.9), rtol=1e-6, atol=1e-8)


def test_importance_scorer_accumulate():
    import akv
    announce("ImportanceScorer")
    sc = akv.ImportanceScorer(akv.ImportanceConfig(strategy=akv.ScoringStrategy.ATTENTION_ACCUMULATION,
                                                   decay_factor=0.9))
    rng = np.random.default_rng(0)
    ref = None
    for n in (10, 10, 14, 12):
        a = rng.random((1, 2, 1, n)).astype(np.float32)
        sc.update(to_dev(a), layer_idx=3)
        ref = oimp.scorer_update(ref, a, "attention_accumulation", 0.9)
    np.testing.assert_allclose(sc.get_scores(3).cpu().numpy(), ref, rtol=1e-6, atol=1e-7)
    assert sc.step_count == 4


def test_compat_kvquantizer_decode():
    import akv
    from akv.fused_attention import fused_decode_attention as compat
    announce("compat fused_decode_attention(KVQuantizer)")
    rng = np.random.default_rng(6)
    q = rng.standard_normal((2, 3, 1, 64)).astype(np.float16)
    k = rng.standard_normal((2, 3, 50, 64)).astype(np.float16)
    v = rng.standard_normal((2, 3, 50, 64)).astype(np.float16)
    qz = akv.KVQuantizer(akv.QuantConfig(bits=4, group_size=32))
    out = compat(to_dev(q), qz.quantize(to_dev(k)), qz.quantize(to_dev(v)), qz)
    kd = oleg.kvq_dequantize(oleg.kvq_quantize(k, 4, 32))
    vd = oleg.kvq_dequantize(oleg.kvq_quantize(v, 4, 32))
    ref, _ = oatt.attention_fp32(q, kd, vd, return_weights=False)
    assert_close_attn(out, ref)
