"""The KIVI baselines (akv/baselines.py) on the device against oracle/kivi.py:
the quantizer's packed codes and fp32 scales / zeros and the dequant bit-exact; the
views ``KIVICache.update`` and ``KIVIFusedCache.update`` return bit-exact after
every update (prefill, decode steps, chunks; several layers; batch > 1); memory
accounting, reset, ``create_baseline``; the reference's KIVI tests
(tests/test_kivi_fused.py) restated at head_dim 64; and
``KIVIFusedCache.fused_attention`` within 2e-3 / 1e-3 of the oracle's fp32 attention
over the same view."""
import numpy as np
import pytest
import torch

from gpu_util import announce, assert_close_attn, bits_equal, to_dev
from oracle import attention as oatt
from oracle import legacy as oleg
from oracle.kivi import KIVIOracle, kivi_dequantize, kivi_quantize

pytestmark = pytest.mark.gpu


def _kv(rng, B, H, n, D, scale=1.0):
    k = (rng.standard_normal((B, H, n, D)) * scale).astype(np.float16).astype(np.float32)
    v = (rng.standard_normal((B, H, n, D)) * scale).astype(np.float16).astype(np.float32)
    return k, v


@pytest.mark.parametrize("bits,gs,D", [(2, 128, 128), (4, 32, 128), (8, 64, 64), (2, 128, 64), (4, 64, 64)])
def test_quantize_and_dequant_bit_exact(bits, gs, D):
    from akv.baselines import dequantize_rows, quantize_rows
    announce(f"KIVI quantize bits={bits} gs={gs} D={D}")
    rng = np.random.default_rng(bits * 10 + gs + D)
    x, _ = _kv(rng, 2, 3, 37, D, scale=2.0)
    x[0, 1, 5] = 0.5  # a constant token: scale clamped at 1e-10
    codes, sc, ze = quantize_rows(to_dev(x, torch.float16), bits, gs)
    oc, osc, oze = kivi_quantize(x, bits, gs)
    bits_equal(codes.reshape(2 * 3 * 37, -1), oleg.arena_pack(oc.reshape(2 * 3 * 37, -1), bits))
    bits_equal(sc.reshape(-1, osc.shape[-1]), osc)
    bits_equal(ze.reshape(-1, oze.shape[-1]), oze)
    deq = dequantize_rows(codes, sc, ze, bits, gs, D)
    bits_equal(deq.reshape(2, 3, 37, D), kivi_dequantize(oc, osc, oze, x.shape))


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("bits,gs,res", [(2, 128, 16), (4, 32, 8)])
def test_update_views_match_oracle(fused, bits, gs, res):
    from akv.baselines import KIVICache, KIVIConfig, KIVIFusedCache, KIVIFusedConfig
    announce(f"KIVI update fused={fused} bits={bits} gs={gs} residual={res}")
    cfg = dict(key_bits=bits, value_bits=bits, group_size=gs, residual_length=res)
    cache = KIVIFusedCache(KIVIFusedConfig(**cfg)) if fused else KIVICache(KIVIConfig(**cfg))
    orc = KIVIOracle(bits, bits, gs, res, fused=fused)
    rng = np.random.default_rng(bits + res + int(fused))
    B, H, D = 2, 4, 128
    for step, n in enumerate([40, 1, 1, 5, 1, 30, 1, 1, 1, 17] + [1] * 12):
        for layer in range(2):
            k, v = _kv(rng, B, H, n, D)
            gk, gv = cache.update(to_dev(k, torch.float16), to_dev(v, torch.float16), layer)
            ok, ov = orc.update(k, v, layer)
            bits_equal(gk, ok.astype(np.float16))
            bits_equal(gv, ov.astype(np.float16))
            if layer in orc.q_k:
                c, s, z = orc.quantized_rows(layer)
                t = cache._quant_keys[layer]
                bits_equal(t.codes[:, : t.n], oleg.arena_pack(c, bits))
                bits_equal(t.sc[:, : t.n], s)
                bits_equal(t["zeros"], z.reshape(-1, z.shape[-1]))
    assert cache.get_seq_length(1) == orc.seq[1]
    assert cache.memory_bytes() == orc.memory_bytes(packed=True)
    cache.reset()
    assert cache.get_seq_length(0) == 0 and len(cache._quant_keys) == 0


def test_reference_kivi_tests_restated():
    """tests/test_kivi_fused.py with head_dim 64 and groups of 32 (this build's quantizer
    shapes)."""
    from akv.baselines import KIVICache, KIVIConfig, KIVIFusedCache, KIVIFusedConfig, create_baseline
    announce("KIVI reference tests restated")
    rng = np.random.default_rng(0)
    naive = KIVICache(KIVIConfig(key_bits=4, value_bits=4, group_size=32, residual_length=8))
    fused = KIVIFusedCache(KIVIFusedConfig(key_bits=4, value_bits=4, group_size=32, residual_length=8))
    for _ in range(20):
        k, v = _kv(rng, 1, 4, 1, 64)
        nk, _ = naive.update(to_dev(k), to_dev(v), layer_idx=0)
        fk, _ = fused.update(to_dev(k), to_dev(v), layer_idx=0)
    assert nk.shape == fk.shape and float((nk - fk).abs().max()) < 0.5
    naive = KIVICache(KIVIConfig(key_bits=2, value_bits=2, group_size=32, residual_length=4))
    fused = KIVIFusedCache(KIVIFusedConfig(key_bits=2, value_bits=2, group_size=32, residual_length=4))
    for _ in range(32):
        k, v = _kv(rng, 1, 4, 1, 64)
        naive.update(to_dev(k), to_dev(v), layer_idx=0)
        fused.update(to_dev(k), to_dev(v), layer_idx=0)
    a, b = naive.memory_bytes(), fused.memory_bytes()
    assert a > 0 and b > 0 and max(a, b) / min(a, b) < 10.0
    fused = KIVIFusedCache(KIVIFusedConfig(key_bits=4, value_bits=4, group_size=32, residual_length=4))
    sizes = []
    for _ in range(16):
        k, v = _kv(rng, 1, 4, 1, 64)
        fused.update(to_dev(k), to_dev(v), layer_idx=0)
        if 0 in fused._quant_keys:
            sizes.append(fused._quant_keys[0]["data"].shape[0])
    assert len(fused._dequant_keys_cache) > 0
    assert sizes and all(y >= x for x, y in zip(sizes, sizes[1:]))
    fused.reset()
    assert len(fused._dequant_keys_cache) == 0 and len(fused._quant_keys) == 0
    for alias in ("kivi_fused", "kivi-fused", "kivifused", "fused_kivi"):
        assert isinstance(create_baseline(alias, key_bits=4, value_bits=4, group_size=32, residual_length=4),
                          KIVIFusedCache)
    assert isinstance(create_baseline("kivi"), KIVICache)
    with pytest.raises(NotImplementedError):
        create_baseline("h2o")
    with pytest.raises(ValueError):
        create_baseline("nope")


@pytest.mark.parametrize("B,H,Hq,M,bits,gs", [(1, 8, 8, 1, 2, 128), (2, 4, 8, 1, 4, 64), (2, 2, 12, 2, 2, 32)])
def test_fused_attention_matches_oracle(B, H, Hq, M, bits, gs):
    from akv.baselines import KIVIFusedCache, KIVIFusedConfig
    announce(f"KIVI fused_attention B={B} H={H} Hq={Hq} M={M} bits={bits} gs={gs}")
    cache = KIVIFusedCache(KIVIFusedConfig(key_bits=bits, value_bits=bits, group_size=gs, residual_length=32))
    orc = KIVIOracle(bits, bits, gs, 32, fused=True)
    rng = np.random.default_rng(B * 100 + H + bits)
    D = 128
    for n in (300, 1, 1, 7, 1, 1):
        k, v = _kv(rng, B, H, n, D)
        cache.update(to_dev(k, torch.float16), to_dev(v, torch.float16), 0)
        ok, ov = orc.update(k, v, 0)
        q = rng.standard_normal((B, Hq, M, D)).astype(np.float32)
        ref, _ = oatt.attention_fp32(q.astype(np.float16), ok.astype(np.float16), ov.astype(np.float16),
                                     return_weights=False)
        assert_close_attn(cache.fused_attention(to_dev(q), 0), ref)
    ref, _ = oatt.attention_fp32(q.astype(np.float16), ok.astype(np.float16), ov.astype(np.float16), sm_scale=0.04,
                                 return_weights=False)
    assert_close_attn(cache.fused_attention(to_dev(q), 0, sm_scale=0.04), ref)


def test_fused_attention_counter_region_shrinks_then_grows():
    """One workspace per device serves every call: query lengths 32 -> 1 -> 32 on 16
    heads halve and then double its split-counter region; each output is checked."""
    from akv.baselines import KIVIFusedCache, KIVIFusedConfig
    announce("KIVI fused_attention M=32,1,32 (shared workspace counter region)")
    cache = KIVIFusedCache(KIVIFusedConfig(key_bits=2, value_bits=2, group_size=128, residual_length=32))
    orc = KIVIOracle(2, 2, 128, 32, fused=True)
    rng = np.random.default_rng(5)
    B, H, D = 2, 16, 128
    k, v = _kv(rng, B, H, 700, D)
    cache.update(to_dev(k, torch.float16), to_dev(v, torch.float16), 0)
    ok, ov = orc.update(k, v, 0)
    for M in (32, 1, 32, 3, 32):
        q = rng.standard_normal((B, H, M, D)).astype(np.float32)
        ref, _ = oatt.attention_fp32(q.astype(np.float16), ok.astype(np.float16), ov.astype(np.float16),
                                     return_weights=False)
        assert_close_attn(cache.fused_attention(to_dev(q), 0), ref)
