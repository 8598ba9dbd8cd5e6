"""ProductionCache (akv/production_cache.py) and PagedKVCache
(akv/packed_layout.py:283-443) on the device against the oracle.

The cache runs a prefill with attention weights, then one-token updates (weights
every 5th) on two layers; after each update the assembled ``get_kv`` view is
bit-exact with oracle/production.py (hot rows, the arenas' dequantized rows, the
migration schedule through the scorer's eviction candidates), and
``fused_attention`` -- one decode launch reading the packed arenas and the hot
buffer in place -- is within 2e-3 max-abs / 1e-3 mean-abs of the oracle's float32
attention over the same rows.  The attention weights are multiples of 2^-12 with
exact sums, so the device scorer's EMA is bit-exact with the oracle's and both
pick the same candidates (equal scores: lowest index first on both sides)."""
import numpy as np
import pytest
import torch

from gpu_util import announce, assert_close_attn, bits_equal, to_dev
from oracle.fp import F16, to_dtype
from oracle.production import ProductionCacheOracle

pytestmark = pytest.mark.gpu


def _rows(rng, H, N, D):
    return to_dtype((rng.standard_normal((H, N, D)) * 1.5).astype(np.float32), F16).astype(np.float32)


def _attn(rng, H, M, N):
    return (rng.integers(0, 64, (1, H, M, N)) / 4096.0).astype(np.float32)


def test_paged_pool_pages_tables_and_reset():
    from akv.packed_layout import PagedKVCache
    announce("PagedKVCache append / get_kv / pages / reset")
    rng = np.random.default_rng(0)
    H, D = 4, 64
    pc = PagedKVCache(num_layers=2, num_heads=H, head_dim=D, page_size=16, max_pages=8)
    a0 = [_rows(rng, H, n, D) for n in (20, 5)]
    a1 = [_rows(rng, H, n, D) for n in (16, 1)]
    for x in a0:
        pc.append(0, to_dev(x, torch.float16), to_dev(-x, torch.float16))
    for x in a1:
        pc.append(1, to_dev(x, torch.float16), to_dev(x, torch.float16))
    k0, v0 = pc.get_kv(0)
    bits_equal(k0, np.concatenate(a0, axis=1).astype(np.float16))
    bits_equal(v0, -np.concatenate(a0, axis=1).astype(np.float16))
    bits_equal(pc.get_kv(1)[0], np.concatenate(a1, axis=1).astype(np.float16))
    # pages come off the end of the free list: layer 0 takes 7 and 6, layer 1 then 5 and 4
    assert pc.get_page_table(0).tolist() == [7, 6] and pc.get_page_table(1).tolist() == [5, 4]
    assert pc.get_seq_length(0) == 25 and pc.get_seq_length(1) == 17
    assert pc.num_free_pages == 4
    assert pc.memory_usage_mb == pytest.approx(4 * H * 16 * D * 2 * 2 / 1e6)
    assert pc.get_page_table(0).dtype == torch.int32 and pc.get_page_table(0).device.type == "cuda"
    # appends that end inside a page, fill it exactly, and cross several pages
    more = [_rows(rng, H, n, D) for n in (7, 1, 39)]
    for x in more:
        pc.append(1, to_dev(x, torch.float16), to_dev(2 * x, torch.float16))
    full = np.concatenate(a1 + more, axis=1).astype(np.float16)
    k1, v1 = pc.get_kv(1)
    bits_equal(k1, full)
    bits_equal(v1, np.concatenate(a1 + [2 * x for x in more], axis=1).astype(np.float16))
    assert pc.get_page_table(1).tolist() == [5, 4, 3, 2] and pc.get_seq_length(1) == 64
    # freeing a page returns it to the end of the free list and zeroes it
    pc.free_page(2)
    assert pc.num_free_pages == 3 and float(pc.k_pool[2].abs().sum()) == 0.0 and pc.allocate_page() == 2
    pc.reset()
    assert pc.num_free_pages == 8 and pc.get_seq_length(0) == 0 and pc.get_kv(0)[0].shape == (H, 0, D)
    assert float(pc.k_pool.abs().sum()) == 0.0  # freed pages are zeroed
    # the reference's free-list order after a reset: layer 0's pages, then layer 1's
    pc.append(0, to_dev(_rows(rng, H, 1, D), torch.float16), to_dev(_rows(rng, H, 1, D), torch.float16))
    assert pc.get_page_table(0).tolist() == [2]
    pc.reset()
    with pytest.raises(RuntimeError, match="exhausted"):
        pc.append(0, torch.zeros(H, 16 * 8 + 1, D, dtype=torch.float16, device="cuda"),
                  torch.zeros(H, 16 * 8 + 1, D, dtype=torch.float16, device="cuda"))


def _config(bits, gs, **kw):
    from akv.production_cache import ProductionCacheConfig
    base = dict(num_layers=2, num_heads=4, head_dim=128, hot_budget=64, warm_budget=80, warm_bits=bits,
                group_size=gs, warm_quantizer="minmax", page_size=16, max_hot_pages=16,
                batch_migration_size=32, protect_initial=4, protect_recent=8, scoring_strategy="importance",
                importance_decay=0.3, device="cuda")
    base.update(kw)
    return ProductionCacheConfig(**base)


def _oracle(cfg):
    return ProductionCacheOracle(cfg.num_layers, cfg.num_heads, cfg.head_dim, cfg.hot_budget, cfg.warm_budget,
                                 cfg.warm_bits, cfg.group_size, migration_threshold=cfg.migration_threshold,
                                 batch_migration_size=cfg.batch_migration_size, decay=cfg.importance_decay,
                                 protect_initial=cfg.protect_initial, protect_recent=cfg.protect_recent,
                                 strategy=cfg.scoring_strategy)


def _check_view(cache, orc, layer, where):
    gk, gv = cache.get_kv(layer)
    ok, ov = orc.get_kv(layer)
    assert gk.shape == (1,) + ok.shape, where
    bits_equal(gk[0], ok.astype(np.float16))
    bits_equal(gv[0], ov.astype(np.float16))
    lay = cache._layers[layer]
    assert lay.hot_len == orc.hot_k[layer].shape[1] and lay.warm_len == orc.warm_k[layer].length, where


@pytest.mark.parametrize("bits,gs,strategy", [(4, 64, "importance"), (2, 32, "importance"), (8, 128, "importance"),
                                              (4, 64, "fifo")])
def test_update_view_and_fused_attention_match_oracle(bits, gs, strategy):
    from akv.production_cache import ProductionCache
    announce(f"ProductionCache bits={bits} group={gs} strategy={strategy}")
    cfg = _config(bits, gs, scoring_strategy=strategy)
    cache, orc = ProductionCache(cfg), _oracle(cfg)
    H, D = cfg.num_heads, cfg.head_dim
    rng = np.random.default_rng(bits * 7 + gs)
    for t in range(-1, 60):
        for layer in range(cfg.num_layers):
            n_new = 150 if t < 0 else 1
            k, v = _rows(rng, H, n_new, D), _rows(rng, H, n_new, D)
            n_keys = cache._layers[layer].hot_len + cache._layers[layer].warm_len + n_new
            attn = _attn(rng, H, n_new, n_keys) if (t < 0 or t % 5 == 0) else None
            ret = cache.update(to_dev(k[None], torch.float16), to_dev(v[None], torch.float16), layer,
                               to_dev(attn) if attn is not None else None)
            orc.update(k, v, layer, attn)
            where = f"step {t} layer {layer}"
            _check_view(cache, orc, layer, where)
            bits_equal(ret[0][0], orc.get_kv(layer)[0].astype(np.float16))
            if t < 0 or t % 10 == 3:
                q = rng.standard_normal((2, H, 1, D)).astype(np.float32)
                assert_close_attn(cache.fused_attention(to_dev(q), layer), orc.attention(q, layer))
    assert orc.migrations > 0 and orc.warm_k[0].dropped > 0  # demotions and arena overflow both ran
    mem = cache.memory_usage()
    assert mem["migrations"] == orc.migrations and mem["total_demoted"] == orc.total_demoted
    assert mem["decode_count"] == orc.decode_count and mem["num_layers"] == 2
    assert cache.get_seq_length(1) == 150 + 60 and len(cache) == 2
    # multi-row queries (M = 4) through the same launch
    q = rng.standard_normal((1, H, 4, D)).astype(np.float32)
    assert_close_attn(cache.fused_attention(to_dev(q, torch.float16), 0), orc.attention(q, 0))
    # the sm_scale keyword of the vLLM backend's call
    assert_close_attn(cache.fused_attention(to_dev(q), 1, sm_scale=0.05), orc.attention(q, 1, sm_scale=0.05))
    cache.reset()
    assert cache._layers[0].hot_len == 0 and cache._layers[0].warm_len == 0 and cache.get_seq_length(0) == 0


def test_hot_only_and_errors():
    from akv.production_cache import ProductionCache, ProductionLayerCache
    announce("ProductionCache hot-only attention / refused configurations")
    cfg = _config(4, 64, hot_budget=1024)
    cache, orc = ProductionCache(cfg), _oracle(cfg)
    rng = np.random.default_rng(4)
    k, v = _rows(rng, 4, 40, 128), _rows(rng, 4, 40, 128)
    cache.update(to_dev(k, torch.float16), to_dev(v, torch.float16), 0)  # (H, N, D) input
    orc.update(k, v, 0)
    _check_view(cache, orc, 0, "hot only")
    q = rng.standard_normal((1, 4, 1, 128)).astype(np.float32)
    assert_close_attn(cache.fused_attention(to_dev(q), 0), orc.attention(q, 0))
    with pytest.raises(RuntimeError, match="empty"):
        cache.fused_attention(to_dev(q), 1)
    with pytest.raises(NotImplementedError, match="TurboQuant"):
        ProductionLayerCache(_config(3, 64, warm_quantizer="turbo"), 0)
    with pytest.raises(ValueError, match="2, 4 or 8"):
        ProductionLayerCache(_config(3, 64), 0)


def test_fused_attention_counter_region_shrinks_then_grows():
    """Query lengths 32 -> 1 -> 32 on 32 heads: the split-counter region of the layer's
    reused workspace halves, the short call writes partials over its tail, and the next
    long call must clear it again (each output checked against the oracle)."""
    from akv.production_cache import ProductionCache
    announce("ProductionCache fused_attention M=32,1,32 (workspace counter region)")
    cfg = _config(4, 64, num_layers=1, num_heads=32, hot_budget=48, warm_budget=256)
    cache, orc = ProductionCache(cfg), _oracle(cfg)
    rng = np.random.default_rng(11)
    H, D = cfg.num_heads, cfg.head_dim
    k, v = _rows(rng, H, 200, D), _rows(rng, H, 200, D)
    attn = _attn(rng, H, 200, 200)
    cache.update(to_dev(k[None], torch.float16), to_dev(v[None], torch.float16), 0, to_dev(attn))
    orc.update(k, v, 0, attn)
    _check_view(cache, orc, 0, "prefill")
    assert cache._layers[0].warm_len > 0
    for M in (32, 1, 32, 5, 32):
        q = rng.standard_normal((1, H, M, D)).astype(np.float32)
        assert_close_attn(cache.fused_attention(to_dev(q), 0), orc.attention(q, 0))


def test_batched_queries_one_launch_and_hot_accounting():
    """fused_attention with B = 3 batch elements and M = 2 queries each (one decode launch,
    rows b * M + m of a head) against the oracle; the hot tier's page accounting follows
    ceil(hot_len / page_size) pages, and a hot tier past its pages raises."""
    from akv.production_cache import ProductionCache
    announce("ProductionCache fused_attention B=3 M=2, hot accounting, exhaustion")
    cfg = _config(4, 64, num_layers=1, hot_budget=40, warm_budget=128, max_hot_pages=8)
    cache, orc = ProductionCache(cfg), _oracle(cfg)
    rng = np.random.default_rng(21)
    H, D = cfg.num_heads, cfg.head_dim
    for n in (70, 1, 1, 9):
        k, v = _rows(rng, H, n, D), _rows(rng, H, n, D)
        attn = _attn(rng, H, n, cache._layers[0].hot_len + cache._layers[0].warm_len + n)
        cache.update(to_dev(k[None], torch.float16), to_dev(v[None], torch.float16), 0, to_dev(attn))
        orc.update(k, v, 0, attn)
        _check_view(cache, orc, 0, f"append {n}")
        q = rng.standard_normal((3, H, 2, D)).astype(np.float32)
        assert_close_attn(cache.fused_attention(to_dev(q), 0), orc.attention(q, 0))
    lay = cache._layers[0]
    pages = -(-lay.hot_len // cfg.page_size)
    assert lay.memory_usage()["hot_mb"] == pytest.approx(pages * H * cfg.page_size * D * 4 / 1e6)
    with pytest.raises(RuntimeError, match="exhausted"):
        lay.append_hot(torch.zeros(H, 8 * 16 - lay.hot_len + 1, D, dtype=torch.float16, device="cuda"),
                       torch.zeros(H, 8 * 16 - lay.hot_len + 1, D, dtype=torch.float16, device="cuda"))


def test_layer_cache_accessors_and_demotion():
    """ProductionLayerCache's own methods (akv/production_cache.py:182-320): append_hot /
    get_hot_kv return the appended rows; demote_to_warm quantizes the given rows into the
    arenas (bit-exact with the oracle's arena quantizer), drops the demoted positions from
    the hot tier keeping the others in order, and get_warm_fp16 / get_warm_packed expose
    the arenas (dequantized / as stored)."""
    from akv.production_cache import ProductionLayerCache
    from oracle import legacy as olg
    announce("ProductionLayerCache append / demote / warm views")
    cfg = _config(4, 64)
    layer = ProductionLayerCache(cfg, 0)
    assert layer.hot_capacity == cfg.page_size * cfg.max_hot_pages
    assert layer.get_warm_fp16() == (None, None)
    assert layer.get_warm_packed() == (None,) * 6
    rng = np.random.default_rng(21)
    k, v = _rows(rng, 4, 30, 128), _rows(rng, 4, 30, 128)
    layer.append_hot(to_dev(k, torch.float16), to_dev(v, torch.float16))
    hk, hv = layer.get_hot_kv()
    bits_equal(hk, k.astype(np.float16))
    bits_equal(hv, v.astype(np.float16))
    idx = np.array([0, 3, 4, 17, 29])
    layer.demote_to_warm(to_dev(idx, torch.long), to_dev(k[:, idx], torch.float16), to_dev(v[:, idx], torch.float16))
    keep = np.setdiff1d(np.arange(30), idx)
    hk, hv = layer.get_hot_kv()
    bits_equal(hk, k[:, keep].astype(np.float16))
    bits_equal(hv, v[:, keep].astype(np.float16))
    pk, sk, zk = olg.arena_quantize(k[:, idx], 4, 64)
    pv, sv, zv = olg.arena_quantize(v[:, idx], 4, 64)
    got = layer.get_warm_packed()
    for g, r in zip(got, (pk, sk, zk, pv, sv, zv)):
        bits_equal(g, r)
    wk, wv = layer.get_warm_fp16()
    bits_equal(wk, olg.arena_dequantize(pk, sk, zk, 4, 64, 128))
    bits_equal(wv, olg.arena_dequantize(pv, sv, zv, 4, 64, 128))
    with pytest.raises(RuntimeError, match="Page pool exhausted"):
        big = to_dev(_rows(rng, 4, layer.hot_capacity, 128), torch.float16)
        layer.append_hot(big, big)
