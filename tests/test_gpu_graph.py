"""Prepared decode calls captured in a HIP graph: every replay equals the eager call.

The decode workspace holds the split-merge arrival counts; each call must leave them
at zero, or the next replay would merge the wrong partials.  Each replay is followed
by eager work of its own and a synchronization, and is checked against an eager call
on identical inputs.  The two agree to the last few bits only: a workgroup hands its
units to its waves from a counter, so the order of the fp32 sums varies between calls."""
import numpy as np
import pytest
import torch

from gpu_util import announce, assert_close_attn, to_dev, warm_from_oracle
from oracle import affine as oaff
from oracle import attention as oatt

pytestmark = pytest.mark.gpu


def _inputs(B, Hq, Hkv, Nh, Nw, bk, bv, seed):
    from akv import workloads as wl
    shape = wl.DecodeShape("g", B, Hq, Hkv, 128, Nh, Nw, bk, bv, block_t=32, group_v=32)
    k, v = wl.make_kv(shape, layer=seed)
    q = wl.make_q(shape, layer=seed)
    (kw, vw), (kh, vh) = wl.split_hot_warm(k, v, Nh)
    w = oaff.quantize_kv_blocked(kw.numpy(), vw.numpy(), bk, bv, 32, 32, 0.0)
    return q.numpy(), kh.numpy(), vh.numpy(), w


@pytest.mark.parametrize("importance", [False, True])
def test_decode_call_graph_replays(importance):
    from akv.warm_tier import DecodeCall
    announce(f"decode graph replays importance={importance}")
    q, kh, vh, w = _inputs(2, 12, 2, 256, 2048, 3, 3, seed=21)
    N = kh.shape[2] + w["N"]
    s0 = np.random.default_rng(5).random(N).astype(np.float32)
    dq, dkh, dvh, wt = to_dev(q), to_dev(kh), to_dev(vh), warm_from_oracle(w)
    s_eager = to_dev(s0) if importance else None
    s_graph = to_dev(s0) if importance else None
    eager = DecodeCall(dq, dkh, dvh, wt, scores=s_eager, decay=0.9)
    graphed = DecodeCall(dq, dkh, dvh, wt, scores=s_graph, decay=0.9)
    torch.cuda.synchronize()

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        graphed()
    torch.cuda.synchronize()

    kd, vd = oaff.dequant_kv_blocked(w)
    ref, _ = oatt.mixed_attention_fp32(q, kh, vh, kd, vd, hot_first=False, return_weights=False)
    scratch = torch.zeros(1 << 20, device="cuda")
    for r in range(4):
        g.replay()
        eager()
        scratch.add_(1.0)  # eager work of the program's own between replays
        torch.cuda.synchronize()
        torch.testing.assert_close(graphed.out, eager.out, atol=2e-4, rtol=2e-3,
                                   msg=f"replay {r}: output differs from the eager call")
        if importance:
            torch.testing.assert_close(s_graph, s_eager, atol=1e-6, rtol=1e-5,
                                       msg=f"replay {r}: scores differ from the eager call")
        # the split-merge arrival counts are back at zero (the workspace starts with them)
        assert int(graphed.workspace[:64].int().sum()) == 0, f"replay {r}: counts not returned to zero"
    assert_close_attn(graphed.out, ref)


def test_two_layers_in_one_graph():
    """Two prepared calls with their own workspaces, captured back to back."""
    from akv.warm_tier import DecodeCall
    announce("decode graph two layers")
    cases = [_inputs(1, 12, 2, 128, 1024, 4, 2, seed=31), _inputs(1, 12, 2, 96, 1000, 2, 4, seed=32)]
    calls, refs = [], []
    for q, kh, vh, w in cases:
        calls.append(DecodeCall(to_dev(q), to_dev(kh), to_dev(vh), warm_from_oracle(w)))
        kd, vd = oaff.dequant_kv_blocked(w)
        refs.append(oatt.mixed_attention_fp32(q, kh, vh, kd, vd, hot_first=False, return_weights=False)[0])
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for c in calls:
            c()
    for _ in range(3):
        for c in calls:
            c.out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for c, ref in zip(calls, refs):
            assert_close_attn(c.out, ref)


def _graph_matches_eager(calls, n_replays=4):
    """Capture `calls` (a list of zero-argument callables returning tensors) in one graph;
    after every replay, with eager work between, each output equals an eager call's."""
    eager_first = [c() for c in calls]
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = [c() for c in calls]
    torch.cuda.synchronize()
    scratch = torch.zeros(1 << 20, device="cuda")
    for r in range(n_replays):
        g.replay()
        eager = [c() for c in calls]
        scratch.add_(1.0)
        torch.cuda.synchronize()
        for i, (o, e) in enumerate(zip(outs, eager)):
            torch.testing.assert_close(o, e, atol=2e-4, rtol=2e-3, msg=f"replay {r}, call {i}")
    return outs, eager_first


def test_production_fused_attention_in_a_graph():
    """ProductionCache.fused_attention over two layers captured once: the layers' decode
    workspaces are reused, so the graph holds only the decode launches."""
    from akv.production_cache import ProductionCache, ProductionCacheConfig
    from oracle.production import ProductionCacheOracle
    announce("ProductionCache.fused_attention graph replays")
    cfg = ProductionCacheConfig(num_layers=2, num_heads=8, head_dim=128, hot_budget=64, warm_budget=512, warm_bits=4,
                                group_size=64, warm_quantizer="minmax", max_hot_pages=16, batch_migration_size=64,
                                device="cuda")
    pc = ProductionCache(cfg)
    orc = ProductionCacheOracle(2, 8, 128, 64, 512, 4, 64, batch_migration_size=64, decay=cfg.importance_decay)
    rng = np.random.default_rng(7)
    for layer in range(2):
        for n in (200, 1, 1):
            k = rng.standard_normal((8, n, 128)).astype(np.float16).astype(np.float32)
            v = rng.standard_normal((8, n, 128)).astype(np.float16).astype(np.float32)
            pc.update(to_dev(k, torch.float16), to_dev(v, torch.float16), layer)
            orc.update(k, v, layer)
    q = rng.standard_normal((1, 8, 1, 128)).astype(np.float32)
    dq = to_dev(q, torch.float16)
    outs, _ = _graph_matches_eager([lambda: pc.fused_attention(dq, 0), lambda: pc.fused_attention(dq, 1)])
    for layer in range(2):
        assert_close_attn(outs[layer], orc.attention(q, layer))


def test_kivi_fused_attention_in_a_graph():
    from akv.baselines import KIVIFusedCache, KIVIFusedConfig
    from oracle.kivi import KIVIOracle
    announce("KIVIFusedCache.fused_attention graph replays")
    cache = KIVIFusedCache(KIVIFusedConfig(key_bits=2, value_bits=2, group_size=128, residual_length=32))
    orc = KIVIOracle(2, 2, 128, 32, fused=True)
    rng = np.random.default_rng(8)
    k = rng.standard_normal((2, 4, 400, 128)).astype(np.float16).astype(np.float32)
    v = rng.standard_normal((2, 4, 400, 128)).astype(np.float16).astype(np.float32)
    cache.update(to_dev(k, torch.float16), to_dev(v, torch.float16), 0)
    ok, ov = orc.update(k, v, 0)
    q = rng.standard_normal((2, 8, 1, 128)).astype(np.float32)
    dq = to_dev(q, torch.float16)
    outs, _ = _graph_matches_eager([lambda: cache.fused_attention(dq, 0)])
    ref, _ = oatt.attention_fp32(q.astype(np.float16), ok.astype(np.float16), ov.astype(np.float16),
                                 return_weights=False)
    assert_close_attn(outs[0], ref)
