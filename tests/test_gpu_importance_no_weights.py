"""Importance EMA without returned weights (the logit stash in the workspace, the
weights kernel after the split kernel): shapes the other decode tests do not reach --
query rows M > 1, scores longer and shorter than N, one full and two row chunks per
kv head, hot-first order -- against the oracle's fp32 attention, on repeated calls
on one workspace and across HIP graph replays with eager calls between them.

Tolerance: rtol 1e-5 / atol 1e-7 on one call (fp32 logits summed in another order
than the oracle's), up to 5e-5 after several compounding calls."""
import numpy as np
import pytest
import torch

from gpu_util import announce, assert_close_attn, to_dev, warm_from_oracle
from oracle import affine as oaff
from oracle import attention as oatt
from oracle import importance as oimp

pytestmark = pytest.mark.gpu


def _case(B, Hq, Hkv, Nh, Nw, bk, bv, M=1, seed=0):
    from akv import workloads as wl
    shape = wl.DecodeShape("t", B, Hq, Hkv, 128, Nh, Nw, bk, bv, block_t=32, group_v=32, M=M)
    k, v = wl.make_kv(shape, layer=seed)
    q = wl.make_q(shape, layer=seed)
    (kw, vw), (kh, vh) = wl.split_hot_warm(k, v, Nh)
    w = oaff.quantize_kv_blocked(kw.numpy(), vw.numpy(), bk, bv, 32, 32, 0.0)
    kd, vd = oaff.dequant_kv_blocked(w)
    return q.numpy(), kh.numpy(), vh.numpy(), w, kd, vd


@pytest.mark.parametrize("B,Hq,Hkv,M,Nh,Nw,extra,hot_first", [
    (8, 12, 2, 1, 1024, 7168, 0, False),     # the 32k workload's shape at 8k tokens
    (2, 12, 2, 1, 64, 448, 37, True),        # scores longer than N
    (2, 8, 2, 3, 96, 1280, -100, False),     # M = 3 query rows, scores shorter than N
    (1, 32, 2, 1, 128, 2048, 0, False),      # 16 query heads per kv head: one full row chunk
    (2, 40, 2, 1, 32, 992, 5, True),         # 20 heads per kv head: two row chunks
])
def test_importance_without_weights_vs_oracle(B, Hq, Hkv, M, Nh, Nw, extra, hot_first):
    from akv.warm_tier import DecodeCall
    announce(f"importance without weights B={B} Hq={Hq} Hkv={Hkv} M={M} Nh={Nh} Nw={Nw} extra={extra} hf={hot_first}")
    q, kh, vh, w, kd, vd = _case(B, Hq, Hkv, Nh, Nw, 3, 3, M=M, seed=B + Hq + M)
    N = Nh + Nw
    s0 = np.random.default_rng(5).random(N + extra).astype(np.float32)
    sc = to_dev(s0)
    call = DecodeCall(to_dev(q), to_dev(kh), to_dev(vh), warm_from_oracle(w), scores=sc, decay=0.9,
                      hot_first=hot_first)
    out = call()
    torch.cuda.synchronize()
    ref, ref_attn = oatt.mixed_attention_fp32(q, kh, vh, kd, vd, hot_first=hot_first)
    assert_close_attn(out, ref)
    full = oimp.fused_importance_update(ref_attn, np.zeros(N, np.float32), 0.9)

    def step(s):
        if extra >= 0:
            return oimp.fused_importance_update(ref_attn, s, 0.9)
        return s * np.float32(0.9) + full[: N + extra]  # the scores cover the first N + extra tokens

    exp = step(s0)
    np.testing.assert_allclose(sc.cpu().numpy(), exp, rtol=1e-5, atol=1e-7)
    # the EMA compounds over repeated calls on the same workspace
    for _ in range(2):
        call()
        exp = step(exp)
    torch.cuda.synchronize()
    np.testing.assert_allclose(sc.cpu().numpy(), exp, rtol=3e-5, atol=1e-7)


def test_importance_in_graph():
    """Captured once, replayed three times with eager calls between: every replay
    applies one EMA step (the split counters are zero again after each launch)."""
    from akv.warm_tier import DecodeCall
    announce("importance without weights in a HIP graph")
    q, kh, vh, w, kd, vd = _case(4, 12, 2, 256, 3840, 3, 3, seed=3)
    N = 4096
    s0 = np.random.default_rng(2).random(N).astype(np.float32)
    sc = to_dev(s0)
    call = DecodeCall(to_dev(q), to_dev(kh), to_dev(vh), warm_from_oracle(w), scores=sc, decay=0.9)
    call()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call()
    _, ref_attn = oatt.mixed_attention_fp32(q, kh, vh, kd, vd, hot_first=False)
    exp = oimp.fused_importance_update(ref_attn, s0, 0.9)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        exp = oimp.fused_importance_update(ref_attn, exp, 0.9)
        np.testing.assert_allclose(sc.cpu().numpy(), exp, rtol=5e-5, atol=1e-7)
        call()  # an eager call between replays
        torch.cuda.synchronize()
        exp = oimp.fused_importance_update(ref_attn, exp, 0.9)
        np.testing.assert_allclose(sc.cpu().numpy(), exp, rtol=5e-5, atol=1e-7)
