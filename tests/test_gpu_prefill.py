"""Chunked-prefill attention on the device vs the oracle's fp32 dequant-attention.

Tolerance (from the task statement): 2e-3 max-abs, 1e-3 mean-abs against the
fp32 attention over the oracle's fp16 dequantized K/V.  bf16 outputs add the
rounding of the output itself: half an ulp of bf16, at most 2^-8 of the value (8
significant bits; the bound is reached at the bottom of a binade)."""
import numpy as np
import pytest
import torch

from gpu_util import announce, assert_close_attn, to_dev, warm_from_oracle
from oracle import affine as oaff
from oracle import attention as oatt

pytestmark = pytest.mark.gpu


def _case(B, Hq, Hkv, Nh, Nw, bk, bv, M, T=32, G=32, seed=0, outl=2):
    from akv import workloads as wl
    shape = wl.DecodeShape("t", B, Hq, Hkv, 128, Nh, Nw, bk, bv, k_outlier_channels=outl,
                           block_t=T, group_v=G, M=M)
    k, v = wl.make_kv(shape, layer=seed)
    q = wl.make_q(shape, layer=seed)
    (kw, vw), (kh, vh) = wl.split_hot_warm(k, v, Nh)
    w = oaff.quantize_kv_blocked(kw.numpy(), vw.numpy(), bk, bv, T, G) if Nw else None
    kd, vd = oaff.dequant_kv_blocked(w) if Nw else (None, None)
    return q, kh.numpy(), vh.numpy(), w, kd, vd


def _prefill(q, kh, vh, w, **kw):
    import akv
    return akv.prefill_attention(to_dev(q), to_dev(kh) if kh is not None and kh.shape[2] else None,
                                 to_dev(vh) if vh is not None and vh.shape[2] else None,
                                 warm_from_oracle(w) if w is not None else None, **kw)


@pytest.mark.parametrize("bk,bv", [(2, 2), (3, 3), (4, 4), (4, 2), (2, 4), (3, 2)])
def test_prefill_bits_ragged(bk, bv):
    announce(f"prefill bits={bk}/{bv} M=24 ragged hot/warm")
    q, kh, vh, w, kd, vd = _case(1, 8, 2, 40, 200, bk, bv, M=24, seed=1)
    out = _prefill(q.numpy(), kh, vh, w)
    ref, _ = oatt.mixed_attention_fp32(q.numpy(), kh, vh, kd, vd, return_weights=False)
    assert_close_attn(out, ref)


@pytest.mark.parametrize("ns", [2, 3, 7])
def test_prefill_token_splits(ns):
    announce(f"prefill num_splits={ns}")
    q, kh, vh, w, kd, vd = _case(2, 4, 2, 64, 448, 3, 3, M=20, seed=2)
    out = _prefill(q.numpy(), kh, vh, w, num_splits=ns)
    ref, _ = oatt.mixed_attention_fp32(q.numpy(), kh, vh, kd, vd, return_weights=False)
    assert_close_attn(out, ref)


def test_prefill_bf16_queries_and_group_sizes():
    announce("prefill bf16 q, G=64, T=64, two row tiles")
    q, kh, vh, w, kd, vd = _case(2, 4, 1, 32, 320, 2, 2, M=40, T=64, G=64, seed=3)
    qb = q.to(torch.bfloat16)
    out = _prefill(qb, kh, vh, w)
    assert out.dtype == torch.bfloat16
    ref, _ = oatt.mixed_attention_fp32(qb.float().numpy(), kh, vh, kd, vd, return_weights=False)
    got = out.float().cpu().numpy()
    err = np.abs(got - ref)
    bound = 2e-3 + np.abs(ref) * 2.0 ** -8
    assert (err <= bound).all(), f"max excess {np.max(err - bound):.3e}"
    assert err.mean() <= 1e-3


def test_prefill_hot_only_and_warm_only():
    announce("prefill hot only / warm only")
    q, kh, vh, w, kd, vd = _case(1, 6, 3, 48, 96, 4, 4, M=8, seed=4)
    out = _prefill(q.numpy(), kh, vh, None)
    ref, _ = oatt.attention_fp32(q.numpy(), kh, vh, return_weights=False)
    assert_close_attn(out, ref)
    out = _prefill(q.numpy(), kh[:, :, :0], vh[:, :, :0], w)
    ref, _ = oatt.attention_fp32(q.numpy(), kd, vd, return_weights=False)
    assert_close_attn(out, ref)


def test_prefill_matches_decode_kernel():
    """Same cache and queries through both device kernels (M = 1 and M = 9)."""
    import akv
    announce("prefill vs decode kernel")
    for M in (1, 9):
        q, kh, vh, w, kd, vd = _case(2, 12, 2, 100, 700, 3, 3, M=M, seed=5)
        a = _prefill(q.numpy(), kh, vh, w)
        b = akv.decode_attention(to_dev(q.numpy()), to_dev(kh), to_dev(vh), warm_from_oracle(w))
        ref, _ = oatt.mixed_attention_fp32(q.numpy(), kh, vh, kd, vd, return_weights=False)
        assert_close_attn(a, ref)
        assert (a.float() - b.float()).abs().max().item() <= 2e-3


def test_prefill_llama70b_128k_slice():
    """The 128k chunked-prefill workload at full size on the device; the oracle
    checks kv-head 0's 8 query heads at the chunk's first 64 positions."""
    import akv
    from akv import workloads as wl
    announce("prefill Llama-70B 128k full size")
    sh = wl.LLAMA70B_PREFILL_128K
    k, v = wl.make_kv(sh, device="cuda")
    q = wl.make_q(sh, device="cuda", dtype=torch.bfloat16)
    (kw, vw), (kh, vh) = wl.split_hot_warm(k, v, sh.n_hot)
    wt = akv.quantize_kv(kw, vw, sh.bits_k, sh.bits_v, sh.block_t, sh.group_v)
    out = akv.prefill_attention(q, kh, vh, wt)
    torch.cuda.synchronize()
    kd, vd = akv.dequantize(wt)  # bit-exact with the oracle's dequant (test_gpu_quant)
    g = sh.Hq // sh.Hkv
    qs = q[:, :g, :64].float().cpu().numpy()
    ref, _ = oatt.mixed_attention_fp32(qs, kh[:, :1].cpu().numpy(), vh[:, :1].cpu().numpy(),
                                       kd[:, :1].cpu().numpy(), vd[:, :1].cpu().numpy(), return_weights=False)
    got = out[:, :g, :64].float().cpu().numpy()
    err = np.abs(got - ref)
    bound = 2e-3 + np.abs(ref) * 2.0 ** -8
    assert (err <= bound).all(), f"max excess {np.max(err - bound):.3e}"
    assert err.mean() <= 1e-3


def _chunk_kv(B, Hkv, M, seed, dtype=torch.float16):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(B, Hkv, M, 128, generator=g).to(dtype), torch.randn(B, Hkv, M, 128, generator=g).to(dtype))


@pytest.mark.parametrize("M,ns", [(24, 0), (40, 0), (33, 3), (70, 5)])
def test_prefill_causal_chunk(M, ns):
    """The chunk's own K/V after the cache, causal: position m sees chunk tokens 0..m
    (ragged last chunk tiles, chunk tiles spread over token splits)."""
    announce(f"prefill causal chunk M={M} splits={ns}")
    q, kh, vh, w, kd, vd = _case(2, 8, 2, 40, 200, 3, 3, M=M, seed=7)
    kq, vq = _chunk_kv(2, 2, M, seed=M)
    out = _prefill(q.numpy(), kh, vh, w, num_splits=ns, k_chunk=to_dev(kq), v_chunk=to_dev(vq))
    kcache = np.concatenate([kh, kd.astype(np.float16)], axis=2)
    vcache = np.concatenate([vh, vd.astype(np.float16)], axis=2)
    ref = oatt.prefill_causal_fp32(q.numpy(), kcache, vcache, kq.numpy(), vq.numpy())
    assert_close_attn(out, ref)


@pytest.mark.parametrize("M,ns", [(100, 13), (100, 11), (80, 6)])
def test_prefill_causal_masked_splits(M, ns):
    """Token splits that begin past the chunk's first tile: early positions see no token
    of such a split (its partial must weigh nothing in the merge).  13 tiles (2 hot,
    7 warm, 4 chunk at M=100) in 13 / 7 splits (asked for 11), and 12 tiles (M=80) in 6."""
    announce(f"prefill causal chunk, fully masked splits M={M} splits={ns}")
    q, kh, vh, w, kd, vd = _case(1, 8, 2, 40, 200, 3, 3, M=M, seed=12)
    kq, vq = _chunk_kv(1, 2, M, seed=13)
    out = _prefill(q.numpy(), kh, vh, w, num_splits=ns, k_chunk=to_dev(kq), v_chunk=to_dev(vq))
    kcache = np.concatenate([kh, kd.astype(np.float16)], axis=2)
    vcache = np.concatenate([vh, vd.astype(np.float16)], axis=2)
    ref = oatt.prefill_causal_fp32(q.numpy(), kcache, vcache, kq.numpy(), vq.numpy())
    assert np.isfinite(out.float().cpu().numpy()).all()
    assert_close_attn(out, ref)


def test_prefill_causal_single_position_and_row_tiles():
    """M = 1: the one new token sees the whole cache and itself (plain attention over
    cache + that token).  M = 300 with 8 query heads per kv head: 2,400 rows per
    (batch, kv-head), ten 256-row tiles, the last one partial; B = 2, bf16."""
    announce("prefill causal chunk M=1, and M=300 over ten row tiles (bf16, B=2)")
    q, kh, vh, w, kd, vd = _case(1, 4, 2, 40, 200, 3, 3, M=1, seed=16)
    kq, vq = _chunk_kv(1, 2, 1, seed=17)
    out = _prefill(q.numpy(), kh, vh, w, k_chunk=to_dev(kq), v_chunk=to_dev(vq))
    kall = np.concatenate([kh, kd.astype(np.float16), kq.numpy()], axis=2)
    vall = np.concatenate([vh, vd.astype(np.float16), vq.numpy()], axis=2)
    ref, _ = oatt.attention_fp32(q.numpy(), kall, vall, return_weights=False)
    assert_close_attn(out, ref)
    q, kh, vh, w, kd, vd = _case(2, 16, 2, 64, 320, 2, 2, M=300, seed=18)
    qb = q.to(torch.bfloat16)
    kq, vq = _chunk_kv(2, 2, 300, seed=19, dtype=torch.bfloat16)
    out = _prefill(qb, kh, vh, w, k_chunk=to_dev(kq), v_chunk=to_dev(vq))
    kcache = np.concatenate([kh, kd.astype(np.float16)], axis=2)
    vcache = np.concatenate([vh, vd.astype(np.float16)], axis=2)
    ref = oatt.prefill_causal_fp32(qb.float().numpy(), kcache, vcache, kq.float().numpy(), vq.float().numpy())
    err = np.abs(out.float().cpu().numpy() - ref)
    bound = 2e-3 + np.abs(ref) * 2.0 ** -8
    assert (err <= bound).all(), f"max excess {np.max(err - bound):.3e}"
    assert err.mean() <= 1e-3


def test_prefill_causal_chunk_only_splits():
    """The chunk alone (no cache) over several token splits: rows before a split's first
    token get nothing from it."""
    announce("prefill causal chunk alone, 4 splits")
    q, _, _, _, _, _ = _case(1, 8, 1, 32, 96, 3, 3, M=128, seed=14)
    kq, vq = _chunk_kv(1, 1, 128, seed=15)
    out = _prefill(q.numpy(), None, None, None, num_splits=4, k_chunk=to_dev(kq), v_chunk=to_dev(vq))
    ref = oatt.prefill_causal_fp32(q.numpy(), None, None, kq.numpy(), vq.numpy())
    assert np.isfinite(out.float().cpu().numpy()).all()
    assert_close_attn(out, ref)


def test_prefill_causal_chunk_bf16_and_chunk_only():
    announce("prefill causal chunk bf16, and the chunk alone")
    q, kh, vh, w, kd, vd = _case(1, 4, 1, 32, 96, 4, 2, M=36, seed=8)
    qb = q.to(torch.bfloat16)
    kq, vq = _chunk_kv(1, 1, 36, seed=9, dtype=torch.bfloat16)
    out = _prefill(qb, kh, vh, w, k_chunk=to_dev(kq), v_chunk=to_dev(vq))
    assert out.dtype == torch.bfloat16
    kcache = np.concatenate([kh, kd.astype(np.float16)], axis=2)
    vcache = np.concatenate([vh, vd.astype(np.float16)], axis=2)
    ref = oatt.prefill_causal_fp32(qb.float().numpy(), kcache, vcache, kq.float().numpy(), vq.float().numpy())
    got = out.float().cpu().numpy()
    err = np.abs(got - ref)
    bound = 2e-3 + np.abs(ref) * 2.0 ** -8
    assert (err <= bound).all(), f"max excess {np.max(err - bound):.3e}"
    assert err.mean() <= 1e-3
    # no cache at all: the chunk's causal self-attention alone
    kq16, vq16 = _chunk_kv(1, 1, 36, seed=10)
    out = _prefill(q.numpy(), None, None, None, k_chunk=to_dev(kq16), v_chunk=to_dev(vq16))
    ref = oatt.prefill_causal_fp32(q.numpy(), None, None, kq16.numpy(), vq16.numpy())
    assert_close_attn(out, ref)


def test_prefill_llama70b_128k_causal_slice():
    """The 128k workload with the chunk's causal self-attention at full size; the oracle
    checks kv-head 0's 8 query heads at the chunk's first and last 32 positions."""
    import akv
    from akv import workloads as wl
    announce("prefill Llama-70B 128k full size, causal chunk")
    sh = wl.LLAMA70B_PREFILL_128K
    k, v = wl.make_kv(sh, device="cuda")
    q = wl.make_q(sh, device="cuda", dtype=torch.bfloat16)
    (kw, vw), (kh, vh) = wl.split_hot_warm(k, v, sh.n_hot)
    wt = akv.quantize_kv(kw, vw, sh.bits_k, sh.bits_v, sh.block_t, sh.group_v)
    kq, vq = (t.to("cuda") for t in _chunk_kv(sh.B, sh.Hkv, sh.M, seed=11, dtype=torch.bfloat16))
    out = akv.prefill_attention(q, kh, vh, wt, k_chunk=kq, v_chunk=vq)
    torch.cuda.synchronize()
    kd, vd = akv.dequantize(wt)
    g = sh.Hq // sh.Hkv
    sel = np.concatenate([np.arange(32), np.arange(sh.M - 32, sh.M)])
    qs = q[:, :g, sel].float().cpu().numpy()
    kcache = np.concatenate([kh[:, :1].cpu().numpy(), kd[:, :1].cpu().numpy()], axis=2)
    vcache = np.concatenate([vh[:, :1].cpu().numpy(), vd[:, :1].cpu().numpy()], axis=2)
    ref = oatt.prefill_causal_fp32(qs, kcache, vcache, kq[:, :1].float().cpu().numpy(),
                                   vq[:, :1].float().cpu().numpy(), positions=sel)
    got = out[:, :g, sel].float().cpu().numpy()
    err = np.abs(got - ref)
    bound = 2e-3 + np.abs(ref) * 2.0 ** -8
    assert (err <= bound).all(), f"max excess {np.max(err - bound):.3e}"
    assert err.mean() <= 1e-3
