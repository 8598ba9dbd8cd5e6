"""Fused dequant-attention on the device vs the oracle's fp32 dequant-attention.

Tolerance (from the task statement): 2e-3 max-abs, 1e-3 mean-abs against the
fp32 attention over the oracle's fp16 dequantized K/V."""
import numpy as np
import pytest
import torch

from gpu_util import announce, assert_close_attn, to_dev, warm_from_oracle
from oracle import affine as oaff
from oracle import attention as oatt
from oracle import importance as oimp

pytestmark = pytest.mark.gpu


def _case(B, Hq, Hkv, D, Nh, Nw, bk, bv, T=32, G=32, of=0.0, M=1, seed=0, outl=2, heavy=0):
    from akv import workloads as wl
    shape = wl.DecodeShape("t", B, Hq, Hkv, D, Nh, Nw, bk, bv, outlier_fraction=of, k_outlier_channels=outl,
                           heavy_tail_channels=heavy, block_t=T, group_v=G, M=M)
    k, v = wl.make_kv(shape, layer=seed)
    q = wl.make_q(shape, layer=seed)
    (kw, vw), (kh, vh) = wl.split_hot_warm(k, v, Nh)
    w = oaff.quantize_kv_blocked(kw.numpy(), vw.numpy(), bk, bv, T, G, of)
    kd, vd = oaff.dequant_kv_blocked(w)
    return q.numpy(), kh.numpy(), vh.numpy(), w, kd, vd


def _run(q, kh, vh, w, hot_first, **kw):
    import akv
    wt = warm_from_oracle(w) if w is not None else None
    return akv.decode_attention(to_dev(q), to_dev(kh) if kh is not None else None,
                                to_dev(vh) if vh is not None else None, wt, hot_first=hot_first, **kw)


@pytest.mark.parametrize("bk,bv", [(4, 4), (3, 3), (2, 2), (4, 2), (4, 3), (3, 2)])
def test_qwen_4k_shape(bk, bv):
    announce(f"decode Qwen 4k shape bits={bk}/{bv}")
    q, kh, vh, w, kd, vd = _case(1, 12, 2, 128, 512, 3584, bk, bv)
    out = _run(q, kh, vh, w, hot_first=False)
    ref, _ = oatt.mixed_attention_fp32(q, kh, vh, kd, vd, hot_first=False, return_weights=False)
    assert_close_attn(out, ref)


@pytest.mark.parametrize("hot_first", [False, True])
def test_weights_and_importance(hot_first):
    announce(f"decode weights+importance hot_first={hot_first}")
    q, kh, vh, w, kd, vd = _case(2, 12, 2, 128, 100, 700, 3, 3, seed=1)
    N = 800
    scores0 = np.random.default_rng(0).random(N + 37).astype(np.float32)
    sc = to_dev(scores0)
    out, attn = _run(q, kh, vh, w, hot_first, scores=sc, decay=0.9, return_weights=True)
    ref, ref_attn = oatt.mixed_attention_fp32(q, kh, vh, kd, vd, hot_first=hot_first)
    assert_close_attn(out, ref)
    a = attn.cpu().numpy()
    np.testing.assert_allclose(a, ref_attn, atol=2e-6, rtol=1e-4)
    np.testing.assert_allclose(a.sum(-1), 1.0, atol=1e-5)
    ref_sc = oimp.fused_importance_update(ref_attn, scores0, 0.9)
    np.testing.assert_allclose(sc.cpu().numpy(), ref_sc, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("Nh,Nw,hot_first", [(37, 700, False), (37, 731, False), (37, 731, True), (3, 61, True)])
def test_weights_ragged_token_counts(Nh, Nw, hot_first):
    """Token counts and tier offsets that are not multiples of 4 (scalar stash / weight stores)."""
    announce(f"decode weights ragged Nh={Nh} Nw={Nw} hot_first={hot_first}")
    q, kh, vh, w, kd, vd = _case(2, 8, 2, 128, Nh, Nw, 4, 2, seed=11, M=2)
    N = Nh + Nw
    scores0 = np.random.default_rng(3).random(N + 5).astype(np.float32)
    sc = to_dev(scores0)
    out, attn = _run(q, kh, vh, w, hot_first, scores=sc, decay=0.8, return_weights=True)
    ref, ref_attn = oatt.mixed_attention_fp32(q, kh, vh, kd, vd, hot_first=hot_first)
    assert_close_attn(out, ref)
    a = attn.cpu().numpy()
    np.testing.assert_allclose(a, ref_attn, atol=2e-6, rtol=1e-4)
    np.testing.assert_allclose(a.sum(-1), 1.0, atol=1e-5)
    ref_sc = oimp.fused_importance_update(ref_attn, scores0, 0.8)
    np.testing.assert_allclose(sc.cpu().numpy(), ref_sc, rtol=1e-5, atol=1e-6)


def test_importance_without_weights_matches():
    announce("decode importance (stash in workspace)")
    q, kh, vh, w, kd, vd = _case(2, 12, 2, 128, 64, 448, 4, 4, seed=2)
    s0 = np.zeros(512, np.float32)
    sc = to_dev(s0)
    _run(q, kh, vh, w, False, scores=sc, decay=0.9)
    _, ref_attn = oatt.mixed_attention_fp32(q, kh, vh, kd, vd, hot_first=False)
    np.testing.assert_allclose(sc.cpu().numpy(), oimp.fused_importance_update(ref_attn, s0, 0.9),
                               rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("Hq,Hkv,M", [(32, 32, 1), (8, 2, 1), (4, 1, 1), (12, 2, 3), (2, 2, 9)])
def test_head_groupings(Hq, Hkv, M):
    announce(f"decode Hq={Hq} Hkv={Hkv} M={M}")
    q, kh, vh, w, kd, vd = _case(2, Hq, Hkv, 128, 48, 320, 4, 2, M=M, seed=3)
    out = _run(q, kh, vh, w, hot_first=True)
    ref, _ = oatt.mixed_attention_fp32(q, kh, vh, kd, vd, hot_first=True, return_weights=False)
    assert_close_attn(out, ref)


def test_outlier_channels_heavy_tails():
    announce("decode outliers + heavy tails (Llama-7B shape, small)")
    q, kh, vh, w, kd, vd = _case(2, 32, 32, 128, 64, 512, 4, 2, of=0.01, outl=0, heavy=4, seed=4)
    assert w["n_out"] == 1
    out = _run(q, kh, vh, w, hot_first=False)
    ref, _ = oatt.mixed_attention_fp32(q, kh, vh, kd, vd, hot_first=False, return_weights=False)
    assert_close_attn(out, ref)


@pytest.mark.parametrize("bk,bv,of", [(4, 2, 0.01), (3, 3, 0.02), (2, 4, 0.03), (4, 4, 0.01)])
def test_fast_outlier_channels(bk, bv, of):
    """Outlier channels on the LDS-streamed kernel (D=128, T=32, G=32): up to
    four fp16 channels per block replace the dequantized K and V values."""
    announce(f"decode fast path outliers bits={bk}/{bv} fraction={of}")
    q, kh, vh, w, kd, vd = _case(2, 8, 4, 128, 80, 700, bk, bv, of=of, outl=0, heavy=4, seed=7)
    assert w["n_out"] == max(1, int(128 * of))
    out = _run(q, kh, vh, w, hot_first=False)
    ref, _ = oatt.mixed_attention_fp32(q, kh, vh, kd, vd, hot_first=False, return_weights=False)
    assert_close_attn(out, ref)


def test_fast_outliers_weights_and_importance():
    """Attention weights and the importance EMA through the outlier variant (the
    corrected scores are what the logit stash holds)."""
    announce("decode fast path outliers + weights + importance")
    q, kh, vh, w, kd, vd = _case(2, 8, 4, 128, 48, 500, 4, 2, of=0.02, outl=0, heavy=4, seed=9)
    N = kh.shape[2] + w["N"]
    s0 = np.random.default_rng(4).random(N).astype(np.float32)
    sc = to_dev(s0)
    out, attn = _run(q, kh, vh, w, False, scores=sc, decay=0.9, return_weights=True)
    ref, ref_attn = oatt.mixed_attention_fp32(q, kh, vh, kd, vd, hot_first=False)
    assert_close_attn(out, ref)
    np.testing.assert_allclose(attn.cpu().numpy(), ref_attn, atol=2e-6, rtol=1e-4)
    np.testing.assert_allclose(sc.cpu().numpy(), oimp.fused_importance_update(ref_attn, s0, 0.9),
                               rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("of", [0.01, 0.02])
def test_fast_outliers_nonzero_meta(of):
    """The stored values replace whatever the codes at an outlier channel
    dequantize to: with the channel's K scale / zero made non-zero, the V scale /
    zero of its 32-channel group re-drawn, and random K and V codes everywhere,
    the output must follow the oracle's dequant of that tier (one outlier channel
    per block at 0.01: the V value goes into the PV operand; two at 0.02: the
    correction MFMAs; K takes the code lookup either way)."""
    announce(f"decode fast path outliers (fraction {of}) with non-zero meta at the outlier channels")
    q, kh, vh, w, kd, vd = _case(1, 4, 2, 128, 48, 320, 4, 2, of=of, outl=0, heavy=2, seed=8)
    assert w["k_oidx"].shape[-1] == (1 if of == 0.01 else 2)
    rng = np.random.default_rng(1)
    w = dict(w)
    ks, kz = w["k_scale"].copy(), w["k_zero"].copy()
    vs, vz = w["v_scale"].copy(), w["v_zero"].copy()
    T, G = 32, 32
    for b in range(ks.shape[0]):
        for blk in range(ks.shape[2]):
            for c in w["k_oidx"][b, blk]:
                ks[b, :, blk, c] = rng.uniform(0.05, 0.5, ks.shape[1]).astype(np.float16)
                kz[b, :, blk, c] = rng.uniform(-1.0, 1.0, ks.shape[1]).astype(np.float16)
            t0, t1 = blk * T, min((blk + 1) * T, vs.shape[2])
            for c in w["v_oidx"][b, blk]:
                g = int(c) // G
                vs[b, :, t0:t1, g] = rng.uniform(0.05, 0.5, (vs.shape[1], t1 - t0)).astype(np.float16)
                vz[b, :, t0:t1, g] = rng.uniform(-1.0, 1.0, (vs.shape[1], t1 - t0)).astype(np.float16)
    w["k_scale"], w["k_zero"], w["v_scale"], w["v_zero"] = ks, kz, vs, vz
    w["k_codes"] = rng.integers(0, 256, w["k_codes"].shape, dtype=np.uint8)
    w["v_codes"] = rng.integers(0, 256, w["v_codes"].shape, dtype=np.uint8)
    kd2, vd2 = oaff.dequant_kv_blocked(w)
    out = _run(q, kh, vh, w, hot_first=False)
    ref, _ = oatt.mixed_attention_fp32(q, kh, vh, kd2, vd2, hot_first=False, return_weights=False)
    assert_close_attn(out, ref)


@pytest.mark.parametrize("D", [64])
def test_head_dim_64(D):
    announce("decode D=64")
    q, kh, vh, w, kd, vd = _case(1, 4, 2, D, 32, 224, 3, 4, seed=5)
    out = _run(q, kh, vh, w, hot_first=False)
    ref, _ = oatt.mixed_attention_fp32(q, kh, vh, kd, vd, hot_first=False, return_weights=False)
    assert_close_attn(out, ref)


def test_ragged_tails_and_tiny_hot():
    announce("decode ragged warm tail, 5 hot tokens")
    q, kh, vh, w, kd, vd = _case(1, 6, 3, 128, 5, 75, 3, 3, seed=6)  # 75 warm: partial block
    out = _run(q, kh, vh, w, hot_first=False)
    ref, _ = oatt.mixed_attention_fp32(q, kh, vh, kd, vd, hot_first=False, return_weights=False)
    assert_close_attn(out, ref)


def test_hot_only_and_warm_only():
    announce("decode hot only / warm only")
    q, kh, vh, w, kd, vd = _case(1, 4, 2, 128, 40, 96, 4, 4, seed=7)
    out = _run(q, kh, vh, None, hot_first=True)
    ref, _ = oatt.attention_fp32(q, kh, vh, return_weights=False)
    assert_close_attn(out, ref)
    out = _run(q, None, None, w, hot_first=True)
    ref, _ = oatt.attention_fp32(q, kd, vd, return_weights=False)
    assert_close_attn(out, ref)


def test_split_counts_agree():
    announce("decode split counts")
    q, kh, vh, w, kd, vd = _case(1, 12, 2, 128, 256, 2048, 3, 3, seed=8)
    ref, _ = oatt.mixed_attention_fp32(q, kh, vh, kd, vd, hot_first=False, return_weights=False)
    for ns in (1, 3, 16, 200):
        assert_close_attn(_run(q, kh, vh, w, False, num_splits=ns), ref)


@pytest.mark.parametrize("B,Hq,M", [(4, 12, 1), (5, 12, 2), (8, 12, 2), (8, 10, 4)])
def test_importance_rows_per_thread(B, Hq, M):
    """The weights / importance pass after the in-kernel merge takes 1, 2, 3, 4 or 8 rows
    per thread (B * Hq * M rows over 32 row lanes): 48, 120, 192 and 320 rows run the 2-,
    4- and 8-row instantiations (320 in two batches of loads), checked with the weights
    returned and with the importance alone."""
    announce(f"decode importance rows per thread: B={B} Hq={Hq} M={M}")
    q, kh, vh, w, kd, vd = _case(B, Hq, 2, 128, 64, 448, 3, 3, M=M, seed=14)
    N = kh.shape[2] + w["N"]
    s0 = np.random.default_rng(6).random(N + 3).astype(np.float32)
    ref, ref_attn = oatt.mixed_attention_fp32(q, kh, vh, kd, vd, hot_first=False)
    ref_sc = oimp.fused_importance_update(ref_attn, s0, 0.9)
    sc = to_dev(s0)
    out, attn = _run(q, kh, vh, w, False, scores=sc, decay=0.9, return_weights=True)
    assert_close_attn(out, ref)
    np.testing.assert_allclose(attn.cpu().numpy(), ref_attn, atol=2e-6, rtol=1e-4)
    np.testing.assert_allclose(sc.cpu().numpy(), ref_sc, rtol=1e-5, atol=1e-6)
    sc2 = to_dev(s0)
    _run(q, kh, vh, w, False, scores=sc2, decay=0.9)
    np.testing.assert_allclose(sc2.cpu().numpy(), ref_sc, rtol=1e-5, atol=1e-6)


@pytest.fixture(scope="module")
def long_case():
    return _case(1, 8, 2, 128, 256, 40960, 2, 2, seed=13)


@pytest.mark.parametrize("weights", [True, False])
def test_long_context_many_splits_importance(long_case, weights):
    """One sequence, 2 kv heads, 40k warm + 256 hot tokens: the planner spreads the two
    (batch, kv-head) pairs over 128 splits each, past what the in-kernel merge takes, so
    the separate merge kernel finishes the output, the weights and the importance EMA
    (with the weights returned, or from the logit stash without them)."""
    announce(f"decode 40k tokens, automatic splits, weights={weights}")
    q, kh, vh, w, kd, vd = long_case
    N = kh.shape[2] + w["N"]
    s0 = np.random.default_rng(5).random(N + 11).astype(np.float32)
    sc = to_dev(s0)
    res = _run(q, kh, vh, w, False, scores=sc, decay=0.95, return_weights=weights)
    ref, ref_attn = oatt.mixed_attention_fp32(q, kh, vh, kd, vd, hot_first=False)
    out = res[0] if weights else res
    assert_close_attn(out, ref)
    if weights:
        a = res[1].cpu().numpy()
        np.testing.assert_allclose(a, ref_attn, atol=2e-6, rtol=1e-4)
        np.testing.assert_allclose(a.sum(-1), 1.0, atol=1e-5)
    np.testing.assert_allclose(sc.cpu().numpy(), oimp.fused_importance_update(ref_attn, s0, 0.95),
                               rtol=1e-5, atol=1e-6)


def test_full_size_qwen_32k_slice():
    """One layer of the 32k workload at full size; the oracle checks one batch element."""
    import akv
    from akv import workloads as wl
    announce("decode Qwen 32k full-size layer")
    shape = wl.QWEN_DECODE_32K
    k, v = wl.make_kv(shape, device="cuda")
    q = wl.make_q(shape, device="cuda")
    (kw, vw), (kh, vh) = wl.split_hot_warm(k, v, shape.n_hot)
    wt = akv.quantize_kv(kw, vw, shape.bits_k, shape.bits_v, shape.block_t, shape.group_v)
    out = akv.decode_attention(q, kh, vh, wt, hot_first=False)
    b = 5
    w1 = oaff.quantize_kv_blocked(kw[b:b + 1].cpu().numpy(), vw[b:b + 1].cpu().numpy(), 3, 3, 32, 32)
    # the device tier of batch b is the oracle's, byte for byte
    assert np.array_equal(wt.k_codes[b:b + 1].cpu().numpy(), w1["k_codes"])
    kd, vd = oaff.dequant_kv_blocked(w1)
    ref, _ = oatt.mixed_attention_fp32(q[b:b + 1].cpu().numpy(), kh[b:b + 1].cpu().numpy(),
                                       vh[b:b + 1].cpu().numpy(), kd, vd, hot_first=False, return_weights=False)
    assert_close_attn(out[b:b + 1], ref)


@pytest.mark.parametrize("B,Hkv,Nw,G", [(1, 1, 333, 128), (1, 1, 517, 64), (2, 2, 328, 128), (2, 2, 332, 64),
                                        (2, 2, 333, 128), (1, 2, 301, 64)])
def test_value_groups_64_128_ragged(B, Hkv, Nw, G):
    """V groups of 64 / 128 channels (1 or 2 scale rows per token) with tier lengths
    that end inside a 16-byte piece of the meta rows: the LDS-streamed kernel clears
    the rows past the tier; per-(batch, head) tiers whose meta would not start on 16
    bytes (odd lengths with B * Hkv > 1) run the general kernel."""
    announce(f"decode G={G} B={B} Hkv={Hkv} Nw={Nw}")
    q, kh, vh, w, kd, vd = _case(B, 4 * Hkv, Hkv, 128, 24, Nw, 4, 2, G=G, seed=12)
    out = _run(q, kh, vh, w, hot_first=False)
    ref, _ = oatt.mixed_attention_fp32(q, kh, vh, kd, vd, hot_first=False, return_weights=False)
    assert_close_attn(out, ref)
