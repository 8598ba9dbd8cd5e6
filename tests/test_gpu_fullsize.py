"""The benchmark configurations at full size on the device, checked against the
oracle: the 32k Qwen decode layer with the importance EMA over all 8 sequences,
the Llama-2-7B 16k MHA decode with outlier channels (batch 4), and the Llama-3
demotion of 16 x 65536 tokens at 2/3/4 bits (quantize + pack of the selected
rows, whose input crosses 2^31 bytes).  Quantized bytes are compared bit for
bit; attention within 2e-3 max-abs / 1e-3 mean-abs; the importance EMA within
rtol 5e-5 (fp32 logits summed in another order than the oracle's)."""
import dataclasses
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

from gpu_util import announce, assert_close_attn, bits_equal
from oracle import affine as oaff
from oracle import attention as oatt
from oracle import importance as oimp
from oracle import selection as osel

pytestmark = pytest.mark.gpu

NAMES = ("k_codes", "k_scale", "k_zero", "v_codes", "v_scale", "v_zero")


def _oracle_tier_by_head(kg, vg, bk, bv, T, G):
    """quantize_kv_blocked of one sequence, one thread per head (the heads are
    independent without outlier channels)."""
    H = kg.shape[1]
    with ThreadPoolExecutor(8) as ex:
        parts = list(ex.map(lambda h: oaff.quantize_kv_blocked(kg[:, h:h + 1], vg[:, h:h + 1], bk, bv, T, G),
                            range(H)))
    return {n: np.concatenate([p[n] for p in parts], axis=1) for n in NAMES}


def _host_tier(wt, b, n_out):
    names = list(NAMES) + (["k_oidx", "v_oidx", "k_odata", "v_odata"] if n_out else [])
    w = {n: getattr(wt, n)[b:b + 1].cpu().numpy() for n in names}
    w.update(bits_k=wt.bits_k, bits_v=wt.bits_v, T=wt.block_t, G=wt.group_v, D=wt.head_dim, N=wt.n_warm, n_out=n_out)
    return w


def test_c2_qwen_32k_importance_all_sequences():
    import akv
    from akv import workloads as wl
    announce("full size: Qwen 32k decode layer + importance EMA (decay 0.9) over 8 sequences")
    s = wl.QWEN_DECODE_32K
    k, v = wl.make_kv(s, device="cuda")
    q = wl.make_q(s, device="cuda")
    (kw, vw), (kh, vh) = wl.split_hot_warm(k, v, s.n_hot)
    wt = akv.quantize_kv(kw, vw, s.bits_k, s.bits_v, s.block_t, s.group_v)
    s0 = np.random.default_rng(70).random(s.N).astype(np.float32)
    sc = torch.from_numpy(s0).cuda()
    out = akv.decode_attention(q, kh, vh, wt, hot_first=False, scores=sc, decay=s.decay)
    torch.cuda.synchronize()
    # the tier of sequence 0 is the oracle's byte for byte; the oracle then dequantizes the
    # device tier of every sequence
    ref0 = _oracle_tier_by_head(kw[:1].cpu().numpy(), vw[:1].cpu().numpy(), 3, 3, 32, 32)
    for n in NAMES:
        bits_equal(getattr(wt, n)[:1], ref0[n])
    host = {n: getattr(wt, n).cpu().numpy() for n in NAMES}
    host.update(bits_k=3, bits_v=3, T=32, G=32, D=128, N=s.n_warm, n_out=0)
    kd, vd = oaff.dequant_kv_blocked(host)
    ref, attn = oatt.mixed_attention_fp32(q.cpu().numpy(), kh.cpu().numpy(), vh.cpu().numpy(), kd, vd,
                                          hot_first=False, return_weights=True)
    assert_close_attn(out, ref)
    exp = oimp.fused_importance_update(attn, s0, s.decay)
    got = sc.cpu().numpy()
    np.testing.assert_allclose(got, exp, rtol=5e-5, atol=1e-7)


def test_c3_llama7b_16k_outliers_batch4():
    import akv
    from akv import workloads as wl
    announce("full size: Llama-2-7B 16k MHA decode, K4/V2, outlier_fraction 0.01, batch 4")
    s = wl.LLAMA7B_DECODE_16K
    k, v = wl.make_kv(s, device="cuda")
    q = wl.make_q(s, device="cuda")
    (kw, vw), (kh, vh) = wl.split_hot_warm(k, v, s.n_hot)
    wt = akv.quantize_kv(kw, vw, s.bits_k, s.bits_v, s.block_t, s.group_v, outlier_fraction=s.outlier_fraction)
    assert wt.n_out == 1
    out = akv.decode_attention(q, kh, vh, wt, hot_first=False)
    torch.cuda.synchronize()
    b = 3
    ref_t = oaff.quantize_kv_blocked(kw[b:b + 1].cpu().numpy(), vw[b:b + 1].cpu().numpy(), s.bits_k, s.bits_v,
                                     s.block_t, s.group_v, outlier_fraction=s.outlier_fraction)
    for n in list(NAMES) + ["k_oidx", "v_oidx", "k_odata", "v_odata"]:
        bits_equal(getattr(wt, n)[b:b + 1], ref_t[n])
    kd, vd = oaff.dequant_kv_blocked(_host_tier(wt, b, 1))
    ref, _ = oatt.mixed_attention_fp32(q[b:b + 1].cpu().numpy(), kh[b:b + 1].cpu().numpy(),
                                       vh[b:b + 1].cpu().numpy(), kd, vd, hot_first=False, return_weights=False)
    assert_close_attn(out[b:b + 1], ref)


@pytest.mark.parametrize("bits", [3, 2, 4])
def test_c4_llama3_demote_16x64k(bits):
    import akv
    from akv import workloads as wl
    from akv.drop_in import select_demote_indices
    announce(f"full size: Llama-3 demotion 16 x 8 x 65536 tokens, {bits}-bit")
    s = wl.LLAMA3_DEMOTE_64K
    k, v, imp = wl.make_demote_inputs(s, device="cuda")
    n = s.S - s.keep_hot
    sel = select_demote_indices(imp, n, s.S, s.hot_budget)
    wt = akv.quantize_kv(k, v, bits, bits, s.block_t, s.group_v, sel=sel)
    torch.cuda.synchronize()
    # the last sequence holds the input rows past 2^31 bytes; the first the smallest offsets
    for b in ((0, s.B - 1) if bits == 3 else (s.B - 1,)):
        sb = sel[b].cpu().numpy()
        np.testing.assert_array_equal(sb, osel.select_demote_indices(imp[b].cpu().numpy(), n, s.S, s.hot_budget))
        kg = k[b:b + 1].cpu().numpy()[:, :, sb]
        vg = v[b:b + 1].cpu().numpy()[:, :, sb]
        ref = _oracle_tier_by_head(kg, vg, bits, bits, s.block_t, s.group_v)
        for nme in NAMES:
            bits_equal(getattr(wt, nme)[b:b + 1], ref[nme])
