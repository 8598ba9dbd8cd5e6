"""The torch-CPU restatement of the reference CPU path (the bench's CPU baseline)
against the numpy oracle: dequantized K/V bit-exact, attention and importance equal up
to fp32 summation order."""
import numpy as np
import pytest
import torch

from oracle import affine as oaff
from oracle import attention as oatt
from oracle import bitpack as obp
from oracle import importance as oimp
from oracle import torch_cpu as otc


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
def test_unpack_matches_oracle(bits):
    rng = np.random.default_rng(bits)
    codes = rng.integers(0, 1 << bits, size=(3, 5, 128), dtype=np.uint8)
    packed = obp.pack(codes, bits)
    got = otc.unpack_codes(torch.from_numpy(packed), bits, 128).numpy()
    assert np.array_equal(got, codes)


@pytest.mark.parametrize("bk,bv,n_out_frac", [(3, 3, 0.0), (4, 2, 0.01), (2, 4, 0.0)])
def test_decode_path_matches_oracle(bk, bv, n_out_frac):
    rng = np.random.default_rng(7)
    B, Hkv, Hq, Nw, Nh, D = 2, 2, 6, 96, 16, 128
    k = rng.standard_normal((B, Hkv, Nw, D)).astype(np.float16)
    v = rng.standard_normal((B, Hkv, Nw, D)).astype(np.float16)
    k[..., 5] *= 10
    w = oaff.quantize_kv_blocked(k, v, bk, bv, 32, 32, outlier_fraction=n_out_frac)
    kd, vd = oaff.dequant_kv_blocked(w)
    tw = {kk: (torch.from_numpy(np.ascontiguousarray(vv)) if isinstance(vv, np.ndarray) else vv) for kk, vv in w.items()}
    tkd, tvd = otc.dequant_kv_blocked(tw)
    assert np.array_equal(tkd.numpy().view(np.uint16), kd.view(np.uint16))
    assert np.array_equal(tvd.numpy().view(np.uint16), vd.view(np.uint16))
    q = rng.standard_normal((B, Hq, 1, D)).astype(np.float16)
    kh = rng.standard_normal((B, Hkv, Nh, D)).astype(np.float16)
    vh = rng.standard_normal((B, Hkv, Nh, D)).astype(np.float16)
    ref, attn = oatt.mixed_attention_fp32(q, kh, vh, kd, vd, hot_first=False)
    out, tattn = otc.decode_attention(torch.from_numpy(q), torch.from_numpy(kh), torch.from_numpy(vh), tkd, tvd,
                                      hot_first=False)
    np.testing.assert_allclose(out.numpy(), ref, rtol=0, atol=2e-6)
    np.testing.assert_allclose(tattn.numpy(), attn, rtol=1e-5, atol=1e-8)
    sc = rng.random(Nw + Nh + 3).astype(np.float32)
    exp = oimp.fused_importance_update(attn, sc, 0.9)
    got = otc.importance_update(tattn, torch.from_numpy(sc), 0.9).numpy()
    np.testing.assert_allclose(got, exp, rtol=1e-5, atol=1e-8)


@pytest.mark.parametrize("of", [0.0, 0.02])
def test_bench_cpu_baseline_runs_on_host_tensors(of):
    """The bench's CPU-baseline leg on a small layer held in host tensors: it runs every
    sequence at least once and reports the fields of the bench line."""
    import bench
    import akv
    from akv import workloads as wl
    rng = np.random.default_rng(3)
    s = wl.DecodeShape("t", 2, 6, 2, 128, 32, 256, 3, 3, decay=0.9)
    k = rng.standard_normal((s.B, s.Hkv, s.n_warm, s.D)).astype(np.float16)
    v = rng.standard_normal((s.B, s.Hkv, s.n_warm, s.D)).astype(np.float16)
    w = oaff.quantize_kv_blocked(k, v, 3, 3, 32, 32, outlier_fraction=of)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x))
    n_out = w.get("n_out", 0)
    warm = akv.WarmTier(t(w["k_codes"]), t(w["k_scale"]), t(w["k_zero"]), t(w["v_codes"]), t(w["v_scale"]),
                        t(w["v_zero"]), 3, 3, 32, 32, 128,
                        *( [t(w["k_oidx"]), t(w["v_oidx"]), t(w["k_odata"]), t(w["v_odata"])] if n_out else []))
    q = torch.randn(s.B, s.Hq, 1, s.D).half()
    kh = torch.randn(s.B, s.Hkv, s.n_hot, s.D).half()
    vh = torch.randn(s.B, s.Hkv, s.n_hot, s.D).half()
    res = bench.cpu_baseline((q, kh, vh, warm, None), s, budget_s=2.0, min_s=0.2)
    assert res["kind"] == "port" and res["unit"] == "GB/s" and res["value"] > 0
    assert res["cores"] >= 1 and "importance" in res["sample"]
