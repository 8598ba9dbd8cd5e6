"""Quantize + pack on the device: codes, scales, zeros and packed bytes bit-exact
with the oracle (the reference's AffineQuantizer / bitpack arithmetic)."""
import numpy as np
import pytest
import torch

from gpu_util import announce, bits_equal, to_dev
from oracle import affine as oaff
from oracle import bitpack as obp
from oracle import legacy as oleg

pytestmark = pytest.mark.gpu


def _kv(B, H, N, D, seed, dtype=np.float16, outlier_ch=2):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((B, H, N, D)).astype(np.float32)
    v = rng.standard_normal((B, H, N, D)).astype(np.float32)
    if outlier_ch:
        for h in range(H):
            ch = rng.permutation(D)[:outlier_ch]
            k[:, h, :, ch] *= 10.0
    return k.astype(dtype), v.astype(dtype)


def _check_warm(wt, ref):
    bits_equal(wt.k_codes, ref["k_codes"])
    bits_equal(wt.k_scale, ref["k_scale"])
    bits_equal(wt.k_zero, ref["k_zero"])
    bits_equal(wt.v_codes, ref["v_codes"])
    bits_equal(wt.v_scale, ref["v_scale"])
    bits_equal(wt.v_zero, ref["v_zero"])
    if ref.get("n_out", 0):
        bits_equal(wt.k_oidx, ref["k_oidx"])
        bits_equal(wt.v_oidx, ref["v_oidx"])
        bits_equal(wt.k_odata, ref["k_odata"])
        bits_equal(wt.v_odata, ref["v_odata"])


@pytest.mark.parametrize("bk,bv", [(4, 4), (3, 3), (2, 2), (4, 2), (4, 3), (2, 4)])
def test_blocked_quant_bit_exact(bk, bv):
    import akv
    announce(f"quantize_kv bits={bk}/{bv}")
    k, v = _kv(2, 3, 200, 128, seed=bk * 10 + bv)
    ref = oaff.quantize_kv_blocked(k, v, bk, bv, T=32, G=32)
    wt = akv.quantize_kv(to_dev(k), to_dev(v), bk, bv, block_t=32, group_v=32)
    _check_warm(wt, ref)


@pytest.mark.parametrize("G,bk,bv,N", [(64, 3, 4, 257), (128, 2, 3, 96), (32, 4, 3, 5)])
def test_fast_path_group_sizes(G, bk, bv, N):
    """fp16, D = 128, 32-token K blocks: the one-wave-per-block kernel for every V group size."""
    import akv
    announce(f"quantize_kv fast path G={G} bits={bk}/{bv} N={N}")
    k, v = _kv(2, 3, N, 128, seed=G + N)
    ref = oaff.quantize_kv_blocked(k, v, bk, bv, T=32, G=G)
    wt = akv.quantize_kv(to_dev(k), to_dev(v), bk, bv, block_t=32, group_v=G)
    _check_warm(wt, ref)


@pytest.mark.parametrize("T,G,D", [(16, 64, 128), (64, 128, 128), (32, 32, 64), (48, 64, 64)])
def test_block_and_group_sizes(T, G, D):
    import akv
    announce(f"quantize_kv T={T} G={G} D={D}")
    k, v = _kv(1, 2, 131, D, seed=T + G + D)
    ref = oaff.quantize_kv_blocked(k, v, 3, 3, T=T, G=G)
    wt = akv.quantize_kv(to_dev(k), to_dev(v), 3, 3, block_t=T, group_v=G)
    _check_warm(wt, ref)


@pytest.mark.parametrize("dtype", [np.float32, "bfloat16"])
def test_input_dtypes(dtype):
    import akv
    from oracle.fp import round_bf16
    announce(f"quantize_kv dtype={dtype}")
    k, v = _kv(1, 2, 96, 128, seed=7, dtype=np.float32)
    if dtype == "bfloat16":
        k, v = round_bf16(k), round_bf16(v)
        ref = oaff.quantize_kv_blocked(k, v, 3, 4, T=32, G=32, dt="bfloat16")
        kd, vd = to_dev(k, torch.bfloat16), to_dev(v, torch.bfloat16)
    else:
        ref = oaff.quantize_kv_blocked(k, v, 3, 4, T=32, G=32)
        kd, vd = to_dev(k), to_dev(v)
    wt = akv.quantize_kv(kd, vd, 3, 4, block_t=32, group_v=32)
    _check_warm(wt, ref)


def test_outlier_protection():
    import akv
    announce("quantize_kv outliers")
    k, v = _kv(2, 4, 100, 128, seed=11, outlier_ch=0)
    rng = np.random.default_rng(5)
    # heavy channels make the ranking tie-free
    for h in range(4):
        ch = rng.permutation(128)[:3]
        k[:, h, :, ch] = (k[:, h, :, ch].astype(np.float32) * 8).astype(np.float16)
        v[:, h, :, ch[:1]] = (v[:, h, :, ch[:1]].astype(np.float32) * 6).astype(np.float16)
    ref = oaff.quantize_kv_blocked(k, v, 4, 2, T=32, G=32, outlier_fraction=0.02)
    wt = akv.quantize_kv(to_dev(k), to_dev(v), 4, 2, block_t=32, group_v=32, outlier_fraction=0.02)
    assert wt.n_out == 2
    _check_warm(wt, ref)


def test_gather_selection():
    import akv
    announce("quantize_kv gather")
    k, v = _kv(2, 2, 300, 128, seed=3)
    rng = np.random.default_rng(9)
    sel = np.stack([np.sort(rng.choice(300, 150, replace=False)) for _ in range(2)]).astype(np.int64)
    ks = np.stack([k[b][:, sel[b]] for b in range(2)])
    vs = np.stack([v[b][:, sel[b]] for b in range(2)])
    ref = oaff.quantize_kv_blocked(ks, vs, 3, 3, T=32, G=32)
    wt = akv.quantize_kv(to_dev(k), to_dev(v), 3, 3, block_t=32, group_v=32, sel=to_dev(sel))
    _check_warm(wt, ref)


def test_constant_and_single_token_blocks():
    """scale == 0 in fp16 -> NaN code -> 0 (the reference's clamp(min=1e-8) is a no-op)."""
    import akv
    announce("quantize_kv degenerate blocks")
    k, v = _kv(1, 2, 33, 128, seed=4)  # last block has a single token
    k[:, :, :32, 5] = np.float16(1.25)   # constant channel
    v[:, :, 7, :] = np.float16(-0.5)     # constant token
    ref = oaff.quantize_kv_blocked(k, v, 4, 3, T=32, G=32)
    wt = akv.quantize_kv(to_dev(k), to_dev(v), 4, 3, block_t=32, group_v=32)
    _check_warm(wt, ref)


@pytest.mark.parametrize("kb,vb,of", [(3, 3, 0.0), (4, 2, 0.01), (2, 2, 0.05)])
def test_affine_quantizer_dict(kb, vb, of):
    import akv
    announce(f"AffineQuantizer bits={kb}/{vb} f={of}")
    rng = np.random.default_rng(kb + vb)
    k = (rng.standard_normal((4, 40, 128)) * np.linspace(0.5, 3, 128)).astype(np.float16)
    v = rng.standard_normal((4, 40, 128)).astype(np.float16)
    qz = akv.AffineQuantizer(akv.AffineQuantConfig(key_bits=kb, value_bits=vb, outlier_fraction=of))
    qk = qz.quantize_keys(to_dev(k))
    rk = oaff.quantize_keys(k, kb, of)
    for key in ("codes", "scale", "zero"):
        bits_equal(qk[key], rk[key])
    assert qk["orig_dim"] == rk["orig_dim"] and qk["bits"] == rk["bits"]
    qv = qz.quantize_values(to_dev(v))
    rv = oaff.quantize_values(v, vb, of)
    for key in ("codes", "scale", "zero"):
        bits_equal(qv[key], rv[key])
    if of > 0:
        bits_equal(qk["outlier_idx"], rk["outlier_idx"])
        bits_equal(qk["outlier_data"], rk["outlier_data"])
        bits_equal(qv["outlier_idx"], rv["outlier_idx"])
    bits_equal(qz.dequantize_keys(qk), oaff.dequantize_keys(rk))
    bits_equal(qz.dequantize_values(qv), oaff.dequantize_values(rv))


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
@pytest.mark.parametrize("gs", [32, 128])
def test_fused_quantize_evict(bits, gs):
    import akv
    announce(f"fused_quantize_evict bits={bits} gs={gs}")
    rng = np.random.default_rng(bits + gs)
    keys = rng.standard_normal((64, 64)).astype(np.float16)
    values = rng.standard_normal((64, 64)).astype(np.float16)
    mask = rng.random(64) < 0.4
    got = akv.fused_quantize_evict(to_dev(keys), to_dev(values), to_dev(mask), bits=bits, group_size=gs)
    ref = oleg.quantize_evict(keys, values, mask, bits, gs)
    for g, r in zip(got, ref):
        bits_equal(g, r)


def test_fused_quantize_evict_empty():
    import akv
    keys = to_dev(np.zeros((8, 64), np.float16))
    out = akv.fused_quantize_evict(keys, keys, to_dev(np.zeros(8, bool)))
    assert all(t.numel() == 0 for t in out)
    assert out[1].dtype == torch.float16 and out[0].dtype == torch.uint8


@pytest.mark.parametrize("bits,gs,sym", [(4, 32, False), (2, 32, False), (8, 64, False), (4, 32, True), (2, 128, True)])
def test_kvquantizer(bits, gs, sym):
    import akv
    announce(f"KVQuantizer bits={bits} gs={gs} sym={sym}")
    rng = np.random.default_rng(bits * gs)
    x = rng.standard_normal((2, 3, 20, 64)).astype(np.float16)
    qz = akv.KVQuantizer(akv.QuantConfig(bits=bits, group_size=gs, symmetric=sym))
    qt = qz.quantize(to_dev(x))
    ref = oleg.kvq_quantize(x, bits, gs, sym)
    bits_equal(qt.data, ref["data"])
    bits_equal(qt.scales, ref["scales"])
    bits_equal(qt.zeros, ref["zeros"])
    bits_equal(qz.dequantize(qt), oleg.kvq_dequantize(ref))


def test_kvquantizer_error_and_compression():
    """KVQuantizer.estimate_error is the MSE of the device round trip (more bits, less
    error), and QuantizedTensor.compression_ratio is fp16 bytes over stored bytes."""
    import akv
    announce("KVQuantizer estimate_error / compression_ratio")
    torch.manual_seed(42)
    t = torch.randn(1, 4, 32, 64, dtype=torch.float16).cuda()
    q = akv.KVQuantizer(akv.QuantConfig(group_size=32))
    errs = {b: q.estimate_error(t, bits=b) for b in (2, 4, 8)}
    assert errs[8] < errs[4] < errs[2]
    rec = q.dequantize(q.quantize(t, bits=4))
    assert errs[4] == (t.float() - rec.float()).pow(2).mean().item()
    qt = akv.KVQuantizer(akv.QuantConfig(bits=4, group_size=32)).quantize(t)
    assert qt.compression_ratio == (1 * 4 * 32 * 64 * 2) / qt.nbytes
    assert qt.compression_ratio > 2.0
