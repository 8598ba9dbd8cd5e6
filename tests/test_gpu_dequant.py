"""Dequant / unpack on the device, bit-exact with the oracle."""
import numpy as np
import pytest
import torch

from gpu_util import announce, bits_equal, to_dev, warm_from_oracle
from oracle import affine as oaff
from oracle import legacy as oleg

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bk,bv,of", [(4, 4, 0.0), (3, 3, 0.0), (2, 2, 0.0), (4, 2, 0.01), (3, 4, 0.03)])
def test_affine_dequant_bit_exact(bk, bv, of):
    import akv
    announce(f"dequantize bits={bk}/{bv} f={of}")
    rng = np.random.default_rng(bk * 7 + bv)
    k = rng.standard_normal((2, 2, 160, 128)).astype(np.float16)
    v = rng.standard_normal((2, 2, 160, 128)).astype(np.float16)
    w = oaff.quantize_kv_blocked(k, v, bk, bv, 32, 32, of)
    kd, vd = oaff.dequant_kv_blocked(w)
    gk, gv = akv.dequantize(warm_from_oracle(w))
    bits_equal(gk, kd)
    bits_equal(gv, vd)


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("sym", [False, True])
def test_dequantize_packed(bits, sym):
    from akv.triton_ops import _dequantize_packed
    announce(f"_dequantize_packed bits={bits} sym={sym}")
    rng = np.random.default_rng(bits)
    x = rng.standard_normal((48, 64)).astype(np.float16)
    qt = oleg.kvq_quantize(x, bits, 32, sym)
    for dtype, odt in ((torch.float16, "float16"), (torch.float32, "float32")):
        got = _dequantize_packed(to_dev(qt["data"]), to_dev(qt["scales"]), to_dev(qt["zeros"]), bits, 32, 48, 64,
                                 torch.device("cuda"), dtype)
        ref = oleg.dequantize_packed(qt["data"], qt["scales"], qt["zeros"], bits, 32, 48, 64, odt)
        bits_equal(got, ref)


def test_dequantize_packed_rejects_3bit():
    from akv.triton_ops import _dequantize_packed
    z = to_dev(np.zeros((4, 2), np.float16))
    with pytest.raises(ValueError):
        _dequantize_packed(to_dev(np.zeros(96, np.uint8)), z, z, 3, 32, 4, 64, torch.device("cuda"), torch.float16)
