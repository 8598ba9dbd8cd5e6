"""Device bit-packing vs the oracle (bit-exact) and the hand-derived byte KATs."""
import json
import os

import numpy as np
import pytest
import torch

from gpu_util import announce, to_dev
from oracle import bitpack as obp

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "kat.json")


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("dim", [64, 128, 256, 24, 8])
def test_pack_unpack_matches_oracle(bits, dim):
    import akv.bitpack as bp
    announce(f"bitpack bits={bits} dim={dim}")
    rng = np.random.default_rng(bits * 1000 + dim)
    codes = rng.integers(0, 1 << bits, size=(3, 17, dim), dtype=np.uint8)
    packed = bp.pack(to_dev(codes), bits)
    ref = obp.pack(codes, bits)
    np.testing.assert_array_equal(packed.cpu().numpy(), ref)
    back = bp.unpack(packed, bits, dim)
    np.testing.assert_array_equal(back.cpu().numpy(), codes)


@pytest.mark.parametrize("dim", [5, 7, 13])
def test_odd_lengths_pad_like_reference(dim):
    import akv.bitpack as bp
    announce(f"bitpack odd dim={dim}")
    rng = np.random.default_rng(dim)
    for bits in (3, 4):
        codes = rng.integers(0, 1 << bits, size=(4, dim), dtype=np.uint8)
        packed = bp.pack(to_dev(codes), bits)
        np.testing.assert_array_equal(packed.cpu().numpy(), obp.pack(codes, bits))
        np.testing.assert_array_equal(bp.unpack(packed, bits, dim).cpu().numpy(), codes)


def test_byte_kats():
    import akv.bitpack as bp
    announce("bitpack KATs")
    kat = json.load(open(GOLDEN))["bitpack"]
    for case in kat:
        codes = np.array([case["codes"]], dtype=np.uint8)
        got = bp.pack(to_dev(codes), case["bits"]).cpu().numpy()[0]
        assert list(got) == case["bytes"], case


def test_passthrough_widths():
    import akv.bitpack as bp
    codes = to_dev(np.arange(64, dtype=np.uint8).reshape(4, 16))
    assert bp.pack(codes, 8) is codes
    assert bp.unpack(codes, 8, 16) is codes
    assert bp.packed_bytes(codes, 4) == 4 * 8
    assert bp.packed_bytes(codes, 3) == 4 * 6
    assert bp.packed_bytes(codes, 8) == 64


@pytest.mark.parametrize("dim", [8, 13, 128])
def test_per_width_functions(dim):
    """The reference's per-width entry points (pack_uint4 / unpack_uint4, pack_uint3 /
    unpack_uint3, pack_uint2 / unpack_uint2) equal the oracle's byte for byte; like the
    reference's, 2-bit unpacking takes only lengths that are multiples of 4."""
    import akv.bitpack as bp
    announce(f"bitpack per-width functions dim={dim}")
    rng = np.random.default_rng(7 * dim)
    for bits, pk, upk, opk in ((4, bp.pack_uint4, bp.unpack_uint4, obp.pack_uint4),
                               (3, bp.pack_uint3, bp.unpack_uint3, obp.pack_uint3),
                               (2, bp.pack_uint2, bp.unpack_uint2, obp.pack_uint2)):
        codes = rng.integers(0, 1 << bits, size=(2, 3, dim), dtype=np.uint8)
        packed = pk(to_dev(codes))
        np.testing.assert_array_equal(packed.cpu().numpy(), opk(codes))
        if bits == 2 and dim % 4:
            with pytest.raises(ValueError):
                upk(packed, dim)
            continue
        np.testing.assert_array_equal(upk(packed, dim).cpu().numpy(), codes)
