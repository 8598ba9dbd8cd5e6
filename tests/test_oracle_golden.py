"""Pin the oracle against the first-principles known answers in golden/kat.json."""
import json
import os

import numpy as np
import pytest

from oracle import affine as oaff
from oracle import bitpack as obp
from oracle import importance as oimp
from oracle import legacy as oleg

KAT = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "kat.json")))


def test_bitpack_kats():
    for case in KAT["bitpack"]:
        codes = np.array(case["codes"], dtype=np.uint8)
        got = obp.pack(codes, case["bits"])
        assert list(got) == case["bytes"], case
        back = obp.unpack(got, case["bits"], len(codes)) if case["bits"] != 2 or len(codes) % 4 == 0 else None
        if back is not None:
            assert list(back) == case["codes"]


@pytest.mark.parametrize("gi", range(3))
def test_affine_group_kats(gi):
    g = KAT["affine_groups"][gi]
    bits = g["bits"]
    for ch in g["channels"]:
        x = np.array(ch["x"], dtype=np.uint16).view(np.float16)
        # as a K block: one head, len(x) tokens, one channel
        q = oaff.quantize_keys(x.reshape(1, -1, 1), bits, packed=False)
        assert int(q["scale"].view(np.uint16).ravel()[0]) == ch["scale"], ch
        assert int(q["zero"].view(np.uint16).ravel()[0]) == ch["zero"], ch
        assert list(q["codes"].ravel()) == ch["codes"], ch
        d = oaff.dequantize_keys(q, packed=False)
        assert list(d.view(np.uint16).ravel()) == ch["deq"], ch
        # the same group as a V row (per-token over channels)
        qv = oaff.quantize_values(x.reshape(1, 1, -1), bits, packed=False)
        assert list(qv["codes"].ravel()) == ch["codes"]
        assert int(qv["scale"].view(np.uint16).ravel()[0]) == ch["scale"]


def test_importance_kats():
    k = KAT["importance"]["decay_kat"]
    out = oimp.fused_importance_update(np.zeros((1, 1, 1, 32), np.float32), np.array(k["scores"], np.float32),
                                       k["decay"])
    np.testing.assert_allclose(out, k["expect"], atol=1e-7)
    s = KAT["importance"]["sum_over_queries"]
    a = np.array(s["attn"], np.float32)
    out = oimp.fused_importance_update(a, np.array(s["scores"], np.float32), s["decay"])
    np.testing.assert_allclose(out, s["expect"], atol=1e-6)


def test_legacy_pack_vectors():
    """tests/test_quantizer.py:88-108 of the reference, restated with the bytes written out."""
    for name, bits in (("4bit", 4), ("2bit", 2)):
        c = KAT["legacy_pack"][name]
        packed = oleg.kvq_pack(np.array(c["codes"], np.uint8), bits)
        assert list(packed) == c["bytes"]
        un = oleg.kvq_unpack(packed, bits, len(c["codes"]))
        np.testing.assert_array_equal(un, np.array(c["codes"], np.float32))
    data = np.array([0, 128, 255, 42], np.uint8)
    np.testing.assert_array_equal(oleg.kvq_unpack(oleg.kvq_pack(data, 8), 8, 4), data.astype(np.float32))
