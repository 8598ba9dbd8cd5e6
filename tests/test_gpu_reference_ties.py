"""The device AffineQuantizer and demote selection against vectors the reference
produced (tests/golden/reference_ties.npz, see tests/golden/make_reference_ties.py):
on tie-free inputs the whole result dict is the reference's -- keys, outlier_idx
as an int64 tensor of shape (n,), codes / scale / zero / outlier_data bit for bit,
orig_dim and bits -- and the selection is the reference's index set.  (Exact ties
are chosen lowest index first, as the oracle does; tests/test_oracle_reference_ties.py
shows both choices are valid top-n sets.)"""
import os

import numpy as np
import pytest
import torch

from gpu_util import announce, to_dev

pytestmark = pytest.mark.gpu
Z = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "reference_ties.npz"))


@pytest.mark.parametrize("kind", ["k", "v"])
@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("frac", [1, 3])
def test_affine_quantizer_dict_equals_reference(kind, bits, frac):
    from akv.affine_quantizer import AffineQuantConfig, AffineQuantizer
    announce(f"AffineQuantizer vs reference kind={kind} bits={bits} frac={frac}")
    tag = f"q_tiefree_{kind}_b{bits}_f{frac}"
    x = to_dev(Z["q_tiefree_x"].view(np.float16))
    q = AffineQuantizer(AffineQuantConfig(key_bits=bits, value_bits=bits, outlier_fraction=frac / 100))
    r = q.quantize_keys(x) if kind == "k" else q.quantize_values(x)
    assert set(r) == {"scale", "zero", "orig_dim", "bits", "outlier_idx", "outlier_data", "codes"}
    assert r["outlier_idx"].dtype == torch.int64 and str(r["outlier_idx"].dtype) == str(Z[tag + "_outlier_idx_dtype"])
    assert r["outlier_data"].dtype == torch.float16
    np.testing.assert_array_equal(r["outlier_idx"].cpu().numpy(), Z[tag + "_outlier_idx"])
    np.testing.assert_array_equal(r["codes"].cpu().numpy(), Z[tag + "_codes"])
    for key in ("scale", "zero", "outlier_data"):
        np.testing.assert_array_equal(r[key].cpu().numpy().view(np.uint16), Z[f"{tag}_{key}"], err_msg=key)
    assert (r["orig_dim"], r["bits"]) == tuple(int(a) for a in Z[tag + "_scalars"])


@pytest.mark.parametrize("name", ["tiefree", "misaligned"])
def test_demote_selection_equals_reference(name):
    from akv.drop_in import select_demote_indices
    announce(f"select_demote_indices vs reference {name}")
    n, hot_len, budget = (int(a) for a in Z[f"s_{name}_args"])
    got = select_demote_indices(to_dev(Z[f"s_{name}_scores"]), n, hot_len, budget)
    np.testing.assert_array_equal(got.cpu().numpy().astype(np.int64), Z[f"s_{name}_idx"])
