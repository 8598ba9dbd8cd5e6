"""Write tests/golden/reference_ties.npz: input/output vectors of two reference
functions for the cases no closed form pins -- the order torch.topk gives among
exactly equal values, and the full result dict of AffineQuantizer.

  * ``AffineQuantizer.quantize_keys`` / ``quantize_values`` with outlier
    channels (akv/affine_quantizer.py:63-176): the channel ranking is
    ``norm(dim=1).mean(dim=0).topk(n)``, so which channels are kept at fp16 when
    channel norms tie is decided by torch.  Cases: tie-free inputs, every channel
    of equal norm, and a few equal-norm channels at the cut.  Every dict entry is
    stored (codes, scale and zero as stored, outlier_idx with its dtype and shape,
    outlier_data, orig_dim, bits).
  * ``AKVLayer._select_demote_indices`` (akv/drop_in.py:392-413):
    ``topk(n, largest=False)`` then an ascending sort.  Cases: tie-free scores,
    all scores equal (a fresh hot tier: every new token has importance 1.0),
    ties at the cut, and a misaligned score vector (FIFO).

This script runs only in the development container, where the reference tree is
at /root/reference; it imports the reference's own package (CPU torch) and
nothing of this repository.  The .npz holds data only (no pickled objects).

Run: python tests/golden/make_reference_ties.py  (rewrites reference_ties.npz)
"""
from __future__ import annotations

import os
import sys
import types

import numpy as np

REF = "/root/reference"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_ties.npz")


def _import_reference():
    here = os.path.dirname(os.path.abspath(__file__))
    # only the reference tree: this repository has a package of the same name
    sys.path[:] = [p for p in sys.path if os.path.abspath(p or ".") not in
                   (os.path.dirname(os.path.dirname(here)), here)]
    sys.path.insert(0, REF)
    import torch
    from akv.affine_quantizer import AffineQuantConfig, AffineQuantizer
    from akv.drop_in import AKVLayer
    assert os.path.dirname(sys.modules["akv"].__file__).startswith(REF)
    return torch, AffineQuantConfig, AffineQuantizer, AKVLayer


def _t(x):
    return x.detach().cpu().numpy()


def quant_cases(torch):
    g = torch.Generator().manual_seed(0)
    H, N, D = 2, 32, 128
    cases = {}
    # tie-free: N(0, 1) with two channels x10 (and one x5 in the second head)
    x = torch.randn(H, N, D, generator=g)
    x[..., 7] *= 10.0
    x[..., 90] *= 10.0
    x[1, :, 41] *= 5.0
    cases["tiefree"] = x.half()
    # every channel of equal L2 norm: +-1 entries
    s = torch.randint(0, 2, (H, N, D), generator=g).float() * 2.0 - 1.0
    cases["alleq"] = s.half()
    # equal-norm channels at the cut: channels 3, 50, 77, 120 share the largest norm
    y = torch.randn(H, N, D, generator=g) * 0.5
    col = torch.randn(H, N, generator=g).sign() * 4.0
    for c in (120, 3, 77, 50):
        y[..., c] = col
    cases["cut"] = y.half()
    return cases


def main():
    torch, AffineQuantConfig, AffineQuantizer, AKVLayer = _import_reference()
    out = {}
    for name, x in quant_cases(torch).items():
        out[f"q_{name}_x"] = _t(x).view(np.uint16)
        for frac in (0.01, 0.03):
            for bits in (2, 3, 4):
                q = AffineQuantizer(AffineQuantConfig(key_bits=bits, value_bits=bits, outlier_fraction=frac))
                for kind, res in (("k", q.quantize_keys(x)), ("v", q.quantize_values(x))):
                    tag = f"q_{name}_{kind}_b{bits}_f{int(frac * 100)}"
                    assert set(res) == {"scale", "zero", "orig_dim", "bits", "outlier_idx", "outlier_data", "codes"}
                    out[tag + "_codes"] = _t(res["codes"])
                    out[tag + "_scale"] = _t(res["scale"]).view(np.uint16)
                    out[tag + "_zero"] = _t(res["zero"]).view(np.uint16)
                    out[tag + "_outlier_idx"] = _t(res["outlier_idx"])
                    out[tag + "_outlier_idx_dtype"] = np.array(str(res["outlier_idx"].dtype))
                    out[tag + "_outlier_data"] = _t(res["outlier_data"]).view(np.uint16)
                    out[tag + "_outlier_data_dtype"] = np.array(str(res["outlier_data"].dtype))
                    out[tag + "_scalars"] = np.array([res["orig_dim"], res["bits"]], dtype=np.int64)
    # demote selection
    g = torch.Generator().manual_seed(1)
    sel_cases = {
        "tiefree": (torch.rand(64, generator=g), 20, 64, 64),
        "alleq": (torch.ones(64), 20, 64, 64),
        "cut": (torch.tensor([0.5, 0.25, 0.25, 0.25] * 16), 17, 64, 256),
        "alleq_long": (torch.full((300,), 0.3), 100, 300, 256),
        "misaligned": (torch.rand(40, generator=g), 10, 64, 64),
    }
    for name, (scores, n_demote, hot_len, hot_budget) in sel_cases.items():
        layer = types.SimpleNamespace(_importance=scores.clone(), hot_budget=hot_budget)
        idx = AKVLayer._select_demote_indices(layer, n_demote, hot_len)
        out[f"s_{name}_scores"] = _t(scores).astype(np.float32)
        out[f"s_{name}_args"] = np.array([n_demote, hot_len, hot_budget], dtype=np.int64)
        out[f"s_{name}_idx"] = _t(idx).astype(np.int64)
    out["torch_version"] = np.array(torch.__version__)
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: {len(out)} arrays, torch {torch.__version__}")


if __name__ == "__main__":
    main()
