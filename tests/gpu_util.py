"""Helpers shared by the GPU parity tests."""
import sys

import numpy as np
import torch

from oracle import affine as oaff

DEV = "cuda"


def announce(msg: str) -> None:
    """Name the case before a GPU step (so a failing run says which one)."""
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def to_dev(x, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(x)) if isinstance(x, np.ndarray) else x
    if dtype is not None:
        t = t.to(dtype)
    return t.to(DEV)


def warm_from_oracle(w: dict):
    """Upload an oracle warm tier (quantize_kv_blocked output) as akv.WarmTier."""
    import akv
    n_out = w.get("n_out", 0)
    return akv.WarmTier(
        to_dev(w["k_codes"]), to_dev(w["k_scale"]), to_dev(w["k_zero"]),
        to_dev(w["v_codes"]), to_dev(w["v_scale"]), to_dev(w["v_zero"]),
        w["bits_k"], w["bits_v"], w["T"], w["G"], w["D"],
        to_dev(w["k_oidx"]) if n_out else None, to_dev(w["v_oidx"]) if n_out else None,
        to_dev(w["k_odata"]) if n_out else None, to_dev(w["v_odata"]) if n_out else None,
    )


def assert_close_attn(got: torch.Tensor, ref: np.ndarray, max_abs=2e-3, mean_abs=1e-3):
    g = got.float().cpu().numpy()
    d = np.abs(g - ref)
    assert np.isfinite(g).all(), "non-finite output"
    assert d.max() <= max_abs, f"max abs err {d.max():.3e} > {max_abs}"
    assert d.mean() <= mean_abs, f"mean abs err {d.mean():.3e} > {mean_abs}"


def bits_equal(a: torch.Tensor, b: np.ndarray):
    an = a.cpu().numpy()
    assert an.shape == b.shape, f"shape {an.shape} != {b.shape}"
    if an.dtype == np.float16:
        an = an.view(np.uint16)
        b = np.asarray(b).astype(np.float16).view(np.uint16)
    neq = np.count_nonzero(an != b)
    assert neq == 0, f"{neq} of {an.size} elements differ"
