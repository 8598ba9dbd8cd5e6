"""akv_decode_attn_noalloc (the decode entry point that allocates nothing and
keeps its scratch in a library-held device array) against akv_decode_attn on
the same inputs, called through the C ABI: two calls in a row, the second on a
smaller input, attention within 2e-3 max-abs / 1e-3 mean-abs and the
importance EMA within rtol 1e-5 of the workspace entry point."""
import ctypes

import numpy as np
import pytest
import torch

from gpu_util import announce

pytestmark = pytest.mark.gpu


def _case(B, N, n_hot, seed):
    import akv
    from akv import workloads as wl
    shape = wl.DecodeShape(f"noalloc{B}x{N}", B, 12, 2, 128, n_hot, N - n_hot, 3, 3, k_outlier_channels=2)
    k, v = wl.make_kv(shape, seed, device="cuda")
    q = wl.make_q(shape, seed, device="cuda")
    (kw, vw), (kh, vh) = wl.split_hot_warm(k, v, shape.n_hot)
    warm = akv.quantize_kv(kw, vw, 3, 3, 32, 32)
    return q, kh, vh, warm


def _args(q, kh, vh, warm, out, scores):
    from akv import _native as nat
    a = nat.DecodeArgs()
    a.abi_version = nat.ABI_VERSION
    B, Hq, M, D = q.shape
    a.B, a.Hq, a.Hkv, a.M, a.D = B, Hq, warm.heads, M, D
    a.q_dtype = nat.DT_F16
    a.q = q.data_ptr()
    a.k_hot, a.v_hot, a.n_hot = kh.data_ptr(), vh.data_ptr(), kh.shape[2]
    a.hot_first = 0
    a.sm_scale = D ** -0.5
    a.warm = warm.desc()
    a.out = out.data_ptr()
    a.scores, a.n_scores, a.decay = scores.data_ptr(), scores.numel(), 0.9
    return a


def _run_both(B, N, n_hot, seed):
    from akv import _native as nat
    lib = nat.load()
    q, kh, vh, warm = _case(B, N, n_hot, seed)
    s0 = torch.rand(N, dtype=torch.float32, device="cuda")
    out_ws, sc_ws = torch.empty_like(q), s0.clone()
    out_na, sc_na = torch.empty_like(q), s0.clone()
    a = _args(q, kh, vh, warm, out_ws, sc_ws)
    nbytes = lib.akv_decode_workspace_bytes(ctypes.byref(a))
    assert 0 < nbytes - 256 <= nat.NOALLOC_SCRATCH_BYTES
    ws = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    a.workspace, a.workspace_bytes = ws.data_ptr(), nbytes
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.akv_decode_attn(ctypes.byref(a), stream) == 0, lib.akv_last_error()
    b = _args(q, kh, vh, warm, out_na, sc_na)  # no workspace
    assert lib.akv_decode_attn_noalloc(ctypes.byref(b), stream) == 0, lib.akv_last_error()
    torch.cuda.synchronize()
    d = (out_na.float() - out_ws.float()).abs()
    assert torch.isfinite(out_na.float()).all()
    assert d.max().item() <= 2e-3 and d.mean().item() <= 1e-3, (d.max().item(), d.mean().item())
    np.testing.assert_allclose(sc_na.cpu().numpy(), sc_ws.cpu().numpy(), rtol=1e-5, atol=1e-7)


def test_noalloc_matches_workspace_entry_two_calls():
    announce("noalloc decode: B4 N4096 (hot 512), then B1 N1050 (hot 80, ragged warm tail)")
    _run_both(4, 4096, 512, 11)
    # a second, smaller call reuses the same device scratch (its counters and stale partials)
    _run_both(1, 1050, 80, 12)
    # and the larger shape again after the smaller one
    _run_both(4, 4096, 512, 13)
