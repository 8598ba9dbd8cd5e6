"""Pinning of the oracle's chunked prefill with the chunk's causal self-attention
(``oracle.attention.prefill_causal_fp32``): a float64 brute-force loop on tiny
shapes, the last position seeing every token (plain attention over cache + chunk),
a lone first position with no cache returning the chunk's first value, and rows
given by explicit positions equal to those rows of the full computation."""
import numpy as np
import pytest

from oracle import attention as oatt


def _case(B, Hq, Hkv, M, N, D, seed):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, Hq, M, D)).astype(np.float32)
    kc = rng.standard_normal((B, Hkv, N, D)).astype(np.float32) if N else None
    vc = rng.standard_normal((B, Hkv, N, D)).astype(np.float32) if N else None
    kq = rng.standard_normal((B, Hkv, M, D)).astype(np.float32)
    vq = rng.standard_normal((B, Hkv, M, D)).astype(np.float32)
    return q, kc, vc, kq, vq


@pytest.mark.parametrize("B,Hq,Hkv,M,N,D,seed", [(1, 2, 1, 4, 0, 8, 0), (2, 4, 2, 5, 3, 8, 1),
                                                 (1, 6, 3, 7, 9, 16, 2), (1, 1, 1, 1, 0, 4, 3)])
def test_causal_prefill_matches_bruteforce(B, Hq, Hkv, M, N, D, seed):
    q, kc, vc, kq, vq = _case(B, Hq, Hkv, M, N, D, seed)
    got = oatt.prefill_causal_fp32(q, kc, vc, kq, vq)
    ref = oatt.prefill_causal_f64_bruteforce(q, kc, vc, kq, vq)
    np.testing.assert_allclose(got, ref, rtol=2e-5, atol=2e-6)


def test_last_position_sees_every_token():
    q, kc, vc, kq, vq = _case(1, 4, 2, 6, 10, 16, 4)
    got = oatt.prefill_causal_fp32(q, kc, vc, kq, vq)
    full, _ = oatt.attention_fp32(q, np.concatenate([kc, kq], 2), np.concatenate([vc, vq], 2),
                                  return_weights=False)
    np.testing.assert_allclose(got[:, :, -1], full[:, :, -1], rtol=1e-6, atol=1e-7)
    # an earlier position does not: the later chunk tokens are masked out
    assert np.abs(got[:, :, 0] - full[:, :, 0]).max() > 1e-3


def test_first_position_without_cache_is_the_first_value():
    q, _, _, kq, vq = _case(1, 2, 1, 3, 0, 8, 5)
    got = oatt.prefill_causal_fp32(q, None, None, kq, vq)
    np.testing.assert_array_equal(got[0, :, 0], np.broadcast_to(vq[0, 0, 0], (2, 8)))


def test_rows_by_position_match_the_full_chunk():
    q, kc, vc, kq, vq = _case(1, 4, 2, 9, 5, 8, 6)
    full = oatt.prefill_causal_fp32(q, kc, vc, kq, vq)
    sel = np.array([0, 3, 8])
    part = oatt.prefill_causal_fp32(q[:, :, sel], kc, vc, kq, vq, positions=sel)
    np.testing.assert_allclose(part, full[:, :, sel], rtol=1e-6, atol=1e-7)
