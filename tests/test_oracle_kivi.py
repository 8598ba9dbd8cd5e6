"""The KIVI oracle (oracle/kivi.py) pinned: codes against a float64 nearest-level
brute force, KATs for ties, a constant group and zero padding, the dequant closed
form for every code, and the reference's own KIVI tests (tests/test_kivi_fused.py)
restated on the oracle."""
import numpy as np
import pytest

from oracle.kivi import KIVIOracle, kivi_dequantize, kivi_quantize


@pytest.mark.parametrize("bits,gs", [(2, 32), (4, 64), (8, 128), (4, 16)])
def test_codes_are_the_nearest_level(bits, gs):
    rng = np.random.default_rng(bits + gs)
    x = (rng.standard_normal((2, 3, 5, 128)) * 2).astype(np.float16).astype(np.float32)
    codes, sc, ze = kivi_quantize(x, bits, gs)
    g = x.reshape(-1, 128 // gs, gs).astype(np.float64)
    levels = np.arange(1 << bits, dtype=np.float64)
    deq = levels[None, None, None, :] * sc.astype(np.float64)[..., None, None] + ze.astype(np.float64)[..., None, None]
    err = np.abs(deq - g[..., None])
    best = err.min(axis=-1)
    chosen = np.take_along_axis(err, codes.astype(np.int64)[..., None], axis=-1)[..., 0]
    # the float32 quotient can move a near-tie by a rounding of the scale
    assert np.all(chosen <= best + 1e-6 * sc[..., None].astype(np.float64) + 1e-12)
    assert codes.max() <= (1 << bits) - 1
    np.testing.assert_array_equal(ze, g.min(axis=-1).astype(np.float32))


def test_kats_ties_constant_and_padding():
    # [0, 0.5, 1.5, 3] at 2 bits: scale 1, quotients 0, 0.5, 1.5, 3 -> half-to-even 0, 0, 2, 3
    codes, sc, ze = kivi_quantize(np.array([[[[0.0, 0.5, 1.5, 3.0] * 8]]], np.float32), 2, 32)
    assert sc[0, 0] == 1.0 and ze[0, 0] == 0.0
    assert codes[0, 0, :4].tolist() == [0, 0, 2, 3]
    # a constant group: scale clamped at 1e-10, codes 0, dequant returns the constant
    x = np.full((1, 1, 1, 64), 0.75, np.float32)
    codes, sc, ze = kivi_quantize(x, 4, 32)
    assert np.all(sc == np.float32(1e-10)) and np.all(codes == 0)
    np.testing.assert_array_equal(kivi_dequantize(codes, sc, ze, x.shape), x.astype(np.float16))
    # head_dim 64 in groups of 128: zero padding joins the min / max
    x = np.full((1, 1, 1, 64), 2.0, np.float32)
    codes, sc, ze = kivi_quantize(x, 2, 128)
    assert codes.shape == (1, 1, 128) and ze[0, 0] == 0.0 and sc[0, 0] == np.float32(2.0 / 3.0)
    assert np.all(codes[0, 0, :64] == 3) and np.all(codes[0, 0, 64:] == 0)


def test_dequant_closed_form_every_code():
    for bits in (2, 4, 8):
        codes = np.arange(1 << bits, dtype=np.uint8).reshape(1, 1, -1)
        codes = np.tile(codes, (1, 1, 256 // codes.shape[-1]))[:, :, :128].reshape(1, 1, 128)
        sc = np.array([[np.float32(0.3071)]], np.float32)
        ze = np.array([[np.float32(-1.25)]], np.float32)
        got = kivi_dequantize(codes, sc, ze, (1, 1, 1, 128)).astype(np.float64).reshape(-1)
        exp = codes.reshape(-1).astype(np.float64) * float(sc[0, 0]) + float(ze[0, 0])
        np.testing.assert_allclose(got, exp, rtol=2 ** -11, atol=2 ** -14)


def _kv(rng, n, H=4, D=64):
    return rng.standard_normal((1, H, n, D)).astype(np.float32), rng.standard_normal((1, H, n, D)).astype(np.float32)


def test_reference_kivi_tests_restated():
    """tests/test_kivi_fused.py on the oracle (group 32, head_dim 64)."""
    naive = KIVIOracle(4, 4, 32, 8, fused=False)
    fused = KIVIOracle(4, 4, 32, 8, fused=True)
    rng = np.random.default_rng(0)
    for _ in range(20):
        k, v = _kv(rng, 1)
        nk, _ = naive.update(k, v, 0)
        fk, _ = fused.update(k, v, 0)
    assert nk.shape == fk.shape and np.abs(nk - fk).max() < 0.5
    naive2, fused2 = KIVIOracle(2, 2, 32, 4, fused=False), KIVIOracle(2, 2, 32, 4, fused=True)
    for _ in range(32):
        k, v = _kv(rng, 1)
        naive2.update(k, v, 0)
        fused2.update(k, v, 0)
    a, b = naive2.memory_bytes(), fused2.memory_bytes()
    assert a > 0 and b > 0 and max(a, b) / min(a, b) < 10
    sizes = []
    grow = KIVIOracle(4, 4, 32, 4, fused=True)
    for _ in range(20):
        k, v = _kv(rng, 1)
        grow.update(k, v, 0)
        if 0 in grow.q_k:
            sizes.append(grow.quantized_rows(0)[0].shape[1])
    assert sizes and all(b >= a for a, b in zip(sizes, sizes[1:]))


def test_fused_view_is_chunkwise_dequant():
    """The fused working copy is the concatenation of each chunk's dequant; the naive
    view re-quantizes the dequantized history (so the two differ after a merge)."""
    rng = np.random.default_rng(5)
    fused = KIVIOracle(2, 2, 32, 4, fused=True)
    chunks = []
    for _ in range(6):
        k, v = _kv(rng, 3)
        chunks.append(k)
        fk, _ = fused.update(k, v, 0)
    allk = np.concatenate(chunks, axis=2).astype(np.float16).astype(np.float32)
    n_q = allk.shape[2] - 4
    np.testing.assert_array_equal(fk[:, :, n_q:], allk[:, :, n_q:])  # the residual window is exact
    assert fk.shape[2] == allk.shape[2]
