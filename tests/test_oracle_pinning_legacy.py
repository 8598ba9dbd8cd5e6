"""Pins of the oracle's legacy-layout functions against exact rational
arithmetic (tests/exact_fp.py), enumerated quantization levels and a
bit-position packer -- not against a retyped copy of their formulas.

  * oracle.legacy.kvq_quantize      <- KVQuantizer.quantize (akv/quantizer.py:71-143)
  * oracle.legacy.dequant_int4_tile <- _dequant_int4_tile (akv/fused_attention.py:293-317)
  * oracle.legacy.quantize_evict    <- fused_quantize_evict (akv/triton_kernels.py:426-507)

Each check is chosen so that a plausible slip in the oracle fails it: floor or
round-half-up for round-half-even, a missing or wrong scale clamp, the zero
padding of a ragged last group dropped from min/max, the nibble or crumb order
swapped, fp32 arithmetic where the reference computes in fp16 (or the reverse).
"""
from fractions import Fraction

import numpy as np
import pytest

from exact_fp import f16, f32, frac, nearest_level, pack_bits_msb
from oracle import legacy as oleg


# ------------------------------------------------------------- KVQuantizer

def _kvq_bruteforce(x: np.ndarray, bits: int, gs: int):
    """KVQuantizer.quantize, asymmetric: fp32 arithmetic on the input values,
    scale = f32(f32(max - min) / maxv) clamped below at f32(1e-10), code = the
    level nearest to f32(f32(x - min) / scale); scales / zeros stored in the
    input dtype.  Returns (codes (rows, G*gs), scales (rows, G), zeros)."""
    maxv = (1 << bits) - 1
    rows, D = x.shape
    G = -(-D // gs)
    lo = f32(Fraction(1e-10))
    codes = np.zeros((rows, G * gs), np.int64)
    scales = np.zeros((rows, G), np.float64)
    zeros = np.zeros((rows, G), np.float64)
    store = f16 if x.dtype == np.float16 else (lambda v: v)
    for r in range(rows):
        vals = [frac(v) for v in x[r]] + [Fraction(0)] * (G * gs - D)  # zero padding joins min/max
        for g in range(G):
            grp = vals[g * gs:(g + 1) * gs]
            mn, mx = min(grp), max(grp)
            s = f32(f32(mx - mn) / maxv)
            s = max(s, lo)
            for j, v in enumerate(grp):
                codes[r, g * gs + j] = nearest_level(f32(f32(v - mn) / s), maxv)
            scales[r, g] = float(store(s))
            zeros[r, g] = float(store(mn))
    return codes, scales, zeros


def _kvq_pack_ref(codes: np.ndarray, bits: int) -> np.ndarray:
    if bits == 8:
        return codes.astype(np.uint8).reshape(-1)
    return pack_bits_msb(codes.reshape(-1), bits, 8 // bits)


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("dtype", [np.float16, np.float32])
def test_kvq_quantize_bruteforce(bits, dtype):
    rng = np.random.default_rng(100 + bits)
    for D, gs in ((64, 32), (40, 32), (24, 64), (96, 32)):  # ragged last group and gs > D included
        x = (rng.standard_normal((3, D)) * rng.choice([0.05, 1.0, 20.0])).astype(dtype)
        qt = oleg.kvq_quantize(x, bits, gs)
        codes, scales, zeros = _kvq_bruteforce(x, bits, gs)
        np.testing.assert_array_equal(qt["data"].reshape(-1), _kvq_pack_ref(codes, bits))
        np.testing.assert_array_equal(qt["scales"].astype(np.float64), scales)
        np.testing.assert_array_equal(qt["zeros"].astype(np.float64), zeros)
        assert qt["scales"].dtype == dtype and qt["zeros"].dtype == dtype


def test_kvq_ties_round_half_even():
    # 2-bit: min 0, max 3 -> scale 1; 0.5 -> 0, 1.5 -> 2, 2.5 -> 2 (floor gives 0, 1, 2; half-up 1, 2, 3)
    x = np.array([[0.0, 0.5, 1.5, 2.5, 3.0, 1.0, 2.0, 0.0]], np.float32)
    qt = oleg.kvq_quantize(x, 2, 8)
    assert list(oleg.kvq_unpack(qt["data"], 2, 8).astype(int)) == [0, 0, 2, 2, 3, 1, 2, 0]


def test_kvq_constant_group_and_clamp():
    # a constant group: scale 0 -> clamp 1e-10 -> every code 0; stored as fp16 the clamp value underflows to 0
    for dt in (np.float16, np.float32):
        x = np.full((2, 32), 1.25, dt)
        qt = oleg.kvq_quantize(x, 4, 32)
        assert np.all(oleg.kvq_unpack(qt["data"], 4, 64) == 0)
        assert np.all(qt["zeros"] == dt(1.25))
        assert np.all(qt["scales"] == (dt(0) if dt == np.float16 else np.float32(1e-10)))
    # the clamp is active: range 1e-9 over 15 levels is below 1e-10, so 1e-9 / 1e-10 -> code 10, not 15
    x = np.zeros((1, 32), np.float32)
    x[0, 1] = 1e-9
    qt = oleg.kvq_quantize(x, 4, 32)
    assert list(oleg.kvq_unpack(qt["data"], 4, 2).astype(int)) == [0, 10]


def test_kvq_ragged_padding_joins_minmax():
    # D = 40, gs = 32: the second group holds 8 values and 24 zero pads; all 8 values are >= 1, so
    # min is the pad 0, not 1 (an oracle that skipped the pads would give scale (4-1)/15 and min 1)
    x = np.zeros((1, 40), np.float32)
    x[0, :32] = np.linspace(-1, 1, 32)
    x[0, 32:] = np.linspace(1, 4, 8)
    qt = oleg.kvq_quantize(x, 4, 32)
    assert qt["zeros"][0, 1] == 0.0
    assert qt["scales"][0, 1] == np.float32(np.float32(4.0) / np.float32(15))


# --------------------------------------------------------- _dequant_int4_tile

def test_dequant_int4_tile_every_code():
    """Every 4-bit code x sampled fp16 (scale, zero): f16(f32(f32(c * s) + z)), both nibbles in order."""
    rng = np.random.default_rng(7)
    H, N, D, gs = 2, 8, 32, 16
    codes = np.tile(np.arange(16, dtype=np.uint8), H * N * D // 16).reshape(H, N, D)
    rng.shuffle(codes.reshape(-1))
    packed = ((codes[..., 0::2] << 4) | codes[..., 1::2]).astype(np.uint8)
    s = (rng.random((H, N, D // gs)) * 3).astype(np.float16)
    z = (rng.standard_normal((H, N, D // gs)) * 4).astype(np.float16)
    s[0, 0, 0] = np.float16(6.1e-5)  # a subnormal-adjacent scale
    z[0, 1, 1] = np.float16(-1000.0)  # a zero far past the product (fp16 rounding of the sum matters)
    got = oleg.dequant_int4_tile(packed, s, z, D, gs)
    assert got.dtype == np.float16
    for h in range(H):
        for n in range(N):
            for d in range(D):
                g = d // gs
                e = f16(f32(f32(int(codes[h, n, d]) * frac(s[h, n, g])) + frac(z[h, n, g])))
                assert Fraction(float(got[h, n, d])) == e, (h, n, d)


def test_dequant_int4_tile_equals_dequantize_packed():
    """Per-head int4 tile (fused_attention.py:293) against the flat legacy dequant
    (triton_ops.py:657) head by head, when the zero-points are not all zero."""
    rng = np.random.default_rng(8)
    H, N, D, gs = 3, 5, 64, 32
    packed = rng.integers(0, 256, (H, N, D // 2), dtype=np.uint8)
    s = (rng.random((H, N, D // gs)) + 0.1).astype(np.float16)
    z = (rng.standard_normal((H, N, D // gs)) + 0.5).astype(np.float16)
    tile = oleg.dequant_int4_tile(packed, s, z, D, gs)
    for h in range(H):
        flat = oleg.dequantize_packed(packed[h].reshape(-1), s[h], z[h], 4, gs, N, D)
        np.testing.assert_array_equal(tile[h], flat)


# ----------------------------------------------------- fused_quantize_evict

def _evict_bruteforce(x: np.ndarray, bits: int, gs: int):
    """quantize_tensor of fused_quantize_evict in the input dtype: each op rounded
    to fp16 (or fp32), clamp(min=1e-8) as the dtype sees it, code = the nearest
    level to f(f(x - min) / scale) (0/0 -> NaN -> 0)."""
    maxv = (1 << bits) - 1
    rnd = f16 if x.dtype == np.float16 else f32
    n, D = x.shape
    G = -(-D // gs)
    lo = rnd(Fraction(1e-8))
    codes = np.zeros((n, G * gs), np.int64)
    sc = np.zeros((n, G))
    zr = np.zeros((n, G))
    for r in range(n):
        vals = [frac(v) for v in x[r]] + [Fraction(0)] * (G * gs - D)
        for g in range(G):
            grp = vals[g * gs:(g + 1) * gs]
            mn, mx = min(grp), max(grp)
            s = max(rnd(rnd(mx - mn) / maxv), lo)
            for j, v in enumerate(grp):
                d = rnd(v - mn)
                if s == 0:
                    q = float("nan") if d == 0 else float("inf")
                else:
                    q = rnd(d / s)
                codes[r, g * gs + j] = nearest_level(q, maxv)
            sc[r, g], zr[r, g] = float(s), float(mn)
    return codes, sc, zr


def _evict_pack_ref(codes: np.ndarray, bits: int) -> np.ndarray:
    n = codes.shape[0]
    if bits in (2, 4):
        return np.stack([pack_bits_msb(codes[r], bits, 8 // bits) for r in range(n)])
    return codes.astype(np.uint8)


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
@pytest.mark.parametrize("D,gs", [(64, 64), (64, 32), (64, 128), (48, 32)])
def test_quantize_evict_bruteforce(bits, D, gs):
    rng = np.random.default_rng(bits * 31 + D + gs)
    keys = (rng.standard_normal((12, D)) * 2).astype(np.float16)
    vals = (rng.standard_normal((12, D)) * 0.3).astype(np.float16)
    keys[3] = np.float16(0.75)  # a constant row: scale 0 -> NaN -> code 0
    mask = rng.random(12) < 0.6
    mask[3] = True
    kp, ks, kz, vp, vs, vz = oleg.quantize_evict(keys, vals, mask, bits, gs)
    for src, p, s, z in ((keys, kp, ks, kz), (vals, vp, vs, vz)):
        codes, sc, zr = _evict_bruteforce(src[mask], bits, gs)
        np.testing.assert_array_equal(p, _evict_pack_ref(codes, bits))
        np.testing.assert_array_equal(s.astype(np.float64), sc)
        np.testing.assert_array_equal(z.astype(np.float64), zr)
        assert s.dtype == np.float16


def test_quantize_evict_fp16_arithmetic_differs_from_fp32():
    """A block whose fp16 codes differ from fp32 arithmetic: the oracle follows fp16."""
    rng = np.random.default_rng(11)
    hits = 0
    for _ in range(200):
        x = (rng.standard_normal((1, 32)) * 7).astype(np.float16)
        _, _, _, vp, _, _ = oleg.quantize_evict(x, x, np.array([True]), 8, 32)
        c32 = np.rint((x.astype(np.float32) - x.min()) / ((np.float32(x.max()) - np.float32(x.min())) / 255))
        hits += int(np.any(vp.astype(np.int64) != np.clip(c32, 0, 255).astype(np.int64)))
        codes, _, _ = _evict_bruteforce(x, 8, 32)
        np.testing.assert_array_equal(vp, codes.astype(np.uint8))
    assert hits > 0


def test_quantize_evict_empty():
    keys = np.zeros((4, 64), np.float16)
    out = oleg.quantize_evict(keys, keys, np.zeros(4, bool), 4, 64)
    assert all(o.size == 0 for o in out)


# ----------------------------------------------------------- PackedKVArena

def _bf16(x: Fraction) -> Fraction:
    from exact_fp import rne
    return rne(x, 7, -126, 127)


def _arena_bruteforce(x: np.ndarray, bits: int, gs: int, dt: str):
    """quantize_and_append's arithmetic with exact rounding: every op rounded to the
    input dtype, clamp(min=1e-10) as that dtype sees it, the nearest level to
    rnd(rnd(x - min) / scale) (0/0 -> NaN -> 0), padding channels dropped."""
    maxv = (1 << bits) - 1
    rnd = {"float16": f16, "bfloat16": _bf16, "float32": f32}[dt]
    H, N, D = x.shape
    G = -(-D // gs)
    lo = rnd(Fraction(1e-10))
    codes = np.zeros((H, N, D), np.int64)
    sc = np.zeros((H, N, G))
    zr = np.zeros((H, N, G))
    for h in range(H):
        for n in range(N):
            vals = [frac(v) for v in x[h, n]] + [Fraction(0)] * (G * gs - D)
            for g in range(G):
                grp = vals[g * gs:(g + 1) * gs]
                mn, mx = min(grp), max(grp)
                s = max(rnd(rnd(mx - mn) / maxv), lo)
                for j, v in enumerate(grp):
                    c = g * gs + j
                    if c >= D:
                        break
                    d = rnd(v - mn)
                    q = (float("nan") if d == 0 else float("inf")) if s == 0 else rnd(d / s)
                    codes[h, n, c] = nearest_level(q, maxv)
                sc[h, n, g], zr[h, n, g] = float(s), float(mn)
    return codes, sc, zr


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("dt", ["float16", "bfloat16", "float32"])
@pytest.mark.parametrize("D,gs", [(64, 64), (64, 32), (64, 128), (128, 128)])
def test_arena_quantize_bruteforce(bits, dt, D, gs):
    from oracle.fp import to_dtype
    rng = np.random.default_rng(bits * 7 + D + gs + len(dt))
    x = to_dtype((rng.standard_normal((2, 3, D)) * 1.7).astype(np.float32), dt).astype(np.float32)
    x[1, 2] = np.float32(0.375)  # a constant token: scale 0 -> the 1e-10 clamp (bf16 / fp32) or NaN -> 0 (fp16)
    p, s, z = oleg.arena_quantize(x, bits, gs, dt=dt, store="float32")
    codes, sc, zr = _arena_bruteforce(x, bits, gs, dt)
    per_byte = 8 // bits
    ref = np.stack([np.stack([pack_bits_msb(codes[h, n], bits, per_byte) if bits < 8 else codes[h, n].astype(np.uint8)
                              for n in range(x.shape[1])]) for h in range(x.shape[0])])
    np.testing.assert_array_equal(p, ref)
    np.testing.assert_array_equal(s.astype(np.float64), sc)
    np.testing.assert_array_equal(z.astype(np.float64), zr)
    assert p.shape == (2, 3, D * bits // 8)
    if dt != "float16":
        assert s[1, 2, 0] > 0  # the clamp took the constant token's scale off zero


def test_arena_dequantize_closed_form():
    """u * s + z with both ops rounded to fp32 and the sum cast to fp16, for every
    code of every width against float64 evaluation of the same steps."""
    rng = np.random.default_rng(3)
    for bits in (2, 4, 8):
        maxv = (1 << bits) - 1
        D, gs = 64, 32
        codes = rng.integers(0, maxv + 1, (2, 5, D))
        codes[0, 0, : maxv + 1 if maxv < D else D] = np.arange(min(maxv + 1, D))
        packed = oleg.arena_pack(codes.astype(np.uint8), bits)
        s = (rng.random((2, 5, 2)) * 0.3).astype(np.float16)
        z = (rng.standard_normal((2, 5, 2))).astype(np.float16)
        got = oleg.arena_dequantize(packed, s, z, bits, gs, D)
        gi = np.arange(D) // gs
        prod = (codes * s.astype(np.float64)[..., gi]).astype(np.float32)  # exact: <= 19 significant bits
        want = (prod.astype(np.float64) + z.astype(np.float64)[..., gi]).astype(np.float32).astype(np.float16)
        np.testing.assert_array_equal(got, want)
        np.testing.assert_array_equal(oleg.arena_unpack(packed, bits, D), codes.astype(np.float32))


def test_arena_matches_quantize_evict_on_fp16():
    """On fp16 inputs the two clamps (1e-8, 1e-10) both round to 0, so the arena's
    codes, scales and zeros equal fused_quantize_evict's row by row (D a multiple of
    the group size: no padding to drop)."""
    rng = np.random.default_rng(9)
    x = (rng.standard_normal((3, 7, 128)) * 2).astype(np.float16)
    for bits, gs in ((4, 128), (2, 32), (8, 64)):
        p, s, z = oleg.arena_quantize(x, bits, gs)
        kp, ks, kz, _, _, _ = oleg.quantize_evict(x.reshape(-1, 128), x.reshape(-1, 128), np.ones(21, bool), bits, gs)
        np.testing.assert_array_equal(p.reshape(21, -1), kp)
        np.testing.assert_array_equal(s.reshape(21, -1), ks)
        np.testing.assert_array_equal(z.reshape(21, -1), kz)
