"""Write tests/golden/kat.json: known-answer vectors derived from first principles.

Nothing here uses the oracle or the reference code.  Every value comes from
exact rational arithmetic (fractions.Fraction) with IEEE-754 binary16
round-to-nearest-even implemented below, or from the bit layouts written out
position by position:

  * bitpack: the byte KATs of the layout (4-bit [3,7]->0x37, [1,15]->0x1F;
    2-bit [0,1,2,3]->0x1B; 3-bit [1..7,0] -> 0x29 0xCB 0xB8) plus vectors
    packed bit by bit from the stated bit positions;
  * affine quantize: K blocks (per channel over tokens) and V rows (per token)
    whose codes depend on each fp16 rounding of the reference's op sequence
    (mx-mn, /maxv, x-zero, /scale, round-half-even); includes a constant
    channel (scale 0 -> NaN -> code 0), a subnormal scale that makes x/scale
    overflow to +inf (-> maxv), a tie that rounds to even, and a block whose
    codes differ from plain fp32 arithmetic;
  * dequant: codes*scale and +zero each rounded to fp16;
  * importance: ones(32)*0.5 + 0 (decay KAT of the reference's tests) and a
    small sum-over-queries case.

Run: python tests/golden/make_kat.py  (rewrites kat.json next to this file)
"""
from __future__ import annotations

import json
import math
import os
import random
from fractions import Fraction as F

HERE = os.path.dirname(os.path.abspath(__file__))

# ----------------------------------------------------------------- binary16

MANT = 10
EMIN = -14
MAXF16 = F(65504)


def rnd16(x):
    """Round a Fraction (or inf/nan float) to the nearest binary16 value, ties to even."""
    if isinstance(x, float):
        return x
    if x == 0:
        return F(0)
    sign = -1 if x < 0 else 1
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if F(2) ** e > a:
        e -= 1
    e = max(e, EMIN)
    ulp = F(2) ** (e - MANT)
    q = a / ulp
    n = q.numerator // q.denominator
    rem = q - n
    if rem > F(1, 2) or (rem == F(1, 2) and n % 2 == 1):
        n += 1
    r = n * ulp
    if r > MAXF16:
        return sign * math.inf
    return sign * r


def f16_bits(v) -> int:
    """binary16 bit pattern of an exactly representable value."""
    if isinstance(v, float):
        if math.isnan(v):
            return 0x7E00
        return 0x7C00 if v > 0 else 0xFC00
    if v == 0:
        return 0
    s = 0x8000 if v < 0 else 0
    a = abs(v)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if F(2) ** e > a:
        e -= 1
    if e < EMIN:  # subnormal
        m = a / (F(2) ** (EMIN - MANT))
        assert m.denominator == 1
        return s | int(m)
    m = a / (F(2) ** (e - MANT))
    assert m.denominator == 1
    return s | ((e + 15) << MANT) | (int(m) - (1 << MANT))


def from_bits(b: int):
    s = -1 if b & 0x8000 else 1
    e = (b >> MANT) & 0x1F
    m = b & 0x3FF
    if e == 0:
        return s * F(m) * F(2) ** (EMIN - MANT)
    return s * (F(1 << MANT) + m) * F(2) ** (e - 15 - MANT)


def div(a, b):
    if isinstance(a, float) or isinstance(b, float):
        raise ValueError
    if b == 0:
        return math.nan if a == 0 else (math.inf if a > 0 else -math.inf)
    return a / b


def code_of(x, zero, scale, maxv):
    d = rnd16(x - zero)
    q = div(d, scale)
    if isinstance(q, float):
        if math.isnan(q):
            return 0
        return maxv if q > 0 else 0
    q = rnd16(q)
    if isinstance(q, float):
        return maxv if q > 0 else 0
    n = math.floor(q)
    r = q - n
    if r > F(1, 2) or (r == F(1, 2) and n % 2 == 1):
        n += 1
    return min(max(n, 0), maxv)


def group_quant(vals, bits):
    """One min/max group: (scale, zero, codes) with the reference's fp16 op sequence."""
    maxv = (1 << bits) - 1
    mn, mx = min(vals), max(vals)
    scale = rnd16(div(rnd16(mx - mn), F(maxv)))  # clamp(min=1e-8) is 0 in fp16
    zero = mn
    return scale, zero, [code_of(x, zero, scale, maxv) for x in vals]


def code_fp32_plain(x, zero, scale_exact, maxv):
    q = (x - zero) / scale_exact if scale_exact else None
    if q is None:
        return 0
    n = math.floor(q)
    r = q - n
    if r > F(1, 2) or (r == F(1, 2) and n % 2 == 1):
        n += 1
    return min(max(n, 0), maxv)


def deq(c, s, z):
    return rnd16(rnd16(F(c) * s) + z)


# ------------------------------------------------------------------ packing

def pack_bits(codes, bits):
    """Bit-position packer: code i of a row occupies the stated bit positions."""
    if bits == 4:
        n = len(codes) + len(codes) % 2
        c = list(codes) + [0] * (n - len(codes))
        out = [0] * (n // 2)
        for i, v in enumerate(c):  # even index -> bits 7..4, odd -> bits 3..0
            out[i // 2] |= (v & 15) << (4 if i % 2 == 0 else 0)
        return out
    if bits == 2:
        n = -(-len(codes) // 4) * 4
        c = list(codes) + [0] * (n - len(codes))
        out = [0] * (n // 4)
        for i, v in enumerate(c):  # position i%4 -> bits (7-2p)..(6-2p)
            out[i // 4] |= (v & 3) << (6 - 2 * (i % 4))
        return out
    n = -(-len(codes) // 8) * 8
    c = list(codes) + [0] * (n - len(codes))
    bitstream = []
    for v in c:  # 3 bits per code, most significant first, 8 codes per 24-bit word
        bitstream += [(v >> 2) & 1, (v >> 1) & 1, v & 1]
    out = []
    for i in range(0, len(bitstream), 8):
        byte = 0
        for bit in bitstream[i:i + 8]:
            byte = (byte << 1) | bit
        out.append(byte)
    return out


def main():
    rnd = random.Random(20261201)
    kat = {}
    bp = [
        {"bits": 4, "codes": [3, 7], "bytes": [0x37]},
        {"bits": 4, "codes": [1, 15], "bytes": [0x1F]},
        {"bits": 2, "codes": [0, 1, 2, 3], "bytes": [0x1B]},
        {"bits": 3, "codes": [1, 2, 3, 4, 5, 6, 7, 0], "bytes": [0x29, 0xCB, 0xB8]},
    ]
    for case in bp:
        assert pack_bits(case["codes"], case["bits"]) == case["bytes"], case
    for bits, n in ((4, 11), (3, 13), (2, 12), (3, 24), (4, 16)):
        codes = [rnd.randrange(1 << bits) for _ in range(n)]
        bp.append({"bits": bits, "codes": codes, "bytes": pack_bits(codes, bits)})
    kat["bitpack"] = bp

    # ---- K block: channels (columns) over tokens (rows), fp16 values as bit patterns
    def f16(x):
        return rnd16(F(x))

    chans = [
        [f16(0.0), f16(1.0), f16(2.0), f16(7.0)],            # exact scale 1
        [f16(-1.0), f16(0.25), f16(0.5), f16(2.5)],          # 1.25/0.5 = 2.5 -> tie -> 2
        [f16(3.0), f16(3.0), f16(3.0), f16(3.0)],            # constant -> scale 0 -> codes 0
        [from_bits(0x0000), from_bits(0x0001), from_bits(0x0000), from_bits(0x0001)],  # subnormal range
        [f16(0.1), f16(0.7), f16(-0.3), f16(1.3)],
    ]
    # a channel whose codes differ from fp32 arithmetic (found by a seeded search)
    for _ in range(100000):
        vals = [rnd16(F(rnd.uniform(-3, 3))) for _ in range(4)]
        s, z, c16 = group_quant(vals, 3)
        exact_scale = (max(vals) - min(vals)) / 7
        c32 = [code_fp32_plain(x, z, exact_scale, 7) for x in vals]
        if c16 != c32:
            chans.append(vals)
            break
    else:
        raise RuntimeError("no distinguishing channel found")
    kblk = []
    for bits in (2, 3, 4):
        ch_out = []
        for vals in chans:
            s, z, codes = group_quant(vals, bits)
            ch_out.append({
                "x": [f16_bits(x) for x in vals],
                "scale": f16_bits(s), "zero": f16_bits(z), "codes": codes,
                "deq": [f16_bits(deq(c, s, z)) for c in codes],
            })
        kblk.append({"bits": bits, "channels": ch_out})
    kat["affine_groups"] = kblk
    # the subnormal channel: (mx-mn)/7 underflows to 0 while x-zero > 0 -> +inf -> maxv
    sub = kblk[1]["channels"][3]
    assert sub["scale"] == 0 and sub["codes"] == [0, 7, 0, 7], sub
    assert kblk[1]["channels"][2]["codes"] == [0, 0, 0, 0]
    assert kblk[1]["channels"][1]["codes"][1] == 2  # tie to even

    kat["importance"] = {
        "decay_kat": {"scores": [1.0] * 32, "decay": 0.5, "expect": [0.5] * 32},
        "sum_over_queries": {
            "attn": [[[[0.5, 0.25, 0.25], [0.0, 1.0, 0.0]]], [[[0.25, 0.5, 0.25], [1.0, 0.0, 0.0]]]],
            "scores": [0.0, 1.0, 2.0], "decay": 0.5,
            # mean over (b, h) then sum over the two queries
            "expect": [0.0 * 0.5 + (0.5 + 0.25) / 2 + (0.0 + 1.0) / 2,
                       1.0 * 0.5 + (0.25 + 0.5) / 2 + (1.0 + 0.0) / 2,
                       2.0 * 0.5 + (0.25 + 0.25) / 2 + 0.0],
        },
    }
    kat["legacy_pack"] = {
        "4bit": {"codes": [3, 7, 1, 15, 0, 8], "bytes": [0x37, 0x1F, 0x08]},
        "2bit": {"codes": [0, 1, 2, 3, 1, 0, 3, 2], "bytes": [0x1B, 0x4E]},
    }
    with open(os.path.join(HERE, "kat.json"), "w") as f:
        json.dump(kat, f, indent=1)
    print("wrote", os.path.join(HERE, "kat.json"))


if __name__ == "__main__":
    main()
