"""The fast quantize kernel replaces the reference's fp16 division by a fused
multiply with an fp32 reciprocal and an fp16 add of 1024 for the rounding; the
C program in tests/exhaustive/ enumerates fp16 inputs and checks that scales
and codes equal the reference's (every scale with AKV_EXHAUSTIVE=1, every 7th
otherwise).  A mutated copy (reciprocal rounded to fp16 first) must fail, so
the check can catch a wrong code path."""
import os
import subprocess
import tempfile

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "exhaustive", "quant_reciprocal.c")


def _build(tmp, src_text=None):
    src = SRC
    if src_text is not None:
        src = os.path.join(tmp, "mut.c")
        open(src, "w").write(src_text)
    exe = os.path.join(tmp, "qr")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-o", exe, src, "-lm"], check=True)
    return exe


def test_fp16_rounding_of_the_check_matches_numpy():
    import numpy as np
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.standard_normal(3000) * 10.0 ** rng.integers(-9, 5, 3000),
                        [65503.9, 65504.0, 65519.99, 65520.0, 1e6, 2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -24 * 1.5,
                         1024.5, 1025.5, 2048.0 + 1.0, -0.0, 0.0]])
    with tempfile.TemporaryDirectory() as tmp:
        r = subprocess.run([_build(tmp), "round"], input="\n".join(float(v).hex() for v in x),
                           capture_output=True, text=True, timeout=60)
    got = np.array([float.fromhex(line) for line in r.stdout.split()])
    with np.errstate(over="ignore"):  # 65520 and 1e6 overflow to inf on purpose
        exp = x.astype(np.float16).astype(np.float64)
    np.testing.assert_array_equal(got, exp)


def test_reciprocal_code_path_matches_division():
    stride = "1" if os.environ.get("AKV_EXHAUSTIVE") else "7"
    with tempfile.TemporaryDirectory() as tmp:
        r = subprocess.run([_build(tmp), stride], capture_output=True, text=True, timeout=1200)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "scale mismatches 0; code mismatches 0" in r.stdout


def test_check_catches_a_wrong_code_path():
    text = open(SRC).read().replace("const float r = 1.0f / s;", "const float r = (float)rnd16(1.0f / s);")
    with tempfile.TemporaryDirectory() as tmp:
        r = subprocess.run([_build(tmp, text), "97"], capture_output=True, text=True, timeout=600)
    assert r.returncode == 1 and "code mismatches 0" not in r.stdout
