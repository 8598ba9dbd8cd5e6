"""The decode kernels split workgroup and lane ids into coordinates with
akv::fast_div (csrc/fastdiv.h: one high multiply, an add and a shift per
division by a run-time divisor).  The C++ program in tests/exhaustive/ checks it
against integer division over every divisor up to 65536 (dense n for the small
ones, quotient boundaries for all), divisors near every power of two and random
divisors up to 2^31; a mutated multiplier must be caught."""
import os
import subprocess
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "exhaustive", "fastdiv.cc")
CSRC = os.path.join(os.path.dirname(HERE), "adaptive-kv-memory_amd", "csrc")


def _run(tmp, header_dir=CSRC, *args):
    exe = os.path.join(tmp, "fd")
    subprocess.run(["g++", "-O2", "-std=c++17", "-I", header_dir, "-o", exe, SRC], check=True)
    return subprocess.run([exe, *args], capture_output=True, text=True, timeout=600)


def test_fast_div_equals_integer_division():
    with tempfile.TemporaryDirectory() as tmp:
        r = _run(tmp)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "mismatches 0" in r.stdout


def test_check_catches_a_wrong_multiplier():
    text = open(os.path.join(CSRC, "fastdiv.h")).read().replace(") / d) + 1;", ") / d);")
    assert text != open(os.path.join(CSRC, "fastdiv.h")).read()
    with tempfile.TemporaryDirectory() as tmp:
        open(os.path.join(tmp, "fastdiv.h"), "w").write(text)
        r = _run(tmp, tmp)
    assert r.returncode == 1 and "mismatches 0" not in r.stdout
