"""The C ABI library loads and exports every entry point include/akv_hip.h
declares; the ctypes mirrors match the C structs; argument validation runs on
the host (no GPU needed) and maps to the reference's exception types."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "akv_hip.h")


def _declared():
    txt = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char \*)\s*\*?\s*(akv_\w+)\s*\(", txt, re.M)))


def test_library_exports_every_declared_symbol():
    from akv import _native as nat
    nat.load()
    out = subprocess.run(["nm", "-D", "--defined-only", nat.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (akv_\w+)", out))
    declared = _declared()
    assert declared, "no declarations parsed"
    missing = [s for s in declared if s not in exported]
    assert not missing, f"declared but not exported: {missing}"
    assert set(declared) == set(nat.EXPORTS)


def test_struct_layouts_match():
    from akv import _native as nat
    lib = nat.load()
    for i, st in enumerate(nat.STRUCTS):
        assert lib.akv_struct_size(i) == ctypes.sizeof(st), st.__name__
    assert lib.akv_struct_size(99) == -1
    assert lib.akv_abi_version() == nat.ABI_VERSION


def test_host_side_validation_without_gpu():
    from akv import _native as nat
    lib = nat.load()
    a = nat.DecodeArgs()
    a.abi_version = nat.ABI_VERSION
    assert lib.akv_decode_workspace_bytes(ctypes.byref(a)) == -1
    assert b"float16" in lib.akv_last_error() or lib.akv_last_error()
    a.abi_version = 99
    assert lib.akv_decode_attn(ctypes.byref(a), None) == nat.AKV_E_ABI
    q = nat.QuantArgs()
    q.abi_version = nat.ABI_VERSION
    q.B, q.H, q.D, q.n_src, q.n_sel = 1, 1, 128, 4, 4
    q.bits_k, q.bits_v, q.block_t, q.group_v = 5, 3, 32, 32
    assert lib.akv_quant_pack(ctypes.byref(q), None) == nat.AKV_E_BITS
    assert b"Unsupported bits: 5" in lib.akv_last_error()
    with pytest.raises(ValueError, match="Unsupported bits"):
        nat.check(nat.AKV_E_BITS, "x")
    assert lib.akv_bitpack(None, None, 1, 8, 7, None) == nat.AKV_E_BITS
    assert lib.akv_bitunpack(None, None, 1, 2, 9, 2, None) == nat.AKV_E_SHAPE


def test_decode_shape_checks():
    from akv import _native as nat
    lib = nat.load()
    a = nat.DecodeArgs()
    a.abi_version = nat.ABI_VERSION
    a.q_dtype = nat.DT_F16
    a.B, a.Hq, a.Hkv, a.M, a.D = 1, 12, 5, 1, 128
    a.n_hot = 4
    assert lib.akv_decode_workspace_bytes(ctypes.byref(a)) == -1
    assert b"multiple of Hkv" in lib.akv_last_error()
    a.Hkv, a.D = 2, 96
    assert lib.akv_decode_workspace_bytes(ctypes.byref(a)) == -1
    assert b"head_dim" in lib.akv_last_error()
