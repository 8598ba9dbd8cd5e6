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
    assert lib.akv_stream_read(None, 24, None, None) == nat.AKV_E_SHAPE  # not a multiple of 16
    assert lib.akv_stream_read(None, 32, None, None) == nat.AKV_E_INVALID
    assert lib.akv_stream_read(ctypes.c_void_p(8), 32, ctypes.c_void_p(16), None) == nat.AKV_E_ALIGN
    assert lib.akv_stream_read(None, 0, None, None) == nat.AKV_OK
    # the normal build records no decode timeline (the timeline build does: make timeline)
    assert lib.akv_timeline_words() == 0
    assert lib.akv_timeline_fetch(None, 0) == nat.AKV_E_UNSUPPORTED
    assert lib.akv_timeline_clear(None) == nat.AKV_E_UNSUPPORTED


def test_decode_shape_checks():
    from akv import _native as nat
    lib = nat.load()
    a = nat.DecodeArgs()
    a.abi_version = nat.ABI_VERSION
    a.q_dtype = nat.DT_F16
    a.B, a.Hq, a.Hkv, a.M, a.D = 1, 12, 5, 1, 128
    a.n_hot = 4
    a.sm_scale = 128 ** -0.5
    assert lib.akv_decode_workspace_bytes(ctypes.byref(a)) == -1
    assert b"multiple of Hkv" in lib.akv_last_error()
    a.Hkv, a.D = 2, 96
    assert lib.akv_decode_workspace_bytes(ctypes.byref(a)) == -1
    assert b"head_dim" in lib.akv_last_error()
    # weights buffers take 16-byte accesses (host-side check; pointers never dereferenced)
    a.D = 128
    a.q = a.out = a.k_hot = a.v_hot = 0x10000
    a.attn_weights = 0x10004
    assert lib.akv_decode_workspace_bytes(ctypes.byref(a)) == -1
    assert b"attn_weights must be 16-byte aligned" in lib.akv_last_error()
    a.attn_weights = 0x10010
    assert lib.akv_decode_workspace_bytes(ctypes.byref(a)) > 0
    # the online softmax needs a positive, finite scale
    for bad in (0.0, -0.1, float("inf"), float("nan")):
        a.sm_scale = bad
        assert lib.akv_decode_workspace_bytes(ctypes.byref(a)) == -1
        assert b"sm_scale must be positive" in lib.akv_last_error()
    b = _prefill_args(nat, sm_scale=-1.0)
    assert lib.akv_prefill_workspace_bytes(ctypes.byref(b)) == -1
    assert b"sm_scale must be positive" in lib.akv_last_error()


def test_legacy_warm_heads_and_strides():
    """A legacy tier is shared (1), per kv head (Hkv) or per (batch, kv head) (B * Hkv);
    a token stride below n_warm is refused, and one above it needs a forced branch
    (the symmetric-branch detection reads dense rows)."""
    from akv import _native as nat
    lib = nat.load()
    a = nat.DecodeArgs()
    a.abi_version = nat.ABI_VERSION
    a.q_dtype = nat.DT_F16
    a.B, a.Hq, a.Hkv, a.M, a.D = 3, 8, 4, 1, 128
    a.sm_scale = 128 ** -0.5
    a.q = a.out = 0x10000  # host-side checks only: never dereferenced
    w = a.warm
    w.kind = nat.WARM_LEGACY
    w.bits_k = w.bits_v = 4
    w.n_warm = 100
    w.k_codes = w.v_codes = w.k_scale = w.k_zero = w.v_scale = w.v_zero = 0x20000
    w.group_size, w.meta_dtype, w.legacy_sym = 64, nat.DT_F16, 0
    for heads, ok in ((1, True), (4, True), (12, True), (3, False), (8, False)):
        w.warm_heads = heads
        assert (lib.akv_decode_workspace_bytes(ctypes.byref(a)) > 0) == ok, heads
    w.warm_heads = 12
    w.token_stride = 99
    assert lib.akv_decode_workspace_bytes(ctypes.byref(a)) == -1 and b"token_stride" in lib.akv_last_error()
    w.token_stride = 128
    assert lib.akv_decode_workspace_bytes(ctypes.byref(a)) > 0
    w.legacy_sym = -1
    assert lib.akv_decode_workspace_bytes(ctypes.byref(a)) == -1 and b"force legacy_sym" in lib.akv_last_error()


@pytest.mark.parametrize("B,Hq,Hkv,M", [(1, 12, 2, 1), (8, 12, 2, 1), (4, 32, 32, 1), (2, 12, 2, 3), (3, 64, 2, 1),
                                          (2, 2, 2, 9)])
def test_decode_counter_region(B, Hq, Hkv, M):
    """The split arrival counters are the workspace's first bytes: 8 bytes per
    (batch, kv-head, 16-row chunk), rounded up to 256, inside the workspace."""
    from akv import _native as nat
    lib = nat.load()
    a = nat.DecodeArgs()
    a.abi_version = nat.ABI_VERSION
    a.q_dtype = nat.DT_F16
    a.B, a.Hq, a.Hkv, a.M, a.D = B, Hq, Hkv, M, 128
    a.q = a.out = a.k_hot = a.v_hot = 0x10000  # host-side planning only: never dereferenced
    a.n_hot = 512
    a.sm_scale = 128 ** -0.5
    nchunk = -(-(Hq // Hkv * M) // 16)
    expect = -(-(B * Hkv * nchunk * 8) // 256) * 256
    assert lib.akv_decode_counter_bytes(ctypes.byref(a)) == expect
    assert lib.akv_decode_workspace_bytes(ctypes.byref(a)) > expect
    a.scores, a.n_scores, a.decay = 0x20000, 512, 0.9  # the logit stash comes after the counters
    assert lib.akv_decode_counter_bytes(ctypes.byref(a)) == expect
    a.Hkv = 5  # invalid shapes are refused the same way as by the workspace query
    assert lib.akv_decode_counter_bytes(ctypes.byref(a)) == -1


def test_noalloc_limits_checked_before_any_launch():
    """akv_decode_attn_noalloc refuses requests beyond its scratch on the host
    (pointers are never dereferenced: the call returns before any HIP call)."""
    from akv import _native as nat
    lib = nat.load()
    a = nat.DecodeArgs()
    a.abi_version = nat.ABI_VERSION
    a.q_dtype = nat.DT_F16
    a.B, a.Hq, a.Hkv, a.M, a.D = 8, 12, 2, 1, 128
    a.q = a.out = a.k_hot = a.v_hot = 0x10000
    a.n_hot = 65536  # logit stash 8 * 12 * 65536 * 4 B = 24 MiB > 16 MiB
    a.scores, a.n_scores, a.decay = 0x20000, 65536, 0.9
    a.sm_scale = 128 ** -0.5
    assert lib.akv_decode_workspace_bytes(ctypes.byref(a)) > nat.NOALLOC_SCRATCH_BYTES
    assert lib.akv_decode_attn_noalloc(ctypes.byref(a), None) == nat.AKV_E_WORKSPACE
    assert b"no-allocation entry point holds 16777216" in lib.akv_last_error()
    # more (batch, kv-head, row chunk) counters than the counter region holds
    a.B, a.Hq, a.Hkv, a.n_hot, a.scores, a.n_scores = 4096, 4, 4, 16, None, 0
    assert lib.akv_decode_attn_noalloc(ctypes.byref(a), None) == nat.AKV_E_WORKSPACE
    assert b"split counters" in lib.akv_last_error()


def _prefill_args(nat, **kw):
    a = nat.PrefillArgs()
    a.abi_version = nat.ABI_VERSION
    a.B, a.Hq, a.Hkv, a.M, a.D = 1, 64, 8, 512, 128
    a.q_dtype = nat.DT_BF16
    a.q = a.out = a.k_hot = a.v_hot = 0x10000  # host-side checks only: never dereferenced
    a.n_hot = 4096
    a.sm_scale = 128 ** -0.5
    a.warm.kind = nat.WARM_AFFINE
    a.warm.bits_k = a.warm.bits_v = 2
    a.warm.n_warm = 126976
    a.warm.block_t, a.warm.group_v = 32, 32
    a.warm.k_codes = a.warm.v_codes = a.warm.k_scale = a.warm.k_zero = a.warm.v_scale = a.warm.v_zero = 0x20000
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def test_prefill_planning_and_checks():
    from akv import _native as nat
    lib = nat.load()
    a = _prefill_args(nat)
    # 128k workload: 32 row tiles x 8 kv-heads x 2 token splits = two workgroups per CU
    assert lib.akv_prefill_workspace_bytes(ctypes.byref(a)) == 8 * 256 * 2 * 16 * 132 * 4
    a = _prefill_args(nat, num_splits=1)
    assert lib.akv_prefill_workspace_bytes(ctypes.byref(a)) == 0
    # a short chunk splits the cache: partials of (B*Hkv*ceil(R/16)) chunks x splits x 16 rows x (D+4) fp32
    a = _prefill_args(nat, M=16)
    nb = lib.akv_prefill_workspace_bytes(ctypes.byref(a))
    assert nb > 0 and nb % 256 == 0
    assert nb >= 1 * 8 * 8 * 2 * 16 * 132 * 4
    a = _prefill_args(nat, D=64)
    assert lib.akv_prefill_workspace_bytes(ctypes.byref(a)) == -1
    assert b"head_dim 128" in lib.akv_last_error()
    a = _prefill_args(nat, q_dtype=nat.DT_F32)
    assert lib.akv_prefill_attn(ctypes.byref(a), None) == nat.AKV_E_DTYPE
    a = _prefill_args(nat)
    a.warm.block_t = 16
    assert lib.akv_prefill_attn(ctypes.byref(a), None) == nat.AKV_E_UNSUPPORTED
    a = _prefill_args(nat)
    a.warm.n_out = 1
    assert lib.akv_prefill_attn(ctypes.byref(a), None) == nat.AKV_E_UNSUPPORTED
    a = _prefill_args(nat, M=16, num_splits=3)
    assert lib.akv_prefill_attn(ctypes.byref(a), None) == nat.AKV_E_WORKSPACE


def test_prefill_chunk_kv_checks():
    """The chunk's own K / V (causal part) come as a pair, 16-byte aligned, and
    alone are enough tokens to attend to; their tiles join the token splits."""
    from akv import _native as nat
    lib = nat.load()
    a = _prefill_args(nat, k_chunk=0x30000)
    assert lib.akv_prefill_workspace_bytes(ctypes.byref(a)) == -1
    assert b"k_chunk and v_chunk go together" in lib.akv_last_error()
    a = _prefill_args(nat, k_chunk=0x30000, v_chunk=0x30008)
    assert lib.akv_prefill_attn(ctypes.byref(a), None) == nat.AKV_E_ALIGN
    a = _prefill_args(nat, n_hot=0)
    a.warm.kind = nat.WARM_NONE
    assert lib.akv_prefill_workspace_bytes(ctypes.byref(a)) == -1
    assert b"no tokens" in lib.akv_last_error()
    a = _prefill_args(nat, n_hot=0, k_chunk=0x30000, v_chunk=0x40000)
    a.warm.kind = nat.WARM_NONE
    assert lib.akv_prefill_workspace_bytes(ctypes.byref(a)) >= 0
    a = _prefill_args(nat, k_chunk=0x30000, v_chunk=0x40000)
    assert lib.akv_prefill_workspace_bytes(ctypes.byref(a)) >= 0
