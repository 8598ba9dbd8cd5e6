"""ctypes binding of libakv_hip.so (the C ABI declared in include/akv_hip.h).

The library is built in-tree (``adaptive-kv-memory_amd/csrc/Makefile``) and
loaded from this directory.  There is no fallback: if the library is missing,
or a tensor is not on a ROCm device, the ops raise.
"""
from __future__ import annotations

import ctypes
import math
import os
from typing import Optional

import torch

ABI_VERSION = 5

AKV_OK = 0
AKV_E_INVALID = -1
AKV_E_BITS = -2
AKV_E_SHAPE = -3
AKV_E_ALIGN = -4
AKV_E_DTYPE = -5
AKV_E_WORKSPACE = -6
AKV_E_UNSUPPORTED = -7
AKV_E_HIP = -8
AKV_E_ABI = -9

DT_F16, DT_BF16, DT_F32 = 0, 1, 2
# scratch limits of akv_decode_attn_noalloc (AKV_NOALLOC_* in include/akv_hip.h)
NOALLOC_SCRATCH_BYTES = 16 << 20
NOALLOC_COUNTER_BYTES = 64 << 10
WARM_NONE, WARM_AFFINE, WARM_LEGACY = 0, 1, 2
QUANT_AFFINE, QUANT_TOKEN_GROUPS, QUANT_KVQ, QUANT_ARENA = 0, 1, 2, 3

LIB_NAME = "libakv_hip.so"
# AKV_LIB names another build of the same library (for example one compiled with
# different tuning macros); by default the in-tree build next to this file loads.
LIB_PATH = os.environ.get("AKV_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64


class WarmDesc(ctypes.Structure):
    _fields_ = [
        ("kind", _i32), ("bits_k", _i32), ("bits_v", _i32),
        ("n_warm", _i64),
        ("block_t", _i32), ("group_v", _i32), ("n_out", _i32), ("_pad0", _i32),
        ("k_codes", _vp), ("v_codes", _vp),
        ("k_scale", _vp), ("k_zero", _vp), ("v_scale", _vp), ("v_zero", _vp),
        ("k_oidx", _vp), ("v_oidx", _vp),
        ("k_odata", _vp), ("v_odata", _vp),
        ("group_size", _i32), ("meta_dtype", _i32), ("warm_heads", _i32), ("legacy_sym", _i32),
        ("token_stride", _i64),
    ]


class DecodeArgs(ctypes.Structure):
    _fields_ = [
        ("abi_version", _i32), ("B", _i32), ("Hq", _i32), ("Hkv", _i32), ("M", _i32), ("D", _i32),
        ("q_dtype", _i32),
        ("q", _vp), ("k_hot", _vp), ("v_hot", _vp),
        ("n_hot", _i64),
        ("hot_first", _i32), ("sm_scale", ctypes.c_float),
        ("warm", WarmDesc),
        ("out", _vp), ("attn_weights", _vp), ("scores", _vp),
        ("n_scores", _i64),
        ("decay", ctypes.c_float), ("num_splits", _i32),
        ("workspace", _vp), ("workspace_bytes", _i64),
        ("hot_stride", _i64),
    ]


class PrefillArgs(ctypes.Structure):
    _fields_ = [
        ("abi_version", _i32), ("B", _i32), ("Hq", _i32), ("Hkv", _i32), ("M", _i32), ("D", _i32),
        ("q_dtype", _i32),
        ("q", _vp), ("k_hot", _vp), ("v_hot", _vp),
        ("n_hot", _i64),
        ("sm_scale", ctypes.c_float), ("num_splits", _i32),
        ("warm", WarmDesc),
        ("out", _vp),
        ("workspace", _vp), ("workspace_bytes", _i64),
        ("k_chunk", _vp), ("v_chunk", _vp),
    ]


class QuantArgs(ctypes.Structure):
    _fields_ = [
        ("abi_version", _i32), ("B", _i32), ("H", _i32), ("D", _i32),
        ("in_dtype", _i32), ("layout", _i32),
        ("k", _vp), ("v", _vp),
        ("n_src", _i64), ("sel", _vp), ("n_sel", _i64),
        ("bits_k", _i32), ("bits_v", _i32), ("block_t", _i32), ("group_v", _i32),
        ("n_out", _i32), ("symmetric", _i32),
        ("k_codes", _vp), ("k_scale", _vp), ("k_zero", _vp),
        ("v_codes", _vp), ("v_scale", _vp), ("v_zero", _vp),
        ("k_oidx", _vp), ("v_oidx", _vp), ("k_odata", _vp), ("v_odata", _vp),
    ]


class DequantArgs(ctypes.Structure):
    _fields_ = [
        ("abi_version", _i32), ("B", _i32), ("Hkv", _i32), ("D", _i32),
        ("out_dtype", _i32), ("_pad0", _i32),
        ("warm", WarmDesc),
        ("k_out", _vp), ("v_out", _vp), ("workspace", _vp),
        ("block_of_token", _vp), ("n_blocks", _i64),
        ("out_slot", _vp), ("out_tokens", _i64),
    ]


class ImportanceArgs(ctypes.Structure):
    _fields_ = [
        ("abi_version", _i32), ("attn_dtype", _i32),
        ("attn", _vp),
        ("B", _i64), ("H", _i64), ("M", _i64), ("N", _i64),
        ("scores", _vp), ("n_scores", _i64),
        ("decay", ctypes.c_float), ("q_window", _i32), ("pool_kernel", _i32), ("_pad0", _i32),
    ]


EXPORTS = (
    "akv_abi_version", "akv_last_error", "akv_struct_size",
    "akv_decode_workspace_bytes", "akv_decode_counter_bytes", "akv_decode_attn", "akv_decode_attn_noalloc",
    "akv_quant_pack", "akv_dequant_unpack",
    "akv_bitpack", "akv_bitunpack", "akv_importance_update",
    "akv_prefill_workspace_bytes", "akv_prefill_attn", "akv_select_demote", "akv_stream_read",
    "akv_timeline_words", "akv_timeline_fetch", "akv_timeline_clear",
)
STRUCTS = (WarmDesc, DecodeArgs, QuantArgs, DequantArgs, ImportanceArgs, PrefillArgs)

_lib: Optional[ctypes.CDLL] = None


def load() -> ctypes.CDLL:
    """Load libakv_hip.so (once).  Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `make -C adaptive-kv-memory_amd/csrc` "
            "(or __graft_entry__.build()); akv has no CPU fallback")
    lib = ctypes.CDLL(LIB_PATH)
    lib.akv_abi_version.restype = ctypes.c_int
    lib.akv_last_error.restype = ctypes.c_char_p
    lib.akv_struct_size.restype = _i64
    lib.akv_struct_size.argtypes = [_i32]
    lib.akv_decode_workspace_bytes.restype = _i64
    lib.akv_decode_workspace_bytes.argtypes = [ctypes.POINTER(DecodeArgs)]
    lib.akv_decode_counter_bytes.restype = _i64
    lib.akv_decode_counter_bytes.argtypes = [ctypes.POINTER(DecodeArgs)]
    lib.akv_decode_attn.restype = ctypes.c_int
    lib.akv_decode_attn.argtypes = [ctypes.POINTER(DecodeArgs), _vp]
    lib.akv_decode_attn_noalloc.restype = ctypes.c_int
    lib.akv_decode_attn_noalloc.argtypes = [ctypes.POINTER(DecodeArgs), _vp]
    lib.akv_quant_pack.restype = ctypes.c_int
    lib.akv_quant_pack.argtypes = [ctypes.POINTER(QuantArgs), _vp]
    lib.akv_dequant_unpack.restype = ctypes.c_int
    lib.akv_dequant_unpack.argtypes = [ctypes.POINTER(DequantArgs), _vp]
    lib.akv_bitpack.restype = ctypes.c_int
    lib.akv_bitpack.argtypes = [_vp, _vp, _i64, _i32, _i32, _vp]
    lib.akv_bitunpack.restype = ctypes.c_int
    lib.akv_bitunpack.argtypes = [_vp, _vp, _i64, _i32, _i32, _i32, _vp]
    lib.akv_importance_update.restype = ctypes.c_int
    lib.akv_importance_update.argtypes = [ctypes.POINTER(ImportanceArgs), _vp]
    lib.akv_prefill_workspace_bytes.restype = _i64
    lib.akv_prefill_workspace_bytes.argtypes = [ctypes.POINTER(PrefillArgs)]
    lib.akv_prefill_attn.restype = ctypes.c_int
    lib.akv_prefill_attn.argtypes = [ctypes.POINTER(PrefillArgs), _vp]
    lib.akv_select_demote.restype = ctypes.c_int
    lib.akv_select_demote.argtypes = [_vp, _i64, _i64, _i64, _i32, _i32, _vp, _vp]
    lib.akv_stream_read.restype = ctypes.c_int
    lib.akv_stream_read.argtypes = [_vp, _i64, _vp, _vp]
    lib.akv_timeline_words.restype = _i64
    lib.akv_timeline_words.argtypes = []
    lib.akv_timeline_fetch.restype = ctypes.c_int
    lib.akv_timeline_fetch.argtypes = [_vp, _i64]
    lib.akv_timeline_clear.restype = ctypes.c_int
    lib.akv_timeline_clear.argtypes = [_vp]
    if lib.akv_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{LIB_PATH} has ABI {lib.akv_abi_version()}, expected {ABI_VERSION}")
    for i, st in enumerate(STRUCTS):
        if lib.akv_struct_size(i) != ctypes.sizeof(st):
            raise RuntimeError(f"struct {st.__name__} layout mismatch with {LIB_PATH}")
    _lib = lib
    return lib


def check(rc: int, what: str = "akv") -> None:
    """Map a library status code to the exception type the reference raises."""
    if rc == AKV_OK:
        return
    msg = (load().akv_last_error() or b"").decode(errors="replace")
    if rc in (AKV_E_BITS, AKV_E_SHAPE, AKV_E_INVALID, AKV_E_ALIGN):
        raise ValueError(f"{what}: {msg}")
    if rc == AKV_E_DTYPE:
        raise TypeError(f"{what}: {msg}")
    if rc == AKV_E_UNSUPPORTED:
        raise NotImplementedError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg} (status {rc})")


# ------------------------------------------------------------------ helpers

_DT = {torch.float16: DT_F16, torch.bfloat16: DT_BF16, torch.float32: DT_F32}


def dtype_code(dt: torch.dtype) -> int:
    if dt not in _DT:
        raise TypeError(f"unsupported dtype {dt}")
    return _DT[dt]


def require_device(*tensors) -> None:
    """The MI355X build computes on ROCm devices only: no CPU path."""
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError("akv (MI355X build) runs on ROCm devices only; got a CPU tensor")


def dev_contig(t: Optional[torch.Tensor], dtype: Optional[torch.dtype] = None) -> Optional[torch.Tensor]:
    """Contiguous, 16-byte-aligned device tensor (copied if needed)."""
    if t is None:
        return None
    if dtype is not None and t.dtype != dtype:
        t = t.to(dtype)
    t = t.contiguous()
    if t.data_ptr() % 16:
        t = t.clone()
    return t


def ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def workspace(nbytes: int, device, zero_prefix: int = 0) -> torch.Tensor:
    """Device scratch for one call; its first ``zero_prefix`` bytes are zeroed (a decode
    workspace's split arrival counters must read zero when a call starts, and each call
    leaves them so; the rest needs no initial value)."""
    n = max(int(nbytes), 256)
    ws = torch.empty(n, dtype=torch.uint8, device=device)
    if zero_prefix > 0:
        ws[: min(int(zero_prefix), n)].zero_()
    return ws


class DecodeWorkspace:
    """A decode workspace reused across calls on one device and stream.

    A call needs its first ``counter_bytes`` bytes (the split arrival counters) at
    zero and leaves exactly those bytes at zero when it completes; the bytes after
    them hold its split partials.  So after a call only the prefix that call used is
    known to be zero: a later call with a smaller counter region writes partials over
    the tail of the larger one, and a call after that with the larger region must
    zero it again.  ``get`` keeps the last call's counter size (not the largest ever
    zeroed) and clears the prefix whenever a call needs more of it.  Calls that share
    one workspace must be ordered on one stream."""

    def __init__(self):
        self._buf: Optional[torch.Tensor] = None
        self._zero = 0  # bytes at the start known to be zero when the next call starts

    def get(self, nbytes: int, counter_bytes: int, device) -> torch.Tensor:
        buf = self._buf
        if buf is None or buf.numel() < nbytes or buf.device != torch.device(device):
            self._buf = buf = workspace(nbytes, device, zero_prefix=counter_bytes)
        elif counter_bytes > self._zero:
            buf[:counter_bytes].zero_()
        self._zero = int(counter_bytes)
        return buf


def default_sm_scale(d: int) -> float:
    return 1.0 / math.sqrt(d)
