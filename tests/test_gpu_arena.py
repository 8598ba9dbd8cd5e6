"""PackedKVArena (akv/packed_layout.py:56-281) against the oracle: the packed
codes, scales and zeros of quantize_and_append bit-exact for 2/4/8 bits, fp16 /
bf16 / fp32 inputs and a head_dim below the group size; appends that overflow
evict the oldest tokens; dequantize_slice bit-exact; get_packed_slice views and
the byte accounting."""
import numpy as np
import pytest
import torch

from gpu_util import announce, bits_equal, to_dev
from oracle import legacy as oleg
from oracle.fp import BF16, F16, F32, to_dtype

pytestmark = pytest.mark.gpu

_DT = {torch.float16: F16, torch.bfloat16: BF16, torch.float32: F32}


def _keys(H, N, D, dtype, seed):
    """Seeded N(0, 1.5) keys in `dtype` (host copy as float32 holding those values),
    one channel x10 and one constant token per head."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((H, N, D)) * 1.5).astype(np.float32)
    x[:, :, 3] *= 10.0
    x[:, N // 2] = 0.625
    host = to_dtype(x, _DT[dtype]).astype(np.float32)
    return torch.from_numpy(host).to(dtype).cuda(), host


def _arena(H, S, D, bits, gs, dtype=torch.float16):
    from akv.packed_layout import PackedKVArena, PackedKVConfig
    return PackedKVArena(PackedKVConfig(max_seq_len=S, num_heads=H, head_dim=D, bits=bits, group_size=gs,
                                        device="cuda", dtype=dtype))


@pytest.mark.parametrize("bits,D,gs", [(4, 128, 128), (2, 128, 32), (8, 128, 64), (4, 64, 128), (2, 64, 128),
                                       (8, 64, 32)])
def test_quantize_and_append_matches_oracle(bits, D, gs):
    announce(f"arena append bits={bits} D={D} group={gs}")
    H, N = 8, 300
    arena = _arena(H, 512, D, bits, gs)
    k, host = _keys(H, N, D, torch.float16, seed=bits + D + gs)
    assert arena.quantize_and_append(k) == 0
    p, s, z = oleg.arena_quantize(host, bits, gs, dt=F16, store=F16)
    data, sc, ze = arena.get_packed_slice(0, N)
    bits_equal(data, p)
    bits_equal(sc, s)
    bits_equal(ze, z)
    assert arena.length == N
    assert bool(arena.valid[:N].all()) and not bool(arena.valid[N:].any())
    # the oracle's dequant of the same tier
    deq = arena.dequantize_slice(0, N)
    bits_equal(deq, oleg.arena_dequantize(p, s, z, bits, gs, D, store=F16))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_input_dtype_arithmetic_and_clamp(dtype):
    """bf16 / fp32 keys: every op in the input dtype, the constant token's scale
    clamped at 1e-10 as that dtype rounds it, scales stored as the arena's fp16."""
    announce(f"arena append {dtype}")
    H, N, D, bits, gs = 4, 96, 128, 4, 32
    arena = _arena(H, 128, D, bits, gs)
    k, host = _keys(H, N, D, dtype, seed=5)
    arena.quantize_and_append(k)
    p, s, z = oleg.arena_quantize(host, bits, gs, dt=_DT[dtype], store=F16)
    data, sc, ze = arena.get_packed_slice(0, N)
    bits_equal(data, p)
    bits_equal(sc, s)
    bits_equal(ze, z)


def test_overflow_evicts_oldest():
    """Capacity 100: appends of 30, 30, 30 fill 90; the next 30 evict the oldest 30
    (survivors shift to the front) and land at slot 60; an append of 70 into the 90
    held evicts 70; an append as large as the arena empties it first."""
    announce("arena eviction on overflow")
    H, D, bits, gs = 4, 128, 2, 64
    arena = _arena(H, 100, D, bits, gs)
    chunks = [_keys(H, n, D, torch.float16, seed=20 + i) for i, n in enumerate((30, 30, 30, 30, 70, 100))]
    ref = [oleg.arena_quantize(h, bits, gs) for _, h in chunks]
    starts = [arena.quantize_and_append(k) for k, _ in chunks[:4]]
    assert starts == [0, 30, 60, 60] and arena.length == 90
    for i, j in enumerate((1, 2, 3)):
        data, sc, ze = arena.get_packed_slice(30 * i, 30 * (i + 1))
        bits_equal(data, ref[j][0])
        bits_equal(sc, ref[j][1])
        bits_equal(ze, ref[j][2])
    assert arena.quantize_and_append(chunks[4][0]) == 20  # 90 + 70 > 100: the oldest 70 leave, 20 stay
    bits_equal(arena.get_packed_slice(0, 20)[0], ref[3][0][:, 10:])
    bits_equal(arena.get_packed_slice(20, 90)[0], ref[4][0])
    assert arena.quantize_and_append(chunks[5][0]) == 0 and arena.length == 100
    bits_equal(arena.get_packed_slice(0, 100)[0], ref[5][0])


def test_views_bytes_and_reset():
    announce("arena views / bytes_used / reset")
    H, D = 2, 128
    arena = _arena(H, 64, D, 4, 128)
    k, _ = _keys(H, 10, D, torch.float16, seed=3)
    arena.quantize_and_append(k)
    data, sc, ze = arena.get_packed_slice(2, 7)
    assert data.data_ptr() == arena.data[:, 2:7].data_ptr()  # views, no copy
    assert data.shape == (H, 5, 64) and sc.shape == (H, 5, 1)
    assert arena.bytes_used == H * 10 * 64 + 2 * H * 10 * 2
    arena.reset()
    assert arena.length == 0 and arena.bytes_used == 0 and not bool(arena.valid.any())
    assert arena.dequantize_slice(0, 0).shape == (H, 0, D)


def test_pack_unpack_helpers_match_oracle():
    from akv.packed_layout import PackedKVArena
    announce("arena _pack/_unpack")
    rng = np.random.default_rng(2)
    for bits in (2, 4, 8):
        codes = rng.integers(0, 1 << bits, (3, 5, 64)).astype(np.uint8)
        got = PackedKVArena._pack(to_dev(codes), bits)
        bits_equal(got, oleg.arena_pack(codes, bits))
        back = PackedKVArena._unpack(got, bits, 64)
        np.testing.assert_array_equal(back.cpu().numpy(), codes.astype(np.float32))
