"""packed_layout.measure_packed_bytes (akv/packed_layout.py:501-543) on host
tensors: the codes count at the length the reference's packers produce (checked
against the oracle's actual packed arrays, not a formula), or as stored when the
dict says they are packed already ('bits' key); scale / zero / group_mean /
group_std add their stored sizes; anything else is ignored."""
import numpy as np
import torch

from oracle import bitpack as obp


def test_measure_packed_bytes_matches_packed_lengths():
    from akv import packed_layout
    rng = np.random.default_rng(0)
    for bits in (2, 3, 4, 8):
        for dim in (1, 3, 7, 8, 9, 31, 64, 128, 130):
            codes = rng.integers(0, 1 << min(bits, 8), size=(2, 5, dim), dtype=np.uint8)
            packed_len = obp.pack(codes, bits).nbytes if bits in (2, 3, 4) else codes.nbytes
            scale = torch.zeros(2, 5, 1, dtype=torch.float16)
            zero = torch.zeros(2, 5, 1, dtype=torch.float32)
            q = {"codes": torch.from_numpy(codes), "scale": scale, "zero": zero, "note": "ignored", "group_mean": 3}
            assert packed_layout.measure_packed_bytes(q, bits) == packed_len + 2 * 10 + 4 * 10, (bits, dim)


def test_measure_packed_bytes_already_packed_and_empty():
    from akv import packed_layout
    packed = torch.zeros(4, 48, dtype=torch.uint8)
    gm, gs = torch.zeros(4, 2, dtype=torch.float16), torch.zeros(4, 2, dtype=torch.float16)
    q = {"codes": packed, "bits": 3, "group_mean": gm, "group_std": gs}
    assert packed_layout.measure_packed_bytes(q, 3) == 4 * 48 + 2 * 8 + 2 * 8
    assert packed_layout.measure_packed_bytes({}, 4) == 0
    assert packed_layout.measure_packed_bytes({"scale": gm}, 4) == 0
