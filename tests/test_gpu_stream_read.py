"""akv_stream_read, the benchmark's streaming-read reference: it reads the given bytes and
writes its 4-byte sink only when the XOR of the data equals its sentinel."""
import ctypes

import pytest
import torch

from gpu_util import announce

pytestmark = pytest.mark.gpu


def test_stream_read_runs_and_leaves_the_sink():
    from akv import _native as nat
    announce("stream read 64 MiB + 16 B")
    lib = nat.load()
    buf = torch.ones((64 << 20) // 2 + 8, dtype=torch.float16, device="cuda")  # XOR of equal words is 0
    sink = torch.full((1,), 7, dtype=torch.int32, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    nat.check(lib.akv_stream_read(ctypes.c_void_p(buf.data_ptr()), buf.numel() * 2, ctypes.c_void_p(sink.data_ptr()),
                                  ctypes.c_void_p(s)), "stream read")
    torch.cuda.synchronize()
    assert int(sink.item()) == 7
