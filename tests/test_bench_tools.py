"""The counter summary's split of one default bench run into workloads (no GPU:
synthetic dispatch lists with the kernel names rocprofv3 records)."""
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import bench  # noqa: E402


def _d(name, n, grid=256):
    return [(f"void akv::{name}(akv::Params)", grid, {"SQ_WAVES": 1.0}, 1000 + i) for i in range(n)]


def test_workload_dispatches_split():
    steps, warmup = 2, 1
    n_rep = (steps + warmup) * 28
    disp = (_d("decode_fast_kernel<3, 3, 4, 2, 0, false>", 2 * n_rep)
            + _d("prefill_kernel<2, 2, 4, false>", 3) + _d("prefill_kernel<2, 2, 4, true>", 3)
            + _d("decode_fast_kernel<4, 4, 2, 2, 0, true>", 5) + _d("decode_fast_kernel<2, 2, 1, 2, 0, true>", 4)
            + _d("quant_fast_kernel<3, 3, 4>", 2, grid=64) + _d("quant_fast_kernel<3, 3, 4>", 3, grid=512))
    out = bench._workload_dispatches(disp, steps, warmup)
    key, ds = out[("llama70b_prefill_128k", "all")]
    assert key == "prefill_kernel<2, 2, 4, false>" and len(ds) == 3
    key, ds = out[("llama70b_prefill_128k_causal", "all")]
    assert key == "prefill_kernel<2, 2, 4, true>" and len(ds) == 3
    assert len(out[("qwen_decode_32k", "attention_only")][1]) == n_rep
    assert len(out[("qwen_decode_32k", "with_importance")][1]) == n_rep
    assert len(out[("production_decode_4k", "all")][1]) == 5
    assert len(out[("kivi_decode_4k", "all")][1]) == 4
    assert [g for g, _, _ in out[("llama3_demote_64k", "all")][1]] == [512] * 3
