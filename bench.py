#!/usr/bin/env python
"""Decode dequant-attention on one MI355X: Qwen2.5-1.5B shape, 32k context.

Workload (one step = one decode token through all 28 layers): batch 8,
12 query / 2 KV heads, head_dim 128, context 32768 = 1024 hot fp16 tokens +
31744 warm tokens in the packed 3-bit block-affine tier (K per channel over
32-token blocks, V per token over 32-channel groups), importance EMA
(decay 0.9) updated every layer.  The 28 layers hold distinct buffers
(about 2.06 GB), so the 256 MB Infinity Cache cannot serve a step.  The
step is captured once in a HIP graph and replayed.

Prints one JSON line: value = effective KV GB/s (hot + warm codes + scale /
zero bytes read per layer / time per layer, the full step with importance),
plus us_per_layer, the roofline of the dequant-attention op and the CPU
baseline (the oracle's restatement of the reference CPU path on a bounded
sample).

The line's "workloads" field summarises the other configurations, each
measured after the headline on its own inputs (metric, value, roofline, CPU
baseline): qwen_decode_4k (one Qwen layer at 4k context, 4/4-bit, with the
reference CPU path beside it), llama7b_decode_16k (MHA, K4/V2 with outlier
channels), llama3_demote_64k (select + gather + quantize + pack, 3-bit; and
at 2 and 4 bits), llama70b_prefill_128k (MFMA chunked prefill; and with the
chunk's causal self-attention) and production_decode_4k
(ProductionCache.fused_attention over the 4-bit arenas at the cache's default
sizes, with the reference's torch design timed beside it) and kivi_decode_4k
(the KIVI baseline's attention at the same sizes, 2 bits).  --workload NAME
prints one of them on its own line instead.

The roofline is taken on the attention-only replay (per layer: one launch of
decode_fast_kernel, which also merges its splits): achieved = the op's
algorithmic bytes / its per-layer time, from HIP events on the stream the
kernel runs on.  `traffic` (HBM bytes per launch of each workload's dominant
kernel) comes from the FETCH_SIZE / WRITE_SIZE counter runs recorded in
profiles/hbm_traffic_by_workload.json, scaled by the same counters on a copy of
known size (--calib-copy adds that copy to the run; --summarize-counters turns
the rocprofv3 output directories into that file).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "adaptive-kv-memory_amd"))

METRIC = "decode-attn µs/layer + effective KV GB/s (% HBM peak) at 32K ctx, 1×MI355X"
HBM_PEAK_GBPS = 8000.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic_by_workload.json")
CALIB_BYTES = 256 << 20  # the calibration copy reads and writes this many bytes


def layer_bytes(s):
    """Algorithmic bytes of one decode layer, each byte counted once."""
    from akv.warm_tier import packed_row_bytes
    nblk = (s.n_warm + s.block_t - 1) // s.block_t
    q = s.B * s.Hq * s.M * s.D * 2
    hot = s.B * s.Hkv * s.n_hot * s.D * 2 * 2
    codes = s.B * s.Hkv * s.n_warm * (packed_row_bytes(s.D, s.bits_k) + packed_row_bytes(s.D, s.bits_v))
    kmeta = s.B * s.Hkv * nblk * s.D * 2 * 2
    vmeta = s.B * s.Hkv * s.n_warm * (s.D // s.group_v) * 2 * 2
    out = q
    imp = s.N * 4 * 2
    return {"q": q, "hot": hot, "codes": codes, "kmeta": kmeta, "vmeta": vmeta, "out": out, "importance": imp,
            "kv": hot + codes + kmeta + vmeta, "attn_total": q + hot + codes + kmeta + vmeta + out}


def cpu_baseline(layer0, s, budget_s=15.0, min_s=10.0):
    """The reference CPU path restated with torch CPU ops (fp16 dequant, head expansion
    and concatenation, fp32 attention, importance update) on layer 0, batch elements
    taken one at a time (cycling) for min_s to budget_s seconds of CPU work."""
    import torch
    from oracle import torch_cpu as otc
    cores = len(os.sched_getaffinity(0))
    q, kh, vh, warm, _ = layer0
    names = ["k_codes", "k_scale", "k_zero", "v_codes", "v_scale", "v_zero"]
    n_out = 0 if warm.k_oidx is None else warm.k_oidx.shape[-1]
    if n_out:
        names += ["k_oidx", "v_oidx", "k_odata", "v_odata"]
    host = {k: getattr(warm, k).cpu() for k in names}
    for k in ("k_oidx", "v_oidx"):
        if k in host:
            host[k] = host[k].long()
    qc, khc, vhc = q.cpu(), kh.cpu(), vh.cpu()
    done, t_cpu = 0, 0.0
    scores = torch.zeros(s.N, dtype=torch.float32)
    threads = torch.get_num_threads()
    torch.set_num_threads(cores)
    try:
        # every sequence of the layer at least once, cycling until min_s of work, at most budget_s
        while (done < s.B or t_cpu < min_s) and t_cpu < budget_s:
            b = done % s.B
            w = {k: v[b:b + 1] for k, v in host.items()}
            w.update(bits_k=s.bits_k, bits_v=s.bits_v, T=s.block_t, G=s.group_v, D=s.D, N=s.n_warm, n_out=n_out)
            t0 = time.perf_counter()
            kd, vd = otc.dequant_kv_blocked(w)
            _, attn = otc.decode_attention(qc[b:b + 1], khc[b:b + 1], vhc[b:b + 1], kd, vd, hot_first=False,
                                           return_weights=s.decay is not None)
            if s.decay is not None:
                scores = otc.importance_update(attn, scores, s.decay)
            t_cpu += time.perf_counter() - t0
            done += 1
    finally:
        torch.set_num_threads(threads)
    kv_bytes = layer_bytes(s)["kv"] * done / s.B
    return {"value": round(kv_bytes / t_cpu / 1e9, 4), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"layer 0, {done} sequence passes over its {s.B} sequences (torch CPU: fp16 dequant, "
                      f"repeat_kv + cat, fp32 "
                      f"attention{' + importance' if s.decay is not None else ''}), "
                      f"{t_cpu:.1f} s on {cores} host threads",
            "us_per_layer_equiv": round(t_cpu / done * s.B * 1e6, 1)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--layers", type=int, default=0, help="override layer count (profiling only)")
    ap.add_argument("--calib-copy", action="store_true",
                    help="end with one device copy of 256 MiB (reference dispatch for counter runs)")
    ap.add_argument("--workload", default="qwen_decode_32k",
                    choices=["qwen_decode_32k", "llama7b_decode_16k", "llama70b_prefill_128k",
                             "llama70b_prefill_128k_causal", "llama3_demote_64k", "qwen_decode_4k",
                             "production_decode_4k", "kivi_decode_4k"],
                    help="the headline decode step (default; the other workloads are summarised in its "
                         "'workloads' field), or one other workload on its own line")
    ap.add_argument("--no-other-workloads", action="store_true",
                    help="headline only: skip the summaries of the other workloads")
    ap.add_argument("--bits", type=int, default=3, help="demotion workload: code width (2, 3 or 4)")
    ap.add_argument("--summarize-counters", nargs="+", metavar="DIR",
                    help="no GPU work: summarise rocprofv3 --pmc output directories of a default run made with "
                         "the same --steps/--warmup and --no-cpu-baseline --calib-copy")
    ap.add_argument("--write-traffic", action="store_true",
                    help="with --summarize-counters: record the HBM bytes per dispatch for the bench line")
    ap.add_argument("--timeline", choices=["attn", "full"],
                    help="per-wave phase timestamps of one 32k decode launch (attention only, or with the "
                         "importance stash) from the timeline build of the library (make -C "
                         "adaptive-kv-memory_amd/csrc timeline); prints a table, not the bench line")
    args = ap.parse_args()
    if args.summarize_counters:
        return summarize_counters(args.summarize_counters, args.steps, args.warmup, args.write_traffic)
    if args.timeline:
        return bench_timeline(args)
    if args.gpus != 1:
        print(json.dumps({"error": "one GPU only: the warm-tier path has no multi-GPU leg (a (batch, kv-head) "
                                   "shard per GPU needs no communication)", "n_gpus": args.gpus}))
        sys.exit(2)

    import torch
    import akv
    from akv import workloads as wl
    from akv.warm_tier import DecodeCall
    if args.workload != "qwen_decode_32k":
        fn = {"llama70b_prefill_128k": bench_prefill, "llama3_demote_64k": bench_demote,
              "llama70b_prefill_128k_causal": lambda a: bench_prefill(a, causal=True),
              "llama7b_decode_16k": bench_decode_mha, "qwen_decode_4k": bench_c1,
              "production_decode_4k": bench_production, "kivi_decode_4k": bench_kivi}[args.workload]
        print(json.dumps(fn(args)), flush=True)
        return

    s = wl.QWEN_DECODE_32K
    L = args.layers or s.layers
    dev = "cuda"
    print(f"[bench] building {L} layers of {s.name}", file=sys.stderr, flush=True)
    layers = []
    for layer in range(L):
        k, v = wl.make_kv(s, layer, device=dev)
        q = wl.make_q(s, layer, device=dev)
        (kw, vw), (kh, vh) = wl.split_hot_warm(k, v, s.n_hot)
        warm = akv.quantize_kv(kw, vw, s.bits_k, s.bits_v, s.block_t, s.group_v)
        scores = torch.zeros(s.N, dtype=torch.float32, device=dev)
        layers.append((q, kh, vh, warm, scores))
        del k, v, kw, vw
    torch.cuda.synchronize()
    full = [DecodeCall(q, kh, vh, w, scores=sc, decay=s.decay, hot_first=False) for (q, kh, vh, w, sc) in layers]
    attn_only = [DecodeCall(q, kh, vh, w, hot_first=False) for (q, kh, vh, w, _) in layers]
    for c in full + attn_only:
        c()
    torch.cuda.synchronize()

    def capture(calls):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for c in calls:
                c()
        return g

    g_full, g_attn = capture(full), capture(attn_only)

    def timed(g, steps, warmup):
        for _ in range(warmup):
            g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record()
        for _ in range(steps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        return e0.elapsed_time(e1) / steps, wall * 1e3 / steps

    print("[bench] timing", file=sys.stderr, flush=True)
    ev_ms, wall_ms = timed(g_full, args.steps, args.warmup)
    ev_attn_ms, _ = timed(g_attn, args.steps, args.warmup)
    nb = layer_bytes(s)
    us_layer = ev_ms * 1e3 / L
    us_layer_attn = ev_attn_ms * 1e3 / L
    kv_gbps = nb["kv"] / (us_layer * 1e-6) / 1e9
    alg = nb["attn_total"]
    achieved = alg / (us_layer_attn * 1e-6) / 1e9
    traffic = recorded_traffic(s.name, "attention_only")
    res = {
        "metric": METRIC,
        "value": round(kv_gbps, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded N(0,1) K/V, 2 K channels per kv head x10, quantized on the device)",
        "config": {"workload": s.name, "B": s.B, "Hq": s.Hq, "Hkv": s.Hkv, "D": s.D, "context": s.N,
                   "n_hot": s.n_hot, "n_warm": s.n_warm, "bits_k": s.bits_k, "bits_v": s.bits_v,
                   "block_t": s.block_t, "group_v": s.group_v, "layers": L, "importance_decay": s.decay},
        "us_per_layer": round(us_layer, 3),
        "us_per_layer_attn_only": round(us_layer_attn, 3),
        "effective_kv_gbps_attn_only": round(nb["kv"] / (us_layer_attn * 1e-6) / 1e9, 2),
        "hbm_frac_effective_kv": round(kv_gbps / HBM_PEAK_GBPS, 4),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "kernel": "akv_decode_attn attention per layer (decode_fast_kernel, splits merged in the kernel)",
                     "algorithmic_bytes_per_launch": alg,
                     "us_per_launch": round(us_layer_attn, 3)},
    }
    del g_full, g_attn, full, attn_only
    torch.cuda.empty_cache()
    add_stream_reference(res["roofline"])
    if not args.no_cpu_baseline:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        res["cpu_baseline"] = cpu_baseline(layers[0], s)
    if not args.no_other_workloads and L == s.layers:
        del layers
        torch.cuda.empty_cache()
        res["workloads"] = other_workloads(args)
    if args.calib_copy:
        src = torch.zeros(CALIB_BYTES // 2, dtype=torch.float16, device=dev)
        dst = torch.empty_like(src)
        torch.neg(src, out=dst)  # one elementwise kernel: reads and writes CALIB_BYTES
        torch.cuda.synchronize()
    print(json.dumps(res), flush=True)


# Words of the per-wave timeline the timeline build of the decode kernel records (one
# launch; times in ticks of the 100 MHz real-time clock): index -> (label, kind).
_TL_WORDS = [(0, "wave start"), (10, "first load issued"), (13, "start barrier passed"),
             (1, "first unit landed"), (2, "warm units done"), (3, "last item done"),
             (11, "12 waves merged in LDS"), (4, "partial written and acknowledged")]


def bench_timeline(args):
    """Per-phase timestamps of one launch of layer 13 of the 32k decode (after the graph
    of all 28 layers has been timed and replayed): the timeline build records 16 words
    per wave and writes them where the wave leaves the kernel."""
    import numpy as np
    lib_path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "adaptive-kv-memory_amd", "akv",
                            "libakv_hip_timeline.so")
    if not os.path.exists(lib_path):
        sys.exit(f"{lib_path} is missing: build it with make -C adaptive-kv-memory_amd/csrc timeline")
    os.environ["AKV_LIB"] = lib_path
    import ctypes
    import torch
    import akv
    from akv import _native as nat
    from akv import workloads as wl
    from akv.warm_tier import DecodeCall
    lib = nat.load()
    words = lib.akv_timeline_words()
    if words <= 0:
        sys.exit("the library loaded records no timeline")
    s = wl.QWEN_DECODE_32K
    L = args.layers or s.layers
    calls = []
    for layer in range(L):
        k, v = wl.make_kv(s, layer, device="cuda")
        q = wl.make_q(s, layer, device="cuda")
        (kw, vw), (kh, vh) = wl.split_hot_warm(k, v, s.n_hot)
        warm = akv.quantize_kv(kw, vw, s.bits_k, s.bits_v, s.block_t, s.group_v)
        sc = torch.zeros(s.N, dtype=torch.float32, device="cuda") if args.timeline == "full" else None
        calls.append(DecodeCall(q, kh, vh, warm, scores=sc, decay=s.decay, hot_first=False))
        del k, v, kw, vw
    for c in calls:
        c()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for c in calls:
            c()
    for _ in range(args.warmup):
        g.replay()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    us_layer = e0.elapsed_time(e1) * 1e3 / args.steps / L
    st = torch.cuda.current_stream().cuda_stream
    nat.check(lib.akv_timeline_clear(ctypes.c_void_p(st)), "timeline clear")
    calls[13 % L]()
    torch.cuda.synchronize()
    buf = np.zeros(words, dtype=np.uint64)
    nat.check(lib.akv_timeline_fetch(ctypes.c_void_p(buf.ctypes.data), words), "timeline fetch")
    t = buf.reshape(-1, 16).astype(np.float64)
    live = t[:, 0] > 0
    nw_per_wg = 12  # waves of the kernel's workgroup (no outlier channels)
    nwg = (int(np.nonzero(live)[0].max()) + 1) // nw_per_wg
    t = t[: nwg * nw_per_wg]
    live = t[:, 0] > 0
    t0 = t[live, 0].min()
    rel = lambda col: (t[:, col] - t0) / 100.0

    def pct(x):
        return {"p10": round(float(np.percentile(x, 10)), 2), "p50": round(float(np.median(x)), 2),
                "p90": round(float(np.percentile(x, 90)), 2), "max": round(float(x.max()), 2)}

    rows = [(label, pct(rel(col)[live])) for col, label in _TL_WORDS]
    role = t[:, 5].astype(np.uint64) & np.uint64(3)
    m5 = t[:, 5] > 0
    t5 = ((t[:, 5].astype(np.uint64) >> np.uint64(2)).astype(np.float64) - t0) / 100.0
    rows.append(("arrival counted (device-scope atomic)", pct(t5[m5])))
    m12 = t[:, 12] > 0
    rows.append(("merging workgroup's partial loads done", pct(rel(12)[m12])))
    m6 = t[:, 6] > 0
    rows.append(("merging workgroup done", pct(rel(6)[m6])))
    t3 = rel(3).reshape(nwg, nw_per_wg)
    out = {"mode": "timeline", "workload": "qwen_decode_32k", "phase": args.timeline, "layers": L,
           "graph_us_per_layer": round(us_layer, 3), "workgroups": nwg, "waves": int(live.sum()),
           "phases_us": {label: v for label, v in rows},
           "items_per_wave": pct(t[live, 7]), "ticks_waiting_for_ring_data_us": pct(t[live, 8] / 100.0),
           "workgroup_spread_of_last_item_us": pct(t3.max(1) - t3.min(1)),
           "merging_workgroups": int((role[m5] != 0).sum()) // nw_per_wg,
           "items_by_wave_index": [round(float(x), 2) for x in t[:, 7].reshape(nwg, nw_per_wg).mean(0)]}
    print(f"| phase (us from the launch's first wave) | p10 | p50 | p90 | max |")
    print("|---|---:|---:|---:|---:|")
    for label, v in rows:
        print(f"| {label} | {v['p10']} | {v['p50']} | {v['p90']} | {v['max']} |")
    print(json.dumps(out), flush=True)


def stream_read_reference(nbytes, launches=28, steps=10):
    """The same byte count read once by akv_stream_read (16-byte non-temporal loads over
    a grid-stride loop, nothing else): what a read-once kernel of that size reaches on
    this GPU, launch included.  Successive launches read different regions of a buffer
    of at least 1 GiB, so the 256 MB Infinity Cache does not serve them; sizes above
    1 GiB are timed at 1 GiB and scaled."""
    import ctypes
    import torch
    from akv import _native as nat
    lib = nat.load()
    n = min(int(nbytes) // 16 * 16, 1 << 30)
    regions = max(1, (1 << 30) // n)
    buf = torch.ones((regions * n) // 2, dtype=torch.float16, device="cuda")
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")

    def launch(k):  # on the current stream (the capture stream inside the graph)
        stream = torch.cuda.current_stream().cuda_stream
        nat.check(lib.akv_stream_read(ctypes.c_void_p(buf.data_ptr() + (k % regions) * n), n,
                                      ctypes.c_void_p(sink.data_ptr()), ctypes.c_void_p(stream)), "stream read")
    launch(0)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for k in range(launches):
            launch(k)
    ms, _ = _event_time(g.replay, steps, 2)
    us = ms * 1e3 / launches
    gbps = n / (us * 1e-6) / 1e9
    del g, buf
    torch.cuda.empty_cache()
    return {"GBps": round(gbps, 1), "us_per_launch": round(nbytes / (gbps * 1e9) * 1e6, 3),
            "bytes_timed": n, "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4)}


def add_stream_reference(roof):
    """Put the streaming-read figure for the roofline's algorithmic bytes beside it."""
    try:
        ref = stream_read_reference(roof["algorithmic_bytes_per_launch"])
        ref["kernel_frac_of_stream"] = round(roof["achieved"] / ref["GBps"], 4)
        roof["stream_read"] = ref
    except Exception as e:  # the reference figure is informative only
        roof["stream_read"] = {"error": f"{type(e).__name__}: {e}"}


SUMMARY_KEYS = ("metric", "value", "unit", "ms_per_call", "us_per_layer", "ms_quantize_only", "roofline",
                "cpu_baseline", "config", "gpu_us_per_layer", "reference_design_gpu")


def other_workloads(args):
    """The other benchmark configurations, each on its own synthetic inputs, summarised
    (metric, value, roofline, CPU baseline) inside the headline line so one default run
    records every configuration."""
    import copy
    import torch
    out = {}

    def demote_at(bits):  # the demotion workload at another code width (GPU line only)
        def run(a):
            a = copy.copy(a)
            a.bits, a.no_cpu_baseline = bits, True
            return bench_demote(a)
        return run

    def prefill_causal(a):  # the prefill workload with the chunk's causal self-attention (GPU line only)
        a = copy.copy(a)
        a.no_cpu_baseline = True
        return bench_prefill(a, causal=True)

    for name, fn in (("qwen_decode_4k", bench_c1), ("llama7b_decode_16k", bench_decode_mha),
                     ("llama3_demote_64k", bench_demote), ("llama3_demote_64k_2bit", demote_at(2)),
                     ("llama3_demote_64k_4bit", demote_at(4)), ("llama70b_prefill_128k", bench_prefill),
                     ("llama70b_prefill_128k_causal", prefill_causal),
                     ("production_decode_4k", bench_production), ("kivi_decode_4k", bench_kivi)):
        print(f"[bench] workload {name}", file=sys.stderr, flush=True)
        try:
            r = fn(args)
            out[name] = {k: r[k] for k in SUMMARY_KEYS if k in r}
        except Exception as e:  # a failing secondary workload is reported, the headline stands
            out[name] = {"error": f"{type(e).__name__}: {e}"}
        torch.cuda.empty_cache()
    return out


def bench_c1(args):
    """Qwen2.5-1.5B shape at 4k context (B1, 12/2 heads, 512 hot + 3584 warm 4/4-bit, two K
    channels per kv head x10): the reference's CPU path -- its fp16 dequant and fp32
    attention (akv/affine_quantizer.py:112-124, akv/triton_kernels.py:350-387) restated
    with torch CPU ops and timed on the host cores -- and the same layer on the GPU (one
    akv_decode_attn launch)."""
    import torch
    import akv
    from akv import workloads as wl
    from akv.warm_tier import DecodeCall
    from oracle import torch_cpu as otc
    s = wl.QWEN_DECODE_4K
    k, v = wl.make_kv(s, device="cuda")
    q = wl.make_q(s, device="cuda")
    (kw, vw), (kh, vh) = wl.split_hot_warm(k, v, s.n_hot)
    warm = akv.quantize_kv(kw, vw, s.bits_k, s.bits_v, s.block_t, s.group_v)
    call = DecodeCall(q, kh, vh, warm, hot_first=False)
    call()
    torch.cuda.synchronize()
    reps = 32  # one graph replays the layer 32 times back to back (no host gaps between launches)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            call()
    ms, _ = _event_time(g.replay, max(args.steps, 20), args.warmup)
    ms /= reps
    nb = layer_bytes(s)
    res = {"metric": "decode-attn us/layer, Qwen2.5-1.5B 4k (reference CPU path and 1xMI355X)",
           "value": round(ms * 1e3, 3), "unit": "us", "higher_is_better": False,
           "gpu_us_per_layer": round(ms * 1e3, 3),
           "config": {"workload": s.name, "B": s.B, "Hq": s.Hq, "Hkv": s.Hkv, "D": s.D, "context": s.N,
                      "n_hot": s.n_hot, "n_warm": s.n_warm, "bits_k": s.bits_k, "bits_v": s.bits_v},
           "roofline": {"bound": "hbm", "achieved": round(nb["attn_total"] / (ms * 1e-3) / 1e9, 2),
                        "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                        "frac": round(nb["attn_total"] / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                        "traffic": recorded_traffic(s.name),
                        "kernel": "akv_decode_attn, 32 launches per graph replay (1.7 MB per layer: launch-bound, "
                                  "and the layer stays in the 256 MB Infinity Cache)",
                        "algorithmic_bytes_per_launch": nb["attn_total"]}}
    add_stream_reference(res["roofline"])
    if not args.no_cpu_baseline:
        cores = len(os.sched_getaffinity(0))
        host = {n: getattr(warm, n).cpu() for n in ("k_codes", "k_scale", "k_zero", "v_codes", "v_scale", "v_zero")}
        host.update(bits_k=s.bits_k, bits_v=s.bits_v, T=s.block_t, G=s.group_v, D=s.D, N=s.n_warm, n_out=0)
        qc, khc, vhc = q.cpu(), kh.cpu(), vh.cpu()
        reps, t_cpu = 0, 0.0
        threads = torch.get_num_threads()
        torch.set_num_threads(cores)
        try:
            while t_cpu < 10.0 or reps < 3:
                t0 = time.perf_counter()
                kd, vd = otc.dequant_kv_blocked(host)
                otc.decode_attention(qc, khc, vhc, kd, vd, hot_first=False, return_weights=False)
                t_cpu += time.perf_counter() - t0
                reps += 1
        finally:
            torch.set_num_threads(threads)
        us = t_cpu / reps * 1e6
        res["cpu_baseline"] = {"value": round(us, 1), "unit": "us per layer", "cores": cores, "kind": "port",
                               "sample": f"the whole layer (torch CPU: fp16 dequant, repeat_kv + cat, fp32 "
                                         f"attention), {reps} runs, "
                                         f"{t_cpu:.1f} s on {cores} host threads",
                               "kv_gbps": round(nb["kv"] / (us * 1e-6) / 1e9, 4)}
    return res


def bench_production(args):
    """ProductionCache.fused_attention at the reference's ProductionCacheConfig defaults
    (akv/production_cache.py:33-70: 32 layers, 32 heads, head_dim 128, hot 1024 + warm
    4096 tokens, group 64) with the minmax arenas at 4 bits: every layer's arenas full and
    1024 hot tokens, one query token.  The 32 layers' calls (one decode launch each over
    the packed arenas and the hot buffer) are captured in one graph; the working set
    (1.14 GB) is beyond the 256 MB Infinity Cache.  Beside it, the reference's design on
    the same GPU: the cached fp16 warm copy plus the hot tokens copied into one buffer,
    then matmul / softmax / matmul (akv/production_cache.py:429-469)."""
    import numpy as np
    import torch
    from threadpoolctl import threadpool_limits
    from akv.production_cache import ProductionCache, ProductionCacheConfig
    from oracle import legacy as oleg
    L, H, D, NH, NW, bits, gs = 32, 32, 128, 1024, 4096, 4, 64
    cfg = ProductionCacheConfig(num_layers=L, num_heads=H, head_dim=D, hot_budget=NH, warm_budget=NW,
                                warm_bits=bits, group_size=gs, warm_quantizer="minmax", max_hot_pages=NH // 16,
                                device="cuda")
    cache = ProductionCache(cfg)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(7)

    def rnd(n):
        return torch.randn(H, n, D, generator=gen, device="cuda", dtype=torch.float16)

    for lay in cache._layers:
        lay._warm_k.quantize_and_append(rnd(NW))
        lay._warm_v.quantize_and_append(rnd(NW))
        lay.append_hot(rnd(NH), rnd(NH))
    q = torch.randn(1, H, 1, D, generator=gen, device="cuda", dtype=torch.float16)

    def calls():
        return [cache.fused_attention(q, i) for i in range(L)]

    calls()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        calls()
    ms, wall_ms = _event_time(graph.replay, max(args.steps, 20), args.warmup)
    us_layer = ms * 1e3 / L
    qo = 2 * H * D * 2
    hot = H * NH * D * 2 * 2
    codes = H * NW * (D * bits // 8) * 2
    meta = H * NW * (D // gs) * 2 * 2 * 2
    alg = qo + hot + codes + meta
    achieved = alg / (us_layer * 1e-6) / 1e9
    # the reference's design: fp16 warm copy + hot copy into one buffer, then torch ops
    bufs = []
    for lay in cache._layers:
        wk, wv = lay.get_warm_fp16()
        kb = torch.empty(H, NW + NH, D, dtype=torch.float16, device="cuda")
        vb = torch.empty_like(kb)
        kb[:, :NW], vb[:, :NW] = wk, wv
        bufs.append((kb, vb))
    qt = q[0].transpose(-1, -2).contiguous()  # (H, D, 1): no transposed right operand

    def ref_design():
        for lay, (kb, vb) in zip(cache._layers, bufs):
            kb[:, NW:] = lay.get_hot_kv()[0]
            vb[:, NW:] = lay.get_hot_kv()[1]
            p = torch.softmax(torch.matmul(kb, qt) * D ** -0.5, dim=1)  # (H, N, 1)
            torch.matmul(p.transpose(1, 2).contiguous(), vb)

    ref_ms, _ = _event_time(ref_design, max(args.steps, 20), args.warmup)
    ref_bytes = hot * 2 + H * (NW + NH) * D * 2 * 2
    res = {"metric": "ProductionCache.fused_attention us/layer + effective KV GB/s (% HBM peak), "
                     "reference defaults (32 heads, 1024 hot + 4096 warm 4-bit), 1xMI355X",
           "value": round((hot + codes + meta) / (us_layer * 1e-6) / 1e9, 2), "unit": "GB/s",
           "higher_is_better": True, "dtype": "f16", "us_per_layer": round(us_layer, 3),
           "config": {"workload": "production_decode_4k", "layers": L, "heads": H, "D": D, "n_hot": NH,
                      "n_warm": NW, "bits": bits, "group_size": gs, "warm_quantizer": "minmax"},
           "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                        "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": recorded_traffic("production_decode_4k"),
                        "kernel": "akv_decode_attn per layer (legacy arena warm tier, decode_fast_kernel LEG variant)",
                        "algorithmic_bytes_per_launch": alg, "us_per_launch": round(us_layer, 3)},
           "reference_design_gpu": {"us_per_layer": round(ref_ms * 1e3 / L, 3),
                                    "bytes_per_layer": ref_bytes,
                                    "what": "cached fp16 warm copy + hot copy, torch matmul/softmax/matmul"}}
    add_stream_reference(res["roofline"])
    if not args.no_cpu_baseline:
        cores = len(os.sched_getaffinity(0))
        lay = cache._layers[0]
        host = [t.cpu().numpy() for a in (lay._warm_k, lay._warm_v) for t in (a.data, a.scales, a.zeros)]
        hk = lay.get_hot_kv()[0].float().cpu().numpy()
        hv = lay.get_hot_kv()[1].float().cpu().numpy()
        qn = q[0, :, 0].float().cpu().numpy()
        reps, t_cpu = 0, 0.0
        with threadpool_limits(limits=cores):
            while t_cpu < 10.0 or reps < 3:
                t0 = time.perf_counter()
                wk = oleg.arena_dequantize(*host[:3], bits, gs, D).astype(np.float32)
                wv = oleg.arena_dequantize(*host[3:], bits, gs, D).astype(np.float32)
                k, v = np.concatenate([wk, hk], axis=1), np.concatenate([wv, hv], axis=1)
                sc = np.einsum("hd,hnd->hn", qn, k) * np.float32(D ** -0.5)
                e = np.exp(sc - sc.max(axis=1, keepdims=True))
                np.einsum("hn,hnd->hd", e / e.sum(axis=1, keepdims=True), v)
                t_cpu += time.perf_counter() - t0
                reps += 1
        us = t_cpu / reps * 1e6
        res["cpu_baseline"] = {"value": round(us, 1), "unit": "us per layer", "cores": cores, "kind": "port",
                               "sample": f"layer 0 (arena dequant + fp32 attention), {reps} runs, "
                                         f"{t_cpu:.1f} s on {cores} host threads"}
    del cache, bufs
    return res


def bench_kivi(args):
    """KIVIFusedCache.fused_attention (akv/baselines.py:426-510 with this build's attention
    leg) at the production cache's sizes: 32 layers, 32 heads, head_dim 128, 4096 tokens
    quantized at 2 bits in groups of 128 plus the 128-token residual window, one query
    token; the 32 layers' calls captured in one graph.  Beside it, the reference's use
    of the baseline on the same GPU: the float16 view ``update`` returns (the working
    copy concatenated with the residual) attended by matmul / softmax / matmul."""
    import numpy as np
    import torch
    from threadpoolctl import threadpool_limits
    from akv.baselines import KIVIFusedCache, KIVIFusedConfig
    from oracle.kivi import kivi_dequantize
    from oracle import legacy as oleg
    L, H, D, NQ, RES, bits, gs = 32, 32, 128, 4096, 128, 2, 128
    cache = KIVIFusedCache(KIVIFusedConfig(key_bits=bits, value_bits=bits, group_size=gs, residual_length=RES))
    gen = torch.Generator(device="cuda")
    gen.manual_seed(11)
    views = []
    for layer in range(L):
        k = torch.randn(1, H, NQ + RES, D, generator=gen, device="cuda", dtype=torch.float16)
        v = torch.randn(1, H, NQ + RES, D, generator=gen, device="cuda", dtype=torch.float16)
        views.append(cache.update(k, v, layer))
        del k, v
    q = torch.randn(1, H, 1, D, generator=gen, device="cuda", dtype=torch.float16)

    def calls():
        return [cache.fused_attention(q, i) for i in range(L)]

    calls()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        calls()
    ms, _ = _event_time(graph.replay, max(args.steps, 20), args.warmup)
    us_layer = ms * 1e3 / L
    qo = 2 * H * D * 2
    hot = H * RES * D * 2 * 2
    codes = H * NQ * (D * bits // 8) * 2
    meta = H * NQ * (D // gs) * 2 * 2 * 2
    alg = qo + hot + codes + meta
    achieved = alg / (us_layer * 1e-6) / 1e9
    qt = q[0].transpose(-1, -2).contiguous()  # (H, D, 1): no transposed right operand

    def ref_design():  # the view update returns, then the attention a model runs on it
        for layer in range(L):
            kv, vv = cache._get_full_kv(layer)
            p = torch.softmax(torch.matmul(kv[0], qt) * D ** -0.5, dim=1)
            torch.matmul(p.transpose(1, 2).contiguous(), vv[0])

    ref_ms, _ = _event_time(ref_design, max(args.steps, 20), args.warmup)
    res = {"metric": "KIVIFusedCache.fused_attention us/layer + effective KV GB/s (% HBM peak), 32 heads, "
                     "4096 tokens at 2 bits + 128 residual, 1xMI355X",
           "value": round((hot + codes + meta) / (us_layer * 1e-6) / 1e9, 2), "unit": "GB/s",
           "higher_is_better": True, "dtype": "f16", "us_per_layer": round(us_layer, 3),
           "config": {"workload": "kivi_decode_4k", "layers": L, "heads": H, "D": D, "quantized": NQ,
                      "residual": RES, "bits": bits, "group_size": gs},
           "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                        "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": recorded_traffic("kivi_decode_4k"),
                        "kernel": "akv_decode_attn per layer (legacy per-(batch, head) tier, decode_fast_kernel LEG "
                                  "variant)",
                        "algorithmic_bytes_per_launch": alg, "us_per_launch": round(us_layer, 3)},
           "reference_design_gpu": {"us_per_layer": round(ref_ms * 1e3 / L, 3),
                                    "what": "float16 working copy + residual concatenated, torch "
                                            "matmul/softmax/matmul"}}
    add_stream_reference(res["roofline"])
    if not args.no_cpu_baseline:
        cores = len(os.sched_getaffinity(0))
        t_k, t_v = cache._quant_keys[0], cache._quant_values[0]
        n = t_k.n
        host = [(np.ascontiguousarray(t.codes[:, :n].cpu().numpy()), t.sc[:, :n].cpu().numpy(),
                 t.ze[:, :n].cpu().numpy()) for t in (t_k, t_v)]
        rk = cache._residual_keys[0][0].float().cpu().numpy()
        rv = cache._residual_values[0][0].float().cpu().numpy()
        qn = q[0, :, 0].float().cpu().numpy()
        reps, t_cpu = 0, 0.0
        with threadpool_limits(limits=cores):
            while t_cpu < 10.0 or reps < 3:
                t0 = time.perf_counter()
                kv = []
                for c, s_, z_ in host:
                    u = oleg.arena_unpack(c, bits, D)
                    kv.append(kivi_dequantize(u.astype(np.uint8).reshape(H * n, 1, D), s_.reshape(H * n, 1),
                                              z_.reshape(H * n, 1), (1, H, n, D))[0].astype(np.float32))
                k = np.concatenate([kv[0], rk], axis=1)
                v = np.concatenate([kv[1], rv], axis=1)
                sc = np.einsum("hd,hnd->hn", qn, k) * np.float32(D ** -0.5)
                e = np.exp(sc - sc.max(axis=1, keepdims=True))
                np.einsum("hn,hnd->hd", e / e.sum(axis=1, keepdims=True), v)
                t_cpu += time.perf_counter() - t0
                reps += 1
        res["cpu_baseline"] = {"value": round(t_cpu / reps * 1e6, 1), "unit": "us per layer", "cores": cores,
                               "kind": "port", "sample": f"layer 0 (dequant + fp32 attention), {reps} runs, "
                                                         f"{t_cpu:.1f} s on {cores} host threads"}
    del cache, views
    return res


def recorded_traffic(workload, phase="all"):
    """HBM bytes per launch of the workload's dominant kernel, from the counter runs
    summarised in TRAFFIC_FILE (None when that file has no entry)."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    with open(TRAFFIC_FILE) as f:
        rec = json.load(f).get("workloads", {}).get(workload, {})
    return rec.get(phase, {}).get("hbm_bytes_per_dispatch")


def _counter_dispatches(csv_path):
    """rocprofv3 counter CSV -> dispatches in order: (kernel name, grid, {counter: value}, ns)."""
    import csv
    by_id = {}
    with open(csv_path) as f:
        for r in csv.DictReader(f):
            d = by_id.setdefault(int(r["Dispatch_Id"]), [r["Kernel_Name"], int(r["Grid_Size"]), {},
                                                          int(r["End_Timestamp"]) - int(r["Start_Timestamp"])])
            d[2][r["Counter_Name"]] = d[2].get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    return [tuple(by_id[i]) for i in sorted(by_id)]


def _workload_dispatches(disp, steps, warmup):
    """Split the dispatches of one default bench run (run with --steps/--warmup as given
    and --no-cpu-baseline --calib-copy) into the workloads' dominant kernels.  The
    headline replays the full step (warmup + steps) x 28 times, then the attention-only
    step as often, so its attention-only dispatches are the last of its kernel."""
    import re
    groups = {}
    for name, grid, ctr, ns in disp:
        m = re.search(r"akv::(\w+_kernel)<([^>]*)>", name)
        key = (m.group(1) + "<" + m.group(2) + ">") if m else ("calibration copy" if "neg_kernel" in name else None)
        if key:
            groups.setdefault(key, []).append((grid, ctr, ns))
    out = {}
    L = 28
    n_rep = (warmup + steps) * L
    for key, ds in groups.items():
        legacy = key.startswith("decode_fast_kernel") and key.endswith("true>")  # the LEG variant
        if legacy and key.startswith("decode_fast_kernel<4, 4,"):
            out[("production_decode_4k", "all")] = (key, ds)
        elif legacy and key.startswith("decode_fast_kernel<2, 2,"):
            out[("kivi_decode_4k", "all")] = (key, ds)
        elif legacy:
            continue
        elif key.startswith("decode_fast_kernel<3, 3,"):
            out[("qwen_decode_32k", "attention_only")] = (key, ds[-n_rep:])
            out[("qwen_decode_32k", "with_importance")] = (key, ds[-2 * n_rep:-n_rep])
        elif key.startswith("decode_fast_kernel<4, 4,"):
            out[("qwen_decode_4k", "all")] = (key, ds)
        elif key.startswith("decode_fast_kernel<4, 2,"):
            out[("llama7b_decode_16k", "all")] = (key, ds)
        elif key.startswith("quant_fast_kernel<3, 3,"):
            big = max(g for g, _, _ in ds)  # the demotion launch covers 16 x 8 heads; the headline's own build less
            out[("llama3_demote_64k", "all")] = (key, [d for d in ds if d[0] == big])
        elif key.startswith("prefill_kernel"):  # the causal variant is the instantiation ending in "true"
            causal = key.endswith("true>")
            out[("llama70b_prefill_128k_causal" if causal else "llama70b_prefill_128k", "all")] = (key, ds)
        elif key == "calibration copy":
            out[("calibration", "all")] = (key, ds[-1:])
    return out


def summarize_counters(run_dirs, steps, warmup, write_json):
    """Average each workload's counters per dispatch over the counter runs in run_dirs
    (each a rocprofv3 -d directory); FETCH_SIZE / WRITE_SIZE (KiB) are scaled by what
    they read for the calibration copy of CALIB_BYTES (read once and written once)."""
    import glob
    ctr = {}
    for d in run_dirs:
        paths = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
        if len(paths) != 1:
            raise SystemExit(f"{d}: expected one counter_collection.csv, found {len(paths)}")
        for wk, (key, ds) in _workload_dispatches(_counter_dispatches(paths[0]), steps, warmup).items():
            e = ctr.setdefault(wk, {"kernel": key, "dispatches": len(ds), "counters": {}, "ns": []})
            e["ns"] += [ns for _, _, ns in ds]
            for name in ds[0][1]:
                e["counters"][name] = sum(c[name] for _, c, _ in ds) / len(ds)
    cal = ctr.get(("calibration", "all"), {}).get("counters", {})
    scale = {c: (CALIB_BYTES / 1024.0) / cal[c] for c in ("FETCH_SIZE", "WRITE_SIZE") if cal.get(c)}
    res = {"calibration_kib": {c: cal.get(c) for c in ("FETCH_SIZE", "WRITE_SIZE")}, "calibration_bytes": CALIB_BYTES,
           "scale": scale, "workloads": {}}
    for (w, phase), e in sorted(ctr.items()):
        if w == "calibration":
            continue
        c = e["counters"]
        rec = {"kernel": e["kernel"], "dispatches": e["dispatches"],
               "avg_ns_under_counters": round(sum(e["ns"]) / len(e["ns"])), "counters_per_dispatch": c}
        if "FETCH_SIZE" in c and "WRITE_SIZE" in c and len(scale) == 2:
            rec["hbm_bytes_per_dispatch"] = round((c["FETCH_SIZE"] * scale["FETCH_SIZE"]
                                                   + c["WRITE_SIZE"] * scale["WRITE_SIZE"]) * 1024)
        if c.get("SQ_WAVES"):
            rec["per_wave"] = {k: round(v / c["SQ_WAVES"], 1) for k, v in c.items()
                               if k.startswith("SQ_INSTS") or k.startswith("SQ_WAIT") or k.startswith("SQ_ACTIVE")}
        res["workloads"].setdefault(w, {})[phase] = rec
    print(json.dumps(res, indent=1))
    if write_json:
        with open(TRAFFIC_FILE, "w") as f:
            json.dump(res, f, indent=1)
            f.write("\n")


def _event_time(fn, steps, warmup):
    """Average ms of fn() over `steps` calls after `warmup`, HIP events on the current stream."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps, (time.perf_counter() - t0) * 1e3 / steps


def bench_decode_mha(args):
    """Llama-2-7B shape MHA decode (B4, 32/32 heads, 16k context: 512 hot +
    15872 warm K4/V2 with outlier_fraction 0.01 -> one fp16 K and one fp16 V
    channel per (batch, block)).  Two distinct layer buffers (302 MB each) are
    rotated so the 256 MB Infinity Cache cannot hold the working set."""
    import torch
    import akv
    from akv import workloads as wl
    from akv.warm_tier import DecodeCall
    s = wl.LLAMA7B_DECODE_16K
    L = args.layers or 2
    dev = "cuda"
    layers = []
    for layer in range(L):
        k, v = wl.make_kv(s, layer, device=dev)
        q = wl.make_q(s, layer, device=dev)
        (kw, vw), (kh, vh) = wl.split_hot_warm(k, v, s.n_hot)
        warm = akv.quantize_kv(kw, vw, s.bits_k, s.bits_v, s.block_t, s.group_v, outlier_fraction=s.outlier_fraction)
        layers.append((q, kh, vh, warm, None))
        del k, v, kw, vw
    torch.cuda.synchronize()
    calls = [DecodeCall(q, kh, vh, w, hot_first=False) for (q, kh, vh, w, _) in layers]
    for c in calls:
        c()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for c in calls:
            c()
    ms, wall_ms = _event_time(g.replay, args.steps, args.warmup)
    us_layer = ms * 1e3 / L
    nb = layer_bytes(s)
    n_out = layers[0][3].k_oidx.shape[-1]
    nblk = (s.n_warm + s.block_t - 1) // s.block_t
    outl = s.B * s.Hkv * s.n_warm * n_out * 2 * 2 + s.B * nblk * n_out * 8 * 2
    alg = nb["attn_total"] + outl
    achieved = alg / (us_layer * 1e-6) / 1e9
    res = {"metric": "decode-attn us/layer + effective KV GB/s (% HBM peak), Llama-2-7B MHA 16k, 1xMI355X",
           "value": round((nb["kv"] + outl) / (us_layer * 1e-6) / 1e9, 2), "unit": "GB/s", "n_gpus": 1,
           "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(wall_ms, 4), "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "f16",
           "data": "synthetic (seeded N(0,1) K/V, 4 channels per head Student-t(3), quantized on the device)",
           "config": {"workload": s.name, "B": s.B, "Hq": s.Hq, "Hkv": s.Hkv, "D": s.D, "context": s.N,
                      "n_hot": s.n_hot, "n_warm": s.n_warm, "bits_k": s.bits_k, "bits_v": s.bits_v,
                      "outlier_fraction": s.outlier_fraction, "n_out": n_out, "layers": L},
           "us_per_layer": round(us_layer, 3),
           "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                        "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": recorded_traffic(s.name),
                        "kernel": "akv_decode_attn per layer (decode_fast_kernel with outlier channels)",
                        "algorithmic_bytes_per_launch": alg, "us_per_launch": round(us_layer, 3)}}
    add_stream_reference(res["roofline"])
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(layers[0], s)
    return res


def bench_prefill(args, causal=False):
    """Chunked prefill, Llama-3-70B attention shape: 512 bf16 queries x 64 heads over
    131072 cached tokens (4096 hot fp16 + 126976 warm at 2/2 bits), batch 1; with
    ``causal`` the chunk's own 512 bf16 keys/values are attended too, position m seeing
    chunk tokens 0..m."""
    import numpy as np
    import torch
    import akv
    from akv import workloads as wl
    from oracle import torch_cpu as otc
    s = wl.LLAMA70B_PREFILL_128K
    print(f"[bench] building {s.name}", file=sys.stderr, flush=True)
    k, v = wl.make_kv(s, device="cuda")
    q = wl.make_q(s, device="cuda", dtype=torch.bfloat16)
    (kw, vw), (kh, vh) = wl.split_hot_warm(k, v, s.n_hot)
    warm = akv.quantize_kv(kw, vw, s.bits_k, s.bits_v, s.block_t, s.group_v)
    del k, v, kw, vw
    kc = vc = None
    if causal:
        gen = torch.Generator(device="cuda").manual_seed(1)
        kc, vc = (torch.randn(s.B, s.Hkv, s.M, s.D, generator=gen, device="cuda").to(torch.bfloat16) for _ in range(2))
    torch.cuda.synchronize()
    ms, wall_ms = _event_time(lambda: akv.prefill_attention(q, kh, vh, warm, k_chunk=kc, v_chunk=vc),
                              args.steps, args.warmup)
    # flops of the attended (query, key) pairs: every cached token, plus chunk tokens 0..m for position m
    flops = 4.0 * s.Hq * s.D * s.B * (s.M * s.N + (s.M * (s.M + 1) // 2 if causal else 0))
    tflops = flops / (ms * 1e-3) / 1e12
    res = {"metric": "chunked-prefill attention TFLOP/s at 128K ctx (Llama-3-70B shape), 1xMI355X" +
                     (", with the chunk's causal self-attention" if causal else ""),
           "value": round(tflops, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": round(wall_ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "dtype": "f16", "data": "synthetic (seeded N(0,1) K/V, bf16 queries, quantized on the device)",
           "config": {"workload": s.name + ("_causal" if causal else ""), "B": s.B, "Hq": s.Hq, "Hkv": s.Hkv,
                      "D": s.D, "M": s.M, "context": s.N, "n_hot": s.n_hot, "n_warm": s.n_warm, "bits_k": s.bits_k,
                      "bits_v": s.bits_v, "causal_chunk": causal},
           "ms_per_call": round(ms, 4),
           "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": 2500.0, "unit": "TFLOP/s",
                        "frac": round(tflops / 2500.0, 4),
                        "traffic": recorded_traffic(s.name + ("_causal" if causal else "")),
                        "kernel": "prefill_kernel (one launch at this shape)", "flops_per_launch": flops}}
    if not args.no_cpu_baseline and not causal:  # the CPU sample is of the cache part only
        # torch CPU restatement: dequant + fp32 attention of kv-head 0's 8 query heads at 16 positions
        host = {n: getattr(warm, n)[:, :1].cpu() for n in ("k_codes", "k_scale", "k_zero", "v_codes", "v_scale",
                                                           "v_zero")}
        host.update(bits_k=s.bits_k, bits_v=s.bits_v, T=s.block_t, G=s.group_v, D=s.D, N=s.n_warm, n_out=0)
        g = s.Hq // s.Hkv
        qs = q[:, :g, :16].cpu()
        khc, vhc = kh[:, :1].cpu(), vh[:, :1].cpu()
        cores = len(os.sched_getaffinity(0))
        threads = torch.get_num_threads()
        torch.set_num_threads(cores)
        reps, t_cpu = 0, 0.0
        try:
            while t_cpu < 10.0 or reps < 3:
                t0 = time.perf_counter()
                kd, vd = otc.dequant_kv_blocked(host)
                otc.decode_attention(qs, khc, vhc, kd, vd, hot_first=True, return_weights=False)
                t_cpu += time.perf_counter() - t0
                reps += 1
        finally:
            torch.set_num_threads(threads)
        f_cpu = 4.0 * g * 16 * s.N * s.D * reps
        res["cpu_baseline"] = {"value": round(f_cpu / t_cpu / 1e12, 6), "unit": "TFLOP/s", "cores": cores,
                               "kind": "port", "sample": f"kv-head 0, 8 query heads x 16 positions, torch CPU: fp16 "
                                                         f"dequant + fp32 attention over 131072 tokens, {reps} runs, "
                                                         f"{t_cpu:.1f} s on {cores} host threads"}
    return res


def bench_demote(args):
    """Demotion: Llama-3-8B GQA shape, 16 x 8 kv-heads x 65536 fp16 tokens; the
    64512 least important tokens per sequence (first 4 and last 16 protected)
    are selected on the device, gathered, quantized per 32-token block and packed."""
    import torch
    import akv
    from akv import workloads as wl
    from akv.drop_in import select_demote_indices
    from threadpoolctl import threadpool_limits
    from oracle import affine as oaff
    s = wl.LLAMA3_DEMOTE_64K
    bits = args.bits
    print(f"[bench] building {s.name}", file=sys.stderr, flush=True)
    k, v, imp = wl.make_demote_inputs(s, device="cuda")
    n = s.S - s.keep_hot
    torch.cuda.synchronize()

    def step():
        sel = select_demote_indices(imp, n, s.S, s.hot_budget)
        return akv.quantize_kv(k, v, bits, bits, s.block_t, s.group_v, sel=sel)

    ms, wall_ms = _event_time(step, args.steps, args.warmup)
    sel_fixed = select_demote_indices(imp, n, s.S, s.hot_budget)
    ms_q, _ = _event_time(lambda: akv.quantize_kv(k, v, bits, bits, s.block_t, s.group_v, sel=sel_fixed),
                          args.steps, 1)
    from akv.warm_tier import packed_row_bytes
    nblk = (n + s.block_t - 1) // s.block_t
    rd = s.B * s.H * n * s.D * 2 * 2 + s.B * s.S * 4
    wr = (s.B * s.H * n * packed_row_bytes(s.D, bits) * 2 + s.B * s.H * nblk * s.D * 2 * 2
          + s.B * s.H * n * (s.D // s.group_v) * 2 * 2 + s.B * n * 8)
    gbps = (rd + wr) / (ms * 1e-3) / 1e9
    res = {"metric": f"demotion quantize+bitpack GB/s at 64K tokens (Llama-3-8B GQA, {bits}-bit), 1xMI355X",
           "value": round(gbps, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": round(wall_ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "dtype": "f16", "data": "synthetic (seeded N(0,1) fp16 K/V, importance U(0,1))",
           "config": {"workload": s.name, "B": s.B, "H": s.H, "D": s.D, "S": s.S, "demoted": n, "bits": bits,
                      "block_t": s.block_t, "group_v": s.group_v},
           "ms_per_call": round(ms, 4),
           "ms_quantize_only": round(ms_q, 4),
           "roofline": {"bound": "hbm", "achieved": round((rd + wr) / (ms_q * 1e-3) / 1e9, 2),
                        "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                        "frac": round((rd + wr) / (ms_q * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                        "traffic": recorded_traffic(s.name) if bits == 3 else None,
                        "kernel": "quant_fast_kernel (gather + quantize + pack, one launch)",
                        "algorithmic_bytes_per_launch": rd + wr,
                        "floor_ms_at_peak": round((rd + wr) / (HBM_PEAK_GBPS * 1e9) * 1e3, 4)}}
    if not args.no_cpu_baseline:
        import numpy as np
        cores = len(os.sched_getaffinity(0))
        sel0 = select_demote_indices(imp[:1], n, s.S, s.hot_budget)[0].cpu().numpy()
        kb = k[:1, :, sel0[:8192]].cpu().numpy()
        vb = v[:1, :, sel0[:8192]].cpu().numpy()
        reps, t_cpu = 0, 0.0
        with threadpool_limits(limits=cores):
            while t_cpu < 10.0 or reps < 3:
                t0 = time.perf_counter()
                oaff.quantize_kv_blocked(kb, vb, bits, bits, s.block_t, s.group_v)
                t_cpu += time.perf_counter() - t0
                reps += 1
        b_cpu = (rd + wr) * (8192 / n) / s.B * reps
        res["cpu_baseline"] = {"value": round(b_cpu / t_cpu / 1e9, 4), "unit": "GB/s", "cores": cores,
                               "kind": "port", "sample": f"sequence 0, 8 kv-heads x 8192 selected tokens "
                                                         f"(quantize + pack), {reps} runs, {t_cpu:.1f} s on {cores} host threads"}
    return res


if __name__ == "__main__":
    main()
