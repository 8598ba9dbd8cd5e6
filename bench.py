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
zero bytes read per layer / time per layer), plus us_per_layer, the
roofline of the fused decode op and the CPU baseline (the oracle's
restatement of the reference CPU path on a bounded sample).
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


def cpu_baseline(layer0, s, budget_s=12.0):
    """Oracle restatement of the reference CPU path on layer 0, batch elements
    taken one at a time until ~budget_s seconds of CPU work."""
    import numpy as np
    from threadpoolctl import threadpool_limits
    from oracle import affine as oaff
    from oracle import attention as oatt
    from oracle import importance as oimp
    cores = len(os.sched_getaffinity(0))
    q, kh, vh, warm, _ = layer0
    host = {k: getattr(warm, k).cpu().numpy() for k in ("k_codes", "k_scale", "k_zero", "v_codes", "v_scale", "v_zero")}
    qn, khn, vhn = q.cpu().numpy(), kh.cpu().numpy(), vh.cpu().numpy()
    done, t_cpu = 0, 0.0
    scores = np.zeros(s.N, np.float32)
    with threadpool_limits(limits=cores):
        while done < s.B and t_cpu < budget_s:
            b = done
            w = {k: v[b:b + 1] for k, v in host.items()}
            w.update(bits_k=s.bits_k, bits_v=s.bits_v, T=s.block_t, G=s.group_v, D=s.D, N=s.n_warm, n_out=0)
            t0 = time.perf_counter()
            kd, vd = oaff.dequant_kv_blocked(w)
            _, attn = oatt.mixed_attention_fp32(qn[b:b + 1], khn[b:b + 1], vhn[b:b + 1], kd, vd, hot_first=False)
            scores = oimp.fused_importance_update(attn, scores, 0.9)
            t_cpu += time.perf_counter() - t0
            done += 1
    kv_bytes = layer_bytes(s)["kv"] * done / s.B
    return {"value": round(kv_bytes / t_cpu / 1e9, 4), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"layer 0, {done} of {s.B} sequences (dequant + fp32 attention + importance), "
                      f"{t_cpu:.1f} s on {cores} host threads",
            "us_per_layer_equiv": round(t_cpu / done * s.B * 1e6, 1)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--layers", type=int, default=0, help="override layer count (profiling only)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; the warm-tier path has no multi-GPU leg "
                                   "(see DESIGN.md for how it would shard)", "n_gpus": args.gpus}))
        sys.exit(2)

    import torch
    import akv
    from akv import workloads as wl
    from akv.warm_tier import DecodeCall

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
    alg = nb["attn_total"] + nb["importance"]
    achieved = alg / (us_layer * 1e-6) / 1e9
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
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": None,
                     "kernel": "akv_decode_attn (split + reduce + importance) per layer",
                     "algorithmic_bytes_per_launch": alg},
    }
    if not args.no_cpu_baseline:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        res["cpu_baseline"] = cpu_baseline(layers[0], s)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
