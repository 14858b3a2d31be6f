"""Benchmark of the PACK3D layer forward on one MI355X (BASELINE.json's headline metric).

Workload ("c2"): PACK3D layer forward, bf16, one
64x64x64 volume (262,144 tokens), batch 1, raster order; dim 192, 4 heads,
4 KV heads, head_dim 48, axial RoPE (8, 8, 8) pairs, radius-2 (5x5x5)
neighbourhood, 4x4x4 summary blocks with pool size 1 (4,096 summaries).
Xavier-uniform to_q / to_kv / to_out from seed 0, pool_weight = slot_bias = 0
("mean" pooling), tokens ~ N(0, 1) from seed 1; synthetic data.

A step is one layer forward (LayerNorm, projections, gate, fused core,
to_out, residual) under torch.inference_mode with every input resident in
HBM.  Prints one JSON line; see DESIGN.md for the fields.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "ms per PACK3D layer fwd @262,144 tokens bf16; % of MFMA/HBM roofline"
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E

SHAPE = (64, 64, 64)
DIM, HEADS, KV_HEADS, HEAD_DIM, BLOCK, RADIUS = 192, 4, 4, 48, (4, 4, 4), 2


def build_layer(device, dtype):
    import pack3d_amd as p3d

    torch.manual_seed(0)
    layer = p3d.PACK3DAttention(DIM, heads=HEADS, kv_heads=KV_HEADS, head_dim=HEAD_DIM,
                                block_volume=math.prod(BLOCK))
    for lin in (layer.to_q, layer.to_kv, layer.to_out):
        torch.nn.init.xavier_uniform_(lin.weight)
    with torch.no_grad():
        layer.pool_weight.zero_()
        layer.slot_bias.zero_()
    return layer.to(device, dtype).eval()


def valid_edges(shape, r):
    """Valid local edges of the complete stencil: per axis sum_i |[i-r, i+r] & [0, n)|."""
    total = 1
    for n in shape:
        total *= sum(min(n - 1, i + r) - max(0, i - r) + 1 for i in range(n))
    return total


def time_events(fn, iters, stream):
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(iters):
        fn()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / iters


def cpu_baseline(shape, threads):
    """The oracle (a restatement of the reference CPU path) on a bounded sample.

    The oracle layer is evaluated in fp32 (the reference computes its core in
    fp32 for bf16 inputs, reference.py:18) with all tokens projected, rotated
    and pooled but only S query rows attended; timing two sample sizes gives
    t(S) = fixed + S * per_row, extrapolated to all N rows.
    """
    from oracle import pack3d_oracle as ref

    torch.set_num_threads(threads)
    n = math.prod(shape)
    torch.manual_seed(0)
    layer = ref.PACK3DAttention(DIM, heads=HEADS, kv_heads=KV_HEADS, head_dim=HEAD_DIM,
                                block_volume=math.prod(BLOCK))
    for lin in (layer.to_q, layer.to_kv, layer.to_out):
        torch.nn.init.xavier_uniform_(lin.weight)
    layout = ref.build_layout(shape, BLOCK, radius=RADIUS, pool_size=1, layout="raster_block")
    x = torch.randn(1, n, DIM, generator=torch.Generator().manual_seed(1))
    rows_all = torch.randperm(n, generator=torch.Generator().manual_seed(2))
    sizes = (1024, 4096)
    times = {}
    with torch.inference_mode():
        layer(x, layout, rows=rows_all[:256], chunk=256)  # warm-up
        for s in sizes:
            t0 = time.perf_counter()
            layer(x, layout, rows=rows_all[:s], chunk=512)
            times[s] = time.perf_counter() - t0
    per_row = max(0.0, (times[sizes[1]] - times[sizes[0]]) / (sizes[1] - sizes[0]))
    fixed = max(0.0, times[sizes[0]] - sizes[0] * per_row)
    ms = 1000.0 * (fixed + n * per_row)
    return {"value": round(ms, 1), "unit": "ms/layer", "cores": threads, "kind": "port",
            "sample": (f"oracle layer fwd, fp32, all {n} tokens projected/rotated/pooled, "
                       f"{sizes[0]} and {sizes[1]} query rows attended ({times[sizes[0]]:.2f}s, "
                       f"{times[sizes[1]]:.2f}s); extrapolated linearly in rows to {n}")}


def load_traffic():
    path = os.path.join(ROOT, "profiles", "traffic_attn_fwd_grid_c2.json")
    if os.path.exists(path):
        with open(path) as f:
            return json.load(f).get("bytes_per_launch")
    return None


def main():
    p = argparse.ArgumentParser(description=__doc__)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-threads", type=int, default=min(16, os.cpu_count() or 1))
    a = p.parse_args()
    if a.gpus != 1:
        print("bench.py: this build runs on one GPU only; --gpus must be 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no HIP device visible", file=sys.stderr)
        sys.exit(2)

    import pack3d_amd as p3d
    from pack3d_amd.core import ForwardPlan

    dev = torch.device("cuda:0")
    dtype = torch.bfloat16
    n = math.prod(SHAPE)
    layer = build_layer(dev, dtype)
    layout = p3d.build_layout(SHAPE, BLOCK, radius=RADIUS, pool_size=1, layout="raster_block", device=dev)
    x = torch.randn(1, n, DIM, generator=torch.Generator().manual_seed(1)).to(dev, dtype)
    stream = torch.cuda.current_stream(dev)

    with torch.inference_mode():
        for _ in range(a.warmup):
            layer(x, layout)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(a.steps):
            layer(x, layout)
        torch.cuda.synchronize()
        ms_layer = 1000.0 * (time.perf_counter() - t0) / a.steps

        # Per-kernel durations with HIP events on the launch stream.
        q, kl, vl, kg, vg, gate, rope = layer.core_inputs(x, layout)
        plan = ForwardPlan(q, kl, vl, kg, vg, layer.pool_weight, layer.slot_bias, gate, layer.local_scale,
                           layer.global_scale, layout.geometry, layer.temperature, rope, rope)
        plan.run()
        iters = max(5, a.steps)
        ms_pool = time_events(plan.pool, iters, stream)
        ms_attn = time_events(plan.attention, iters, stream)
        ms_core = time_events(plan.run, iters, stream)

    m = layout.geometry.num_summaries
    edges = valid_edges(SHAPE, RADIUS)
    flops_summary = 4 * HEADS * n * m * HEAD_DIM
    flops_local = 4 * HEADS * edges * HEAD_DIM
    attn_tflops = (flops_summary + flops_local) / (ms_attn * 1e-3) / 1e12
    pool_bytes = 2 * KV_HEADS * n * HEAD_DIM * 2 + 2 * KV_HEADS * m * HEAD_DIM * 2
    pool_gbs = pool_bytes / (ms_pool * 1e-3) / 1e9
    cpu = None if a.no_cpu_baseline else cpu_baseline(SHAPE, a.cpu_threads)
    out = {
        "metric": METRIC, "value": round(ms_layer, 4), "unit": "ms", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(ms_layer, 4), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "c2: PACK3D layer forward, 64^3 volume (262,144 tokens), batch 1, raster",
                   "dim": DIM, "heads": HEADS, "kv_heads": KV_HEADS, "head_dim": HEAD_DIM, "radius": RADIUS,
                   "block": list(BLOCK), "pool_size": 1, "summaries": m, "valid_edges": edges,
                   "tokens_per_s": round(n / (ms_layer * 1e-3)), "ms_layer": round(ms_layer, 4),
                   "ms_core": round(ms_core, 4), "ms_pool_kernel": round(ms_pool, 4),
                   "ms_attn_kernel": round(ms_attn, 4), "parallelism": "single GPU"},
        "roofline": {"kernel": "k_attn_grid (fused local+global forward)", "bound": "mfma",
                     "achieved": round(attn_tflops, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(attn_tflops / PEAK_BF16_TFLOPS, 4), "traffic": load_traffic(),
                     "algorithmic_flops": flops_summary + flops_local},
        "roofline_pool": {"kernel": "k_pool_fwd", "bound": "hbm", "achieved": round(pool_gbs, 1),
                          "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(pool_gbs / PEAK_HBM_GBS, 4),
                          "algorithmic_bytes": pool_bytes},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
