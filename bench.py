"""Benchmark of the PACK3D layer forward on one MI355X (BASELINE.json's headline metric).

Workload ("c2"): PACK3D layer forward, bf16, one
64x64x64 volume (262,144 tokens), batch 1, raster order; dim 192, 4 heads,
4 KV heads, head_dim 48, axial RoPE (8, 8, 8) pairs, radius-2 (5x5x5)
neighbourhood, 4x4x4 summary blocks with pool size 1 (4,096 summaries).
Xavier-uniform to_q / to_kv / to_out from seed 0, pool_weight = slot_bias = 0
("mean" pooling), tokens ~ N(0, 1) from seed 1; synthetic data.

A step is one layer forward (LayerNorm, projections, gate, fused core,
to_out, residual) under torch.inference_mode with every input resident in
HBM.  The layer's output is checked against the oracle layer before the line
is printed (a failed check raises).  The same line carries the c4 layer
forward + backward with its summary-backward kernels, the
incremental peak of allocated bytes of both, and every row of the
reference's own published table of whole-layer latencies (inference and
forward + backward) beside the medians it publishes.  Prints one JSON line.
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
# v_exp_f32 rate of the whole chip, 16 independent chains per wave at four
# waves per SIMD, measured by `bench.py --probe-rates`
# (profiles/issue_rates.md): the transcendental rate of the summary
# pathway's softmax.
PEAK_EXP_PER_S = 16.53e12

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


class _TimedLib:
    """The loaded library with HIP events on the launch stream around the
    named entry points."""

    def __init__(self, real, names, mark):
        self._real, self._names, self._mark = real, names, mark

    def __getattr__(self, name):
        fn = getattr(self._real, name)
        if name not in self._names:
            return fn

        def timed(*args):
            self._mark(name)
            rc = fn(*args)
            self._mark(name)
            return rc
        return timed


def kernel_times_in_layer(layer, x, layout, steps, stream, fused=True):
    """Mean durations (ms) of the layer's launches within layer steps, by
    name: "p3d_project_pool" (projections with the pooling fused in) and
    "attention"; with fused=False the unfused path's "pool" and "attention"
    (the projections are not wrapped there: every wrapped call adds host
    time, and the pool's start event must not wait on the host)."""
    import pack3d_amd.attention as attention
    from pack3d_amd import _lib
    from pack3d_amd.core import ForwardPlan

    marks = {}

    def mark(name):
        ev = torch.cuda.Event(enable_timing=True)
        ev.record(stream)
        marks.setdefault(name, []).append(ev)

    orig = ForwardPlan.pool, ForwardPlan.attention, _lib.lib, attention.pooled_core

    def pool(self):
        mark("pool")
        orig[0](self)
        mark("pool")

    def attn(self):
        mark("attention")
        orig[1](self)
        mark("attention")

    ForwardPlan.pool, ForwardPlan.attention = pool, attn
    if fused:
        timed = _TimedLib(orig[2](), ("p3d_project_pool",), mark)
        _lib.lib = lambda: timed
    else:
        attention.pooled_core = lambda *args: None
    try:
        for _ in range(steps):
            layer(x, layout)
    finally:
        ForwardPlan.pool, ForwardPlan.attention, _lib.lib, attention.pooled_core = orig
    torch.cuda.synchronize()
    return {name: sum(ev[i].elapsed_time(ev[i + 1]) for i in range(0, len(ev), 2)) / steps
            for name, ev in marks.items()}


def layer_ms_unfused(layer, x, layout, steps):
    """The layer step with the projection pooling switched off (p3d_project,
    then p3d_pool_fwd and the attention), for comparison."""
    import pack3d_amd.attention as attention

    real = attention.pooled_core
    attention.pooled_core = lambda *args: None
    try:
        for _ in range(5):
            layer(x, layout)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            layer(x, layout)
        torch.cuda.synchronize()
        return 1000.0 * (time.perf_counter() - t0) / steps
    finally:
        attention.pooled_core = real


def layer_ms_graph(layer, x, layout, warmup, steps):
    """ms per layer step replayed from a HIP graph of one step (captured
    after two warm-up steps on a side stream), and the graph's output."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            layer(x, layout)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = layer(x, layout)
    for _ in range(max(1, warmup)):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        graph.replay()
    torch.cuda.synchronize()
    return 1000.0 * (time.perf_counter() - t0) / steps, out


def summary_pathway_ms(plan, steps, stream):
    """Mean duration (ms) of the summary pathway alone on the plan's inputs.

    The rows kernel runs the same summary pass (rotated queries against all
    summaries on MFMA, fixed Cauchy-Schwarz reference point) and the same
    epilogue as the fused grid kernel, for every query row, in the mode the
    indexed path uses: the local term sl * o_L is read from y (here the
    layer's y, rewritten by every call) and y = that + gate * sg * o_G is
    stored.  Its duration is the summary pathway's cost plus that read of y
    (2 B x H x N x d, 100.7 MB at c2).
    """
    from pack3d_amd import _lib

    a = plan.attn_args
    rows = _lib.AttnArgs.from_buffer_copy(a)
    rows.o_local_in = None
    rows.lse_local = None
    run = lambda: _lib.call("p3d_attn_fwd_rows", rows, stream.cuda_stream)
    run()
    return time_events(run, max(5, steps), stream)


def oracle_layer(layer):
    """The oracle layer (a restatement of the reference CPU path) holding the
    benchmark layer's weights, as rounded to its storage type, in fp32."""
    from oracle import pack3d_oracle as ref

    oracle = ref.PACK3DAttention(DIM, heads=HEADS, kv_heads=KV_HEADS, head_dim=HEAD_DIM,
                                 block_volume=math.prod(BLOCK))
    oracle.load_state_dict({k: v.detach().float().cpu() for k, v in layer.state_dict().items()})
    return oracle


def cpu_baseline(layer, x, shape, threads, repeats=3):
    """The oracle on the whole c2 layer, timed; returns (record, output).

    The oracle layer runs in fp32, as the reference computes its core for
    bf16 inputs (reference.py:18), on the benchmark layer's weights and input
    (bf16 values held in fp32), over every token and every query row (in
    chunks of 512 query rows, which the reference's dense guards would refuse
    at this size).  The value is the median of ``repeats`` runs after a
    warm-up on 256 rows; the last run's output feeds the correctness gate.
    About 4-6 s per run on the GPU box's host.
    """
    from oracle import pack3d_oracle as ref

    torch.set_num_threads(threads)
    n = math.prod(shape)
    oracle = oracle_layer(layer)
    layout = ref.build_layout(shape, BLOCK, radius=RADIUS, pool_size=1, layout="raster_block")
    xf = x.detach().float().cpu()
    times = []
    with torch.inference_mode():
        oracle(xf, layout, rows=torch.arange(256), chunk=256)  # warm-up
        for _ in range(repeats):
            t0 = time.perf_counter()
            out = oracle(xf, layout, chunk=512)
            times.append(time.perf_counter() - t0)
    med = sorted(times)[len(times) // 2]
    record = {"value": round(1000.0 * med, 1), "unit": "ms/layer", "cores": threads, "kind": "port",
              "host_cpus": os.cpu_count(),
              "sample": (f"the whole c2 layer forward (all {n} tokens and query rows) through the oracle in fp32 "
                         f"on {threads} threads (the one-GPU box's CPU share; the host reports {os.cpu_count()} "
                         f"CPUs); median of {repeats} runs ({', '.join(f'{t:.2f}' for t in times)} s)")}
    return record, out


def correctness_gate(layer, x, got, shape, expected=None, sample_rows=8192):
    """The benchmark layer's own output against the oracle layer: the bar of
    the north star (max abs <= 2e-2 in bf16 on unit-scale activations) beyond
    the output's own rounding to bf16 (half an ulp, 2^-8 |y|), on every row
    when ``expected`` (the oracle's whole-layer output) is given, else on
    ``sample_rows`` evenly spaced rows.  Raises when the bar is missed, so a
    broken kernel never reports a time (benchmarks/attention.py:99-114 of
    amilworks/Pack3D gates its timing the same way)."""
    from oracle import pack3d_oracle as ref

    n = math.prod(shape)
    xf = x.detach().float().cpu()
    if expected is None:
        rows = torch.arange(0, n, max(1, n // sample_rows))
        oracle = oracle_layer(layer)
        layout = ref.build_layout(shape, BLOCK, radius=RADIUS, pool_size=1, layout="raster_block")
        with torch.inference_mode():
            expected = oracle(xf, layout, rows=rows, chunk=512)
        got, xf = got[:, rows.to(got.device)], xf[:, rows]
    else:
        rows = None
    got, exp = got.float().cpu(), expected.float()
    diff = (got - exp).abs()
    beyond = float((diff - 2 ** -8 * exp.abs()).max())
    # The attention's share of y (y minus the residual x) as a relative L2.
    rel = float(((got - xf) - (exp - xf)).norm() / (exp - xf).norm())
    gate = {"rows": n if rows is None else int(rows.numel()), "max_abs": round(float(diff.max()), 6),
            "max_abs_beyond_output_rounding": round(beyond, 6), "bar": 2e-2,
            "rel_l2_attention_part": float(f"{rel:.4g}")}
    if not (beyond <= 2e-2 and rel < 3.5e-2):
        raise RuntimeError(f"correctness gate failed: {gate}")
    return gate


TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "traffic_c2.md")


def load_traffic():
    """HBM bytes per launch measured with rocprofv3 FETCH_SIZE / WRITE_SIZE.

    The summary holds one fenced ``json`` block written from two ``--pmc``
    passes over ``bench.py --traffic-probe``; each counter is scaled by what
    it reads for an elementwise copy of known size in the same process.
    """
    if not os.path.exists(TRAFFIC_SUMMARY):
        return {}
    text = open(TRAFFIC_SUMMARY).read()
    start = text.find("```json")
    if start < 0:
        return {}
    body = text[start + len("```json"):text.find("```", start + 7)]
    return json.loads(body)


def traffic_probe():
    """Launch sequence profiled for HBM traffic (run under rocprofv3 --pmc).

    A 1 GiB fill evicts the caches, an elementwise add over 256 MiB gives the
    counter calibration (268,435,456 bytes read and written), then the fused
    projection pooling, the pool and the attention kernels of the c2 workload
    run three times each.
    """
    import pack3d_amd as p3d
    import pack3d_amd.attention as attention
    from pack3d_amd import _lib
    from pack3d_amd.core import ForwardPlan, _projection_views

    dev = torch.device("cuda:0")
    n = math.prod(SHAPE)
    layer = build_layer(dev, torch.bfloat16)
    layout = p3d.build_layout(SHAPE, BLOCK, radius=RADIUS, pool_size=1, layout="raster_block", device=dev)
    x = torch.randn(1, n, DIM, generator=torch.Generator().manual_seed(1)).to(dev, torch.bfloat16)
    flush = torch.empty(256 * 1024 * 1024, dtype=torch.float32, device=dev)
    src = torch.ones(64 * 1024 * 1024, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    with torch.inference_mode():
        q, kl, vl, kg, vg, gate, rope = layer.core_inputs(x, layout)
        plan = ForwardPlan(q, kl, vl, kg, vg, layer.pool_weight, layer.slot_bias, gate, layer.local_scale,
                           layer.global_scale, layout.geometry, layer.temperature, rope, rope)
        made = attention._project_buffers(layer, x)
        fused = ForwardPlan(*_projection_views(made[1], made[2], HEADS, KV_HEADS), layer.pool_weight,
                            layer.slot_bias, made[3].transpose(1, 2), layer.local_scale, layer.global_scale,
                            layout.geometry, layer.temperature, rope, rope)
        stream = _lib.stream_of(dev)
        for _ in range(3):
            flush.fill_(0.0)
            torch.add(src, 1.0, out=dst)
            flush.fill_(0.0)
            fused.pool_args.norms_cleared = 0
            _lib.call("p3d_project_pool", made[0], fused.pool_args, 1, stream)
            flush.fill_(0.0)
            plan.pool()
            plan.attention()
    torch.cuda.synchronize()
    print("traffic probe done", flush=True)


def gather_probe():
    """Launch sequence profiled for the indexed-gather and rotation kernels
    (run under rocprofv3 --kernel-trace / --pmc).

    A 1 GiB fill evicts the caches and an elementwise add over 256 MiB gives
    the counter calibration, as in --traffic-probe; then, three times each,
    the core forward + backward (pack3d_hip_rope, every input differentiated)
    on geometries that carry no grid tag, so that the indexed kernels
    k_local_gather_fwd / _dq / _dkv run (with k_rotate on kl), at:
      * c2: the 64^3 bf16 core inputs of the benchmark layer on the radius-2
        tables of build_layout passed through prepare_geometry (a reference-
        shaped geometry that adopt_layout has not proven);
      * the adapter's Allen-15 shape: 32 x 128 x 64 bf16, 8 query / 2 kv
        heads, head_dim 64, radius 1, (1, 4, 4) blocks, pool 16, N(0, 0.5^2)
        inputs.
    """
    import pack3d_amd as p3d
    from pack3d_amd.rope import axial_rope

    dev = torch.device("cuda:0")
    n = math.prod(SHAPE)
    layer = build_layer(dev, torch.bfloat16)
    layout = p3d.build_layout(SHAPE, BLOCK, radius=RADIUS, pool_size=1, layout="raster_block", device=dev)
    x = torch.randn(1, n, DIM, generator=torch.Generator().manual_seed(1)).to(dev, torch.bfloat16)
    flush = torch.empty(256 * 1024 * 1024, dtype=torch.float32, device=dev)
    src = torch.ones(64 * 1024 * 1024, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    with torch.no_grad():
        q, kl, vl, kg, vg, gate, rope = layer.core_inputs(x, layout)
    c2 = dict(inputs=[t.contiguous() for t in (q, kl, vl, kg, vg)],
              params=[layer.pool_weight.detach(), layer.slot_bias.detach(), gate.contiguous(),
                      layer.local_scale.detach(), layer.global_scale.detach()],
              geometry=p3d.prepare_geometry(layout.geometry.neighbors, layout.geometry.blocks, 1), rope=rope)
    shape15 = (32, 128, 64)
    n15 = math.prod(shape15)
    lay15 = p3d.build_layout(shape15, (1, 4, 4), radius=1, pool_size=16, layout="raster_block", device=dev)
    gen = torch.Generator().manual_seed(15)
    inputs15 = [(torch.randn(1, h, n15, 64, generator=gen) * 0.5).to(dev, torch.bfloat16) for h in (8, 2, 2, 2, 2)]
    params15 = [(torch.randn(64, generator=gen) * 0.2).to(dev), (torch.randn(16, generator=gen) * 0.2).to(dev),
                torch.rand(1, 8, n15, generator=gen).to(dev, torch.bfloat16),
                (1 + 0.1 * torch.randn(64, generator=gen)).to(dev), (0.25 + 0.1 * torch.randn(64, generator=gen)).to(dev)]
    allen = dict(inputs=inputs15, params=params15,
                 geometry=p3d.prepare_geometry(lay15.geometry.neighbors, lay15.geometry.blocks, 16),
                 rope=axial_rope(64, shape15, lay15.coords))
    for case in (c2, allen):
        assert p3d.core.brick_tag(case["geometry"]) is None
    for _ in range(3):
        flush.fill_(0.0)
        torch.add(src, 1.0, out=dst)
        for case in (c2, allen):
            flush.fill_(0.0)
            xs = [t.detach().requires_grad_() for t in case["inputs"]]
            y = p3d.pack3d_hip_rope(*xs, *case["params"], case["geometry"], case["rope"])
            dy = torch.ones_like(y)
            torch.autograd.grad(y, xs, dy)
    torch.cuda.synchronize()
    print("gather probe done", flush=True)


C4_SHAPE = (32, 128, 64)


# Every row of the reference's published table of whole-layer latencies
# (benchmarks/results/h200_vision_2026-11-18.md:7-14 of amilworks/Pack3D: its
# Triton backend on one H200), with the workload of each row as
# benchmarks/vision.py:33-42,62-77 builds it: name, grid, layout, repack,
# precision, batch, small preset, and the published inference and forward +
# backward medians (ms).
VISION_ROWS = (
    ("Raster volume", (32, 128, 64), "raster_block", None, "BF16", 1, False, 4.644, 15.098),
    ("Morton volume", (32, 128, 64), "native_block_morton", None, "BF16", 1, False, 4.638, 15.316),
    ("Raster volume", (32, 128, 64), "raster_block", None, "FP16", 1, False, 4.655, 15.915),
    ("Morton to raster", (16, 64, 64), "native_block_morton", "raster", "BF16", 1, False, 1.044, 4.105),
    ("Morton to random", (16, 64, 64), "native_block_morton", "random", "BF16", 1, False, 1.054, 4.023),
    ("Raster volume", (16, 64, 64), "raster_block", None, "BF16 autocast", 1, False, 1.276, 4.266),
    ("Image slices", (1, 128, 128), "raster_block", None, "BF16", 2, False, 0.746, 3.306),
    ("Small Morton block", (16, 16, 16), "native_block_morton", None, "BF16", 1, True, 0.568, 4.051),
)


def bench_vision_table(warmups=7, repeats=31, only=None):
    """The rows of VISION_ROWS under the protocol of benchmarks/vision.py:
    seed 205 (repack seed 17); dim 512, 8 / 2 heads, head_dim 64, (1, 4, 4)
    blocks, pool 16 (the small row: dim 64, 4 / 2 heads, head_dim 16, (2, 2, 2)
    blocks, pool 4); radius (0, 1, 1) on single-slice grids, else 1; the model
    and input in the named dtype (fp32 under bf16 autocast for the autocast
    row); inference under inference_mode; forward + backward as
    forward(x).backward(dy) with a preallocated dy, the gradients cleared
    outside the timed region; synchronised wall time per step, the median of
    `repeats` steps after `warmups`.  `only`: indices into VISION_ROWS to
    time (all when None)."""
    import statistics
    from contextlib import nullcontext

    import pack3d_amd as p3d

    dev = torch.device("cuda:0")
    rows = []
    for index, (name, grid, order, repack, prec, batch, small, ref_inf, ref_fb) in enumerate(VISION_ROWS):
        if only is not None and index not in only:
            continue
        torch.manual_seed(205)
        if small:
            dim, heads, groups, head_dim, block, pool = 64, 4, 2, 16, (2, 2, 2), 4
        else:
            dim, heads, groups, head_dim, block, pool = 512, 8, 2, 64, (1, 4, 4), 16
        dtype = {"BF16": torch.bfloat16, "FP16": torch.float16, "BF16 autocast": torch.float32}[prec]
        radius = (0, 1, 1) if grid[0] == 1 else (1, 1, 1)
        layout = p3d.build_layout(grid, block, radius=radius, pool_size=pool, layout=order)
        if repack == "raster":
            layout = layout.repack(layout.order.argsort())
        elif repack == "random":
            layout = layout.repack(torch.randperm(len(layout.order), generator=torch.Generator().manual_seed(17)))
        layout = layout.to(dev)
        model = p3d.PACK3DAttention(dim, heads=heads, kv_heads=groups, head_dim=head_dim,
                                    block_volume=math.prod(block)).to(dev, dtype)
        x = torch.randn(batch, math.prod(grid), dim, device=dev, dtype=dtype, requires_grad=True)
        dy = torch.randn_like(x)

        def forward():
            amp = torch.autocast("cuda", torch.bfloat16) if prec == "BF16 autocast" else nullcontext()
            with amp:
                return model(x, layout)

        row = {"workload": name, "batch": batch, "grid": list(grid), "precision": prec}
        for mode, ref in (("inference", ref_inf), ("forward_backward", ref_fb)):
            times = []
            torch.cuda.synchronize()
            for it in range(warmups + repeats):
                start = time.perf_counter()
                if mode == "inference":
                    with torch.inference_mode():
                        forward()
                else:
                    forward().backward(dy)
                torch.cuda.synchronize()
                if it >= warmups:
                    times.append(1000.0 * (time.perf_counter() - start))
                model.zero_grad(set_to_none=True)
                x.grad = None
            ms = statistics.median(times)
            row[f"{mode}_ms"] = round(ms, 4)
            row[f"{mode}_reference_h200_ms"] = ref
            row[f"{mode}_speedup_vs_reference_h200"] = round(ref / ms, 3)
        rows.append(row)
        del model, x, dy, layout
        torch.cuda.empty_cache()
    return rows


def bench_c4(steps, warmup, kernels=False):
    """c4: layer forward + backward on 32 x 128 x 64
    (262,144 tokens), batch 1, raster, bf16 autocast, upstream gradient N(0, 1).
    A step is one forward and one backward to every parameter and the input.
    Also the incremental peak of allocated bytes over a step (as
    benchmarks/attention.py:133-143 of amilworks/Pack3D measures it) and,
    with ``kernels``, the mean durations of the summary dQ and dK/dV passes
    inside the steps (HIP events on the launch stream)."""
    import pack3d_amd as p3d

    dev = torch.device("cuda:0")
    n = math.prod(C4_SHAPE)
    torch.manual_seed(0)
    layer = p3d.PACK3DAttention(DIM, heads=HEADS, kv_heads=KV_HEADS, head_dim=HEAD_DIM,
                                block_volume=math.prod(BLOCK))
    for lin in (layer.to_q, layer.to_kv, layer.to_out):
        torch.nn.init.xavier_uniform_(lin.weight)
    layer = layer.to(dev)
    layout = p3d.build_layout(C4_SHAPE, BLOCK, radius=RADIUS, pool_size=1, layout="raster_block", device=dev)
    x = torch.randn(1, n, DIM, generator=torch.Generator().manual_seed(1)).to(dev).requires_grad_()
    dy = torch.randn(1, n, DIM, generator=torch.Generator().manual_seed(2)).to(dev)

    def step():
        # Gradients start from None each step, as after optimizer.zero_grad()
        # (set_to_none): the step writes them rather than adding to them.
        layer.zero_grad(set_to_none=True)
        x.grad = None
        with torch.autocast("cuda", dtype=torch.bfloat16):
            y = layer(x, layout)
        y.backward(dy)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    ms = 1000.0 * (time.perf_counter() - t0) / steps
    layer.zero_grad(set_to_none=True)
    x.grad = None
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated(dev)
    torch.cuda.reset_peak_memory_stats(dev)
    step()
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated(dev) - base
    out = {"metric": "ms per PACK3D layer fwd+bwd @c4 (32x128x64, 262,144 tokens) bf16 autocast",
           "value": round(ms, 4), "unit": "ms", "n_gpus": 1, "steps": steps, "warmup": warmup,
           "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
           "dtype": "bf16", "data": "synthetic",
           "config": {"workload": "c4: PACK3D layer forward + backward, 32x128x64 volume, batch 1, raster, "
                                  "bf16 autocast", "dim": DIM, "heads": HEADS, "kv_heads": KV_HEADS,
                      "head_dim": HEAD_DIM, "radius": RADIUS, "block": list(BLOCK), "pool_size": 1,
                      "tokens_per_s": round(n / (ms * 1e-3)), "parallelism": "single GPU",
                      "incremental_peak_allocated_bytes": int(peak)}}
    if kernels:
        from pack3d_amd import _lib

        stream = torch.cuda.current_stream(dev)
        marks = {}

        def mark(name):
            ev = torch.cuda.Event(enable_timing=True)
            ev.record(stream)
            marks.setdefault(name, []).append(ev)

        real = _lib.lib
        timed = _TimedLib(real(), ("p3d_global_bwd_dq", "p3d_global_bwd_dkv"), mark)
        _lib.lib = lambda: timed
        try:
            for _ in range(steps):
                step()
        finally:
            _lib.lib = real
        torch.cuda.synchronize()
        times = {name: sum(ev[i].elapsed_time(ev[i + 1]) for i in range(0, len(ev), 2)) / (len(ev) // 2)
                 for name, ev in marks.items()}
        m = layout.geometry.num_summaries
        base_flops = HEADS * n * m * HEAD_DIM
        for key, name, kernel, mult in (
                ("roofline_global_dq", "p3d_global_bwd_dq",
                 "k_global_dq (summary dQ: scores, dP and dQ = dS sk; with the 1.6 MB summary transpose)", 6),
                ("roofline_global_dkv", "p3d_global_bwd_dkv",
                 "k_global_dkv (summary dK/dV: scores, dP, dK = dS^T q, dV = P^T dO)", 8)):
            flops = mult * base_flops
            tf = flops / (times[name] * 1e-3) / 1e12
            out[key] = {"kernel": kernel, "bound": "mfma", "ms": round(times[name], 4), "achieved": round(tf, 2),
                        "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": round(tf / PEAK_BF16_TFLOPS, 4),
                        "algorithmic_flops": flops}
    return out


def probe_rates():
    """Issue rates and co-issue of the units the summary pathway uses
    (p3d_probe_issue_rates of the measurement library libpack3d_probe.so), every operand in registers, at 1, 2 and 4 waves
    per SIMD on every CU: SIMD cycles per wave-iteration (time x the run's
    shader clock / iterations per SIMD) and, for the single kinds, rates per
    second.  The clock comes from the waves' own shader-clock and 100 MHz
    wall-clock counters."""
    from pack3d_amd import _lib

    probe = _lib.probe_lib()
    dev = torch.device("cuda:0")
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    stream = torch.cuda.current_stream(dev)
    iters = 4096
    kinds = {0: "16 exp", 1: "16 fma", 2: "4 mfma", 3: "16 exp + 4 mfma",
             4: "summary tile pattern (2 tiles x 2 blocks: 14 mfma, 32 exp, 16 cvt)"}
    res = {"cus": cus, "iters": iters, "runs": []}
    for wps in (1, 2, 4):
        blocks = wps * cus
        waves = blocks * 4
        cycles = torch.zeros(2 * waves, dtype=torch.int64, device=dev)
        for kind, name in kinds.items():
            if kind == 4 and wps > 2:
                continue  # its registers allow at most 3 waves per SIMD
            def call(n):
                if probe.p3d_probe_issue_rates(kind, n, blocks, cycles.data_ptr(), stream.cuda_stream):
                    raise RuntimeError(probe.p3d_last_error().decode())
            run = lambda: call(iters)
            call(64)
            ms = time_events(run, 3, stream)
            c = cycles.view(-1, 2).double().sum(0).tolist()
            ghz = c[0] / c[1] * 0.1  # shader cycles per 10 ns tick -> GHz
            per_simd = waves * iters / (4 * cus)
            line = {"kind": name, "waves_per_simd": wps, "ms": round(ms, 4), "ghz": round(ghz, 3),
                    "simd_cycles_per_wave_iter": round(ms * 1e-3 * ghz * 1e9 / per_simd, 1)}
            if kind in (0, 1):
                line["lanes_per_s"] = float(f"{waves * 64 * iters * 16 / (ms * 1e-3):.4g}")
            if kind == 2:
                line["mfma_tflops"] = round(waves * iters * 4 * 32 * 32 * 16 * 2 / (ms * 1e-3) / 1e12, 1)
            res["runs"].append(line)
    return res


def main():
    p = argparse.ArgumentParser(description=__doc__)
    p.add_argument("--gpus", type=int, default=1)
    # The GPU's clocks keep rising for the first ~50 ms of sustained work
    # (per-launch times fall by ~15% over that span): the default warm-up
    # covers it, so the timed steps measure the steady state.
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=50)
    p.add_argument("--no-cpu-baseline", action="store_true",
                   help="skip the CPU timing; the correctness gate then checks a sample of rows")
    p.add_argument("--c4-steps", type=int, default=10, help="timed c4 forward + backward steps")
    p.add_argument("--c4-warmup", type=int, default=10)
    p.add_argument("--cpu-threads", type=int, default=min(16, os.cpu_count() or 1))
    p.add_argument("--traffic-probe", action="store_true",
                   help="only run the launch sequence that the HBM traffic counters are collected over")
    p.add_argument("--gather-probe", action="store_true",
                   help="only run the launch sequence the indexed-gather and rotation counters are collected over")
    p.add_argument("--no-presets", action="store_true",
                   help="skip the rows of the reference's published latency table (reported beside the c2 line)")
    p.add_argument("--c4", action="store_true",
                   help="time the c4 layer forward + backward instead (one JSON line of its own)")
    p.add_argument("--probe-rates", action="store_true",
                   help="measure the exp / fma / MFMA issue rates instead (one JSON line of its own)")
    p.add_argument("--vision", metavar="ROWS",
                   help="time only these rows of the reference's published latency table (comma-separated "
                        "indices, 0-7, or 'all'; one JSON line of its own)")
    a = p.parse_args()
    if a.gpus != 1:
        print("bench.py: this build runs on one GPU only; --gpus must be 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no HIP device visible", file=sys.stderr)
        sys.exit(2)
    if a.traffic_probe:
        traffic_probe()
        return
    if a.gather_probe:
        gather_probe()
        return
    if a.c4:
        print(json.dumps(bench_c4(a.steps, a.warmup)), flush=True)
        return
    if a.probe_rates:
        print(json.dumps(probe_rates()), flush=True)
        return
    if a.vision:
        only = None if a.vision == "all" else {int(v) for v in a.vision.split(",")}
        print(json.dumps({"reference_vision_table": bench_vision_table(only=only)}), flush=True)
        return

    import pack3d_amd as p3d
    from pack3d_amd.core import ForwardPlan

    dev = torch.device("cuda:0")
    dtype = torch.bfloat16
    n = math.prod(SHAPE)
    layer = build_layer(dev, dtype)
    layout = p3d.build_layout(SHAPE, BLOCK, radius=RADIUS, pool_size=1, layout="raster_block", device=dev)
    x = torch.randn(1, n, DIM, generator=torch.Generator().manual_seed(1)).to(dev, dtype)
    stream = torch.cuda.current_stream(dev)

    # The c4 forward + backward leg runs first: its few hundred milliseconds
    # of sustained work also bring the GPU to the clocks it holds under load,
    # so that the c2 steps right after it are timed at those clocks rather
    # than on the ramp of a freshly started process.
    c4 = bench_c4(a.c4_steps, a.c4_warmup, kernels=True)
    vision = None if a.no_presets else bench_vision_table()

    with torch.inference_mode():
        for _ in range(a.warmup):
            layer(x, layout)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(a.steps):
            layer(x, layout)
        torch.cuda.synchronize()
        ms_layer = 1000.0 * (time.perf_counter() - t0) / a.steps

        # The same step captured in a HIP graph and replayed (the way a
        # serving loop runs it: no per-kernel launch from the host).
        ms_graph, y_graph = layer_ms_graph(layer, x, layout, a.warmup, a.steps)

        # Per-kernel durations inside the same layer steps: HIP events on the
        # launch stream around the layer's launches (a second pass over the
        # steps, so the first one runs without them); then the layer step with
        # the projection pooling switched off (p3d_project, p3d_pool_fwd, the
        # attention), for comparison, and its pooling launch.
        fused = kernel_times_in_layer(layer, x, layout, a.steps, stream)
        if "p3d_project_pool" not in fused:
            raise RuntimeError("the benchmark layer did not take the fused projection pooling")
        ms_proj_pool, ms_attn = fused["p3d_project_pool"], fused["attention"]
        ms_layer_unfused = layer_ms_unfused(layer, x, layout, a.steps)
        ms_pool = kernel_times_in_layer(layer, x, layout, a.steps, stream, fused=False)["pool"]
        q, kl, vl, kg, vg, gate, rope = layer.core_inputs(x, layout)
        plan = ForwardPlan(q, kl, vl, kg, vg, layer.pool_weight, layer.slot_bias, gate, layer.local_scale,
                           layer.global_scale, layout.geometry, layer.temperature, rope, rope)
        plan.run()
        ms_core = time_events(plan.run, max(5, a.steps), stream)
        ms_summary = summary_pathway_ms(plan, a.steps, stream)

        # Incremental peak of allocated bytes over one layer step (as
        # benchmarks/attention.py:133-143 of amilworks/Pack3D measures it),
        # and the layer's output for the correctness gate.
        del q, kl, vl, kg, vg, gate, rope, plan
        torch.cuda.synchronize()
        base = torch.cuda.memory_allocated(dev)
        torch.cuda.reset_peak_memory_stats(dev)
        y = layer(x, layout)
        torch.cuda.synchronize()
        peak_c2 = torch.cuda.max_memory_allocated(dev) - base
        if not torch.equal(y_graph, y):
            raise RuntimeError("the graph-replayed layer step differs from the eager step")

    m = layout.geometry.num_summaries
    edges = valid_edges(SHAPE, RADIUS)
    flops_summary = 4 * HEADS * n * m * HEAD_DIM
    flops_local = 4 * HEADS * edges * HEAD_DIM
    attn_tflops = (flops_summary + flops_local) / (ms_attn * 1e-3) / 1e12
    exps = HEADS * n * m + HEADS * edges  # one exponential per (query, summary) and per valid edge
    exp_rate = exps / (ms_attn * 1e-3)
    pool_bytes = 2 * KV_HEADS * n * HEAD_DIM * 2 + 2 * KV_HEADS * m * HEAD_DIM * 2
    pool_gbs = pool_bytes / (ms_pool * 1e-3) / 1e9
    # The fused projection kernel's compulsory HBM bytes: x read; q, kl, vl,
    # the gate and the summaries written (the weights are a few hundred KB).
    proj_pool_bytes = (n * DIM + n * HEADS * HEAD_DIM + 2 * n * KV_HEADS * HEAD_DIM + n * HEADS
                       + 2 * KV_HEADS * m * HEAD_DIM) * 2
    proj_pool_gbs = proj_pool_bytes / (ms_proj_pool * 1e-3) / 1e9
    if a.no_cpu_baseline:
        cpu = None
        gate = correctness_gate(layer, x, y, SHAPE)
    else:
        cpu, expected = cpu_baseline(layer, x, SHAPE, a.cpu_threads)
        gate = correctness_gate(layer, x, y, SHAPE, expected)
    traffic = load_traffic()
    out = {
        "metric": METRIC, "value": round(ms_layer, 4), "unit": "ms", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(ms_layer, 4), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "c2: PACK3D layer forward, 64^3 volume (262,144 tokens), batch 1, raster",
                   "dim": DIM, "heads": HEADS, "kv_heads": KV_HEADS, "head_dim": HEAD_DIM, "radius": RADIUS,
                   "block": list(BLOCK), "pool_size": 1, "summaries": m, "valid_edges": edges,
                   "tokens_per_s": round(n / (ms_layer * 1e-3)), "ms_layer": round(ms_layer, 4),
                   "ms_core": round(ms_core, 4), "ms_project_pool_kernel": round(ms_proj_pool, 4),
                   "ms_attn_kernel": round(ms_attn, 4), "ms_summary_pathway": round(ms_summary, 4),
                   "ms_layer_graph": round(ms_graph, 4),
                   "ms_layer_unfused": round(ms_layer_unfused, 4),
                   "ms_pool_kernel_unfused_layer": round(ms_pool, 4),
                   "incremental_peak_allocated_bytes": int(peak_c2),
                   "parallelism": "single GPU"},
        "correctness_gate": gate,
        "roofline": {"kernel": "k_attn_grid (fused local+global forward)", "bound": "mfma",
                     "achieved": round(attn_tflops, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(attn_tflops / PEAK_BF16_TFLOPS, 4), "traffic": traffic.get("attn_bytes_per_launch"),
                     "algorithmic_flops": flops_summary + flops_local},
        "roofline_exp": {"kernel": "k_attn_grid", "bound": "valu-transcendental", "achieved": float(f"{exp_rate:.4g}"),
                         "peak": PEAK_EXP_PER_S, "unit": "exp/s", "frac": round(exp_rate / PEAK_EXP_PER_S, 4),
                         "algorithmic_exps": exps},
        "roofline_summary": {"kernel": "k_attn_rows (summary pathway + epilogue, local term read from y)",
                             "bound": "mfma", "achieved": round(flops_summary / (ms_summary * 1e-3) / 1e12, 2),
                             "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                             "frac": round(flops_summary / (ms_summary * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                             "algorithmic_flops": flops_summary},
        "roofline_pool": {"kernel": "k_pool_fwd (the unfused pooling: training, other layouts), inside the "
                                    "unfused layer step", "bound": "hbm", "achieved": round(pool_gbs, 1),
                          "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(pool_gbs / PEAK_HBM_GBS, 4),
                          "traffic": traffic.get("pool_bytes_per_launch"),
                          "algorithmic_bytes": pool_bytes},
        "roofline_project_pool": {"kernel": "k_project_pool (LayerNorm, projections, gate and summary pooling, "
                                            "in the layer)", "bound": "hbm", "achieved": round(proj_pool_gbs, 1),
                                  "peak": PEAK_HBM_GBS, "unit": "GB/s",
                                  "frac": round(proj_pool_gbs / PEAK_HBM_GBS, 4),
                                  "traffic": traffic.get("project_pool_bytes_per_launch"),
                                  "algorithmic_bytes": proj_pool_bytes},
        "c4_fwd_bwd": {"workload": c4["config"]["workload"], "ms": c4["value"], "steps": c4["steps"],
                       "warmup": c4["warmup"], "tokens_per_s": c4["config"]["tokens_per_s"],
                       "incremental_peak_allocated_bytes": c4["config"]["incremental_peak_allocated_bytes"]},
        "roofline_global_dq": c4["roofline_global_dq"],
        "roofline_global_dkv": c4["roofline_global_dkv"],
        "reference_vision_table": vision,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
