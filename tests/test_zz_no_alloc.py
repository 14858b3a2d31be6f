"""p3d_attn_fwd_grid_noalloc against the allocating path (p3d_pool_fwd +
p3d_attn_fwd_grid on caller workspace), through the C ABI: two calls in a
row, the second on a smaller problem, must agree bit for bit (same kernels,
same inputs).  Sizes beyond the scratch array are refused before launch."""
import ctypes
import math

import pytest
import torch

import pack3d_amd as p3d
from pack3d_amd import _lib
from pack3d_amd.core import ForwardPlan
from pack3d_amd.rope import axial_rope
from tests._cases import random_core_inputs

pytestmark = pytest.mark.gpu


def _plan(gpu, shape, batch, kv_heads, dtype, kind, seed):
    lay = p3d.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout=kind, device=gpu)
    n, d = math.prod(shape), 48
    inputs = [t.to(gpu) for t in random_core_inputs(batch, 4, kv_heads, n, d, 64, dtype, seed=seed)]
    rope = axial_rope(d, shape, lay.coords)
    return ForwardPlan(*inputs, lay.geometry, 0.8, rope, rope)


def test_no_alloc_forward_matches_the_allocating_path(gpu):
    cases = [((16, 32, 32), 2, 4, torch.bfloat16, "native_block_morton"),
             ((8, 8, 16), 1, 2, torch.float32, "raster_block")]
    stream = _lib.stream_of(gpu)
    for shape, batch, kv_heads, dtype, kind in cases:
        print(f"no-alloc forward {shape} b{batch} g{kv_heads} {dtype} {kind}", flush=True)
        plan = _plan(gpu, shape, batch, kv_heads, dtype, kind, seed=sum(shape))
        assert plan.grid
        y_ref, _ = plan.run()
        y = torch.full_like(plan.y, float("nan"))
        assert y.stride() == plan.y.stride()
        args = _lib.AttnArgs.from_buffer_copy(plan.attn_args)
        args.y = _lib.view(y)
        args.sk = args.svt = args.sk_norm_max = None
        _lib.call("p3d_attn_fwd_grid_noalloc", plan.pool_args, args, stream)
        torch.cuda.synchronize()
        assert torch.equal(y, y_ref)


def test_no_alloc_forward_refuses_oversized_summaries(gpu):
    plan = _plan(gpu, (8, 8, 16), 1, 2, torch.bfloat16, "raster_block", seed=3)
    pool = _lib.PoolArgs.from_buffer_copy(plan.pool_args)
    args = _lib.AttnArgs.from_buffer_copy(plan.attn_args)
    pool.summaries = args.summaries = 1 << 20
    with pytest.raises(RuntimeError, match="scratch"):
        _lib.call("p3d_attn_fwd_grid_noalloc", pool, args, _lib.stream_of(gpu))
    args.summaries = 7
    with pytest.raises(RuntimeError, match="disagree"):
        _lib.call("p3d_attn_fwd_grid_noalloc", pool, args, _lib.stream_of(gpu))
