"""The reference benchmark's own presets (benchmarks/attention.py:84-91 of
amilworks/Pack3D) through the HIP layer, gated the way that harness gates a
backend before it times one (:99-114): on a small probe grid, the output and
the gradients of the input and of every parameter against the oracle layer,
relative L2 below the harness's bar for bf16 (3.5e-2).

The HIP layer runs in bf16 (weights and input, as ``model.to(dtype)`` holds
them there), or in fp32 under bf16 autocast (benchmarks/vision.py:40,79,95: the
"BF16 autocast" row); the oracle runs in fp32 on the CPU with the same
weights and input (rounded to bf16 for the bf16 layer).
"""
import math

import pytest
import torch

import oracle.pack3d_oracle as ref
import pack3d_amd as p3d
from tests._cases import rel_l2

pytestmark = pytest.mark.gpu

PRESETS = {
    # dim, heads, kv_heads, head_dim, block, pool_size, layout, probe grid
    "allen15": (512, 8, 2, 64, (1, 4, 4), 16, "raster_block", (4, 8, 16)),
    "small": (64, 4, 2, 16, (2, 2, 2), 4, "native_block_morton", (4, 4, 4)),
}


@pytest.mark.parametrize("precision", ["bf16", "autocast"])
@pytest.mark.parametrize("preset", sorted(PRESETS))
def test_reference_benchmark_preset_probe(gpu, preset, precision):
    dim, heads, kv_heads, head_dim, block, pool, order, grid = PRESETS[preset]
    print(f"preset {preset} {precision} probe {grid}", flush=True)
    autocast = precision == "autocast"
    dt = torch.float32 if autocast else torch.bfloat16
    torch.manual_seed(31)
    oracle = ref.PACK3DAttention(dim, heads=heads, kv_heads=kv_heads, head_dim=head_dim,
                                 block_volume=math.prod(block))
    with torch.no_grad():
        for prm in oracle.parameters():
            prm.copy_(prm.to(dt).float())
    layer = p3d.PACK3DAttention(dim, heads=heads, kv_heads=kv_heads, head_dim=head_dim,
                                block_volume=math.prod(block))
    layer.load_state_dict(oracle.state_dict())
    layer = layer.to(gpu, dt)
    lay_h = p3d.build_layout(grid, block, radius=1, pool_size=pool, layout=order, device=gpu)
    lay_r = ref.build_layout(grid, block, radius=1, pool_size=pool, layout=order)
    n = math.prod(grid)
    x = torch.randn(1, n, dim, generator=torch.Generator().manual_seed(1)).to(dt)
    dy = torch.randn(1, n, dim, generator=torch.Generator().manual_seed(2))
    xh = x.to(gpu).requires_grad_()
    xr = x.float().requires_grad_()
    with torch.autocast("cuda", torch.bfloat16, enabled=autocast):
        with torch.inference_mode():
            yi = layer(xh.detach(), lay_h)
        yh = layer(xh, lay_h)
    yr = oracle(xr, lay_r)
    yh.backward(dy.to(gpu, yh.dtype))
    yr.backward(dy)
    assert yi.dtype == yh.dtype == dt
    checks = [("inference output", yi, yr), ("output", yh, yr), ("input", xh.grad, xr.grad)]
    expected = dict(oracle.named_parameters())
    checks += [(name, prm.grad, expected[name].grad) for name, prm in layer.named_parameters()]
    for name, got, exp in checks:
        assert got is not None and torch.isfinite(got.float()).all(), name
        err = rel_l2(got.float(), exp)
        print(f"  {name}: rel_l2={err:.3g}", flush=True)
        assert err < 3.5e-2, (name, err)
