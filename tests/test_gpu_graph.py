"""The layer's no-grad forward captured in a HIP graph (torch.cuda.CUDAGraph).

Serving loops replay a captured step instead of launching its kernels one by
one.  The layer's no-grad path allocates its workspaces from torch (the
capture's private pool), clears them with fill kernels rather than
hipMemsetAsync, and launches every kernel on the current stream without a
host synchronisation once the per-geometry checks are cached, so it can be
captured.  Every replay is checked against the eager output, with eager work
and synchronisations between the replays, and a replay on a new input copied
into the captured input buffer against the eager result on that input.
"""
import math

import pytest
import torch

import pack3d_amd as p3d

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_layer_forward_replays_in_a_graph(gpu, dtype):
    print(f"layer forward in a graph {dtype}", flush=True)
    torch.manual_seed(0)
    shape = (8, 16, 16)
    n = math.prod(shape)
    layer = p3d.PACK3DAttention(192, heads=4, kv_heads=4, head_dim=48, block_volume=64).to(gpu, dtype).eval()
    lay = p3d.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout="raster_block", device=gpu)
    gen = torch.Generator().manual_seed(1)
    x = torch.randn(1, n, 192, generator=gen).to(gpu, dtype)
    x2 = torch.randn(1, n, 192, generator=gen).to(gpu, dtype)
    static_x = x.clone()
    with torch.inference_mode():
        eager = layer(x, lay)  # also fills the per-geometry caches
        eager2 = layer(x2, lay)
        torch.cuda.synchronize()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                layer(static_x, lay)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = layer(static_x, lay)
        for i in range(3):
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), i
            again = layer(x, lay)
            torch.cuda.synchronize()
            assert torch.equal(again, eager), i
        static_x.copy_(x2)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager2)
