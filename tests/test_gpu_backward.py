"""Backward parity of the HIP path with the oracle's autograd (reference.py restated).

Bars as in the reference's own gradient tests (tests/test_triton.py:72-95):
relative L2 below 3e-5 / 5e-3 / 3.5e-2 for fp32 / fp16 / bf16 on every
gradient, and assert_close(3e-5) in fp32.
"""
import math

import pytest
import torch

import oracle.pack3d_oracle as ref
import pack3d_amd as p3d
from pack3d_amd.rope import axial_rope as hip_axial
from tests._cases import make_case, random_core_inputs, rel_l2

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 3e-5, torch.float16: 5e-3, torch.bfloat16: 3.5e-2}
NAMES = ["q", "kl", "vl", "kg", "vg", "pool_weight", "slot_bias", "gate", "local_scale", "global_scale"]


def _compare(got, exp, dtype, what):
    # The largest expected gradient entry: the scale of the rounding in the
    # kernels' gradients.
    scale = max(float(e.float().abs().max()) for e in exp)
    for name, a, e in zip(NAMES, got, exp):
        assert torch.isfinite(a).all(), (what, name)
        mx = (a.float().cpu() - e.float()).abs().max().item()
        if dtype == torch.float32:
            torch.testing.assert_close(a.cpu(), e, atol=3e-5, rtol=3e-5)
        if float(e.float().norm()) == 0.0:
            # An exactly zero gradient (radius 0: each local softmax has one
            # key, so its scores get no gradient): the kernels' rounding,
            # against the scale of the other gradients.
            print(f"  {what} d{name}: expected zero, max_abs={mx:.3g} (scale {scale:.3g})", flush=True)
            assert mx <= TOL[dtype] * scale, (what, name, mx, scale)
            continue
        err = rel_l2(a.float().cpu(), e.float())
        print(f"  {what} d{name}: rel_l2={err:.3g} max_abs={mx:.3g}", flush=True)
        assert err < TOL[dtype], (what, name, err)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape", [(37, 16, 2, 4, 2, 4, 3), (131, 64, 1, 8, 2, 16, 2), (19, 32, 1, 2, 2, 3, 1),
                                   (21, 128, 1, 2, 1, 4, 4), (67, 48, 1, 4, 4, 8, 1), (136, 48, 2, 4, 2, 8, 2)])
def test_every_gradient_custom_graph(gpu, dtype, shape):
    print(f"backward custom {shape} {dtype}", flush=True)
    inputs, nb, blocks, pool = make_case(*shape, dtype=dtype)
    og = ref.prepare_geometry(nb, blocks, pool)
    hg = p3d.prepare_geometry(nb.to(gpu), blocks.to(gpu), pool)
    xs = [t.to(gpu).requires_grad_() for t in inputs]
    rs = [t.detach().clone().requires_grad_() for t in inputs]
    y = p3d.pack3d_hip(*xs, hg, temperature=0.7)
    e = ref.pack3d_reference(*rs, og, temperature=0.7)
    up = torch.randn(e.shape, generator=torch.Generator().manual_seed(91)).to(dtype)
    got = torch.autograd.grad(y, xs, up.to(gpu))
    exp = torch.autograd.grad(e, rs, up)
    _compare(got, exp, dtype, f"custom {shape}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("b,h,n,d", [(1, 1, 8, 8), (2, 3, 136, 48), (1, 4, 64, 128)])
def test_transpose_rows(gpu, dtype, b, h, n, d):
    """p3d_transpose_rows (the transposed q / dO_G copies of the summary dK/dV
    pass) is an exact transpose, also from a token-major strided view."""
    print(f"transpose_rows b{b} h{h} n{n} d{d} {dtype}", flush=True)
    from pack3d_amd import _lib
    x = torch.randn(b, n, h, d, generator=torch.Generator().manual_seed(n + d)).to(gpu, dtype)
    src = x.permute(0, 2, 1, 3)  # [B, H, N, d] view, row stride H d
    out = torch.full((b * h * d * n,), float("nan"), dtype=dtype, device=gpu)
    _lib.call("p3d_transpose_rows", _lib.view(src), out.data_ptr(), b, h, n, d, _lib.DTYPES[dtype],
              _lib.stream_of(gpu))
    torch.cuda.synchronize()
    exp = src.transpose(2, 3).reshape(-1)
    assert torch.equal(out.view(torch.int16), exp.contiguous().view(torch.int16))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("kind,kv_heads", [("native_block_morton", 2), ("raster_block", 4)])
def test_every_gradient_grid_rope_fused(gpu, dtype, kind, kv_heads):
    """A complete-grid layout (brick forward) with the rotation fused: the
    gradients of q, kl, kg are those of the unrotated projections."""
    print(f"backward grid {kind} g{kv_heads} {dtype}", flush=True)
    shape, d = (8, 8, 12), 48
    n = math.prod(shape)
    lay_h = p3d.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout=kind)
    lay_r = ref.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout=kind)
    inputs = random_core_inputs(1, 4, kv_heads, n, d, 64, dtype, seed=23)
    xs = [t.to(gpu).requires_grad_() for t in inputs]
    rs = [t.detach().clone().requires_grad_() for t in inputs]
    y = p3d.pack3d_hip_rope(*xs, lay_h.geometry, hip_axial(d, shape, lay_h.coords), temperature=0.8)
    rot = [ref.axial_rope(t, lay_r.coords) if i in (0, 1, 3) else t for i, t in enumerate(rs)]
    e = ref.pack3d_reference(*rot, lay_r.geometry, temperature=0.8)
    up = torch.randn(e.shape, generator=torch.Generator().manual_seed(5)).to(dtype)
    got = torch.autograd.grad(y, xs, up.to(gpu))
    exp = torch.autograd.grad(e, rs, up)
    _compare(got, exp, dtype, f"grid {kind}")


@pytest.mark.parametrize("spread", [False, True])
def test_summary_dq_reference_point_paths(gpu, spread):
    """The summary dQ pass forms dS against one reference point per wave (the
    largest lse of its 64 queries) unless a query's lse lies more than 64
    log2 units below it.  spread=True scales the first query of every wave
    by 200, which puts its summary lse 35-97 log2 units above the rest of
    the wave (computed with the oracle's pooling): some waves take the
    per-query path, the others the reference point near its limit.  Every
    gradient against the oracle."""
    dtype = torch.bfloat16
    print(f"backward dq reference point spread={spread}", flush=True)
    inputs, nb, blocks, pool = make_case(n=256, d=48, b=1, h=2, g=1, volume=8, pool=1, dtype=torch.float32, seed=7)
    if spread:
        q = inputs[0].clone()
        q[:, :, ::64] *= 200.0
        inputs = (q,) + tuple(inputs[1:])
    inputs = tuple(t.to(dtype) for t in inputs)
    og = ref.prepare_geometry(nb, blocks, pool)
    hg = p3d.prepare_geometry(nb.to(gpu), blocks.to(gpu), pool)
    xs = [t.to(gpu).requires_grad_() for t in inputs]
    rs = [t.detach().clone().requires_grad_() for t in inputs]
    y = p3d.pack3d_hip(*xs, hg, temperature=0.7)
    e = ref.pack3d_reference(*rs, og, temperature=0.7)
    up = torch.randn(e.shape, generator=torch.Generator().manual_seed(3)).to(dtype)
    got = torch.autograd.grad(y, xs, up.to(gpu))
    exp = torch.autograd.grad(e, rs, up)
    _compare(got, exp, dtype, f"dq reference point spread={spread}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_singleton_summary_has_no_query_or_key_gradient(gpu, dtype):
    """One token, one summary: the local row is empty and attention to a single
    summary is its value, so q, kl, vl, kg and the pooling parameters get
    exactly zero gradient (tests/test_triton.py:262-271)."""
    inputs, nb, blocks, pool = make_case(n=1, d=16, b=1, h=1, g=1, volume=1, pool=1, dtype=dtype)
    hg = p3d.prepare_geometry(nb.to(gpu), blocks.to(gpu), pool)
    xs = [t.to(gpu).requires_grad_() for t in inputs]
    y = p3d.pack3d_hip(*xs, hg)
    grads = torch.autograd.grad(y, xs, torch.randn_like(y))
    for index in (0, 1, 2, 3, 5, 6):
        assert torch.count_nonzero(grads[index]) == 0, (index, grads[index].abs().max().item())


def test_mutated_saved_geometry_fails_backward(gpu):
    inputs, nb, blocks, pool = make_case()
    hg = p3d.prepare_geometry(nb.to(gpu), blocks.to(gpu), pool)
    xs = [t.to(gpu).requires_grad_() for t in inputs]
    y = p3d.pack3d_hip(*xs, hg)
    hg.neighbors[1, 0] = 1
    with pytest.raises(RuntimeError, match="changed"):
        y.sum().backward()


def test_repeated_backward_is_deterministic(gpu):
    inputs, nb, blocks, pool = make_case(131, 64, 1, 8, 2, 16, 2)
    hg = p3d.prepare_geometry(nb.to(gpu), blocks.to(gpu), pool)
    xs = [t.to(gpu).requires_grad_() for t in inputs]
    y = p3d.pack3d_hip(*xs, hg)
    dy = torch.randn_like(y)
    g1 = torch.autograd.grad(y, xs, dy, retain_graph=True)
    g2 = torch.autograd.grad(y, xs, dy)
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)


def test_layer_gradients_match_oracle(gpu):
    """The whole layer in fp32 on an anisotropic grid: input and every
    parameter gradient against the oracle layer under the same weights."""
    print("layer backward", flush=True)
    torch.manual_seed(0)
    shape = (4, 16, 8)
    oracle = ref.PACK3DAttention(192, heads=4, kv_heads=2, head_dim=48, block_volume=64)
    layer = p3d.PACK3DAttention(192, heads=4, kv_heads=2, head_dim=48, block_volume=64)
    layer.load_state_dict(oracle.state_dict())
    layer = layer.to(gpu)
    lay_h = p3d.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout="raster_block")
    lay_r = ref.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout="raster_block")
    x = torch.randn(1, math.prod(shape), 192, generator=torch.Generator().manual_seed(1))
    xh = x.to(gpu).requires_grad_()
    xr = x.clone().requires_grad_()
    dy = torch.randn(x.shape, generator=torch.Generator().manual_seed(2))
    layer(xh, lay_h).backward(dy.to(gpu))
    oracle(xr, lay_r).backward(dy)
    torch.testing.assert_close(xh.grad.cpu(), xr.grad, atol=3e-5, rtol=3e-5)
    expected = dict(oracle.named_parameters())
    for name, p in layer.named_parameters():
        err = rel_l2(p.grad.cpu(), expected[name].grad)
        print(f"  layer {name}: rel_l2={err:.3g}", flush=True)
        assert err < 1e-4, (name, err)


def test_full_size_c4_backward(gpu):
    """c4: 32 x 128 x 64 (262,144 tokens), bf16 under autocast, through the
    layer's projections: the core output and all ten gradients against the
    oracle's autograd (pack3d_reference_grads, chunked over query rows) on
    every row, at the reference's bf16 relative-L2 bar
    (tests/test_triton.py:83); the rotation's backward for q, kl, kg is the
    oracle's autograd of axial_rope."""
    print("full size c4 backward", flush=True)
    torch.manual_seed(0)
    shape = (32, 128, 64)
    n = math.prod(shape)
    layer = p3d.PACK3DAttention(192, heads=4, kv_heads=4, head_dim=48, block_volume=64)
    for lin in (layer.to_q, layer.to_kv, layer.to_out):
        torch.nn.init.xavier_uniform_(lin.weight)
    layer = layer.to(gpu)
    lay = p3d.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout="raster_block")
    x = torch.randn(1, n, 192, generator=torch.Generator().manual_seed(1)).to(gpu)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        q, kl, vl, kg, vg, gate, rope = layer.core_inputs(x, lay)
    core = [t.detach().requires_grad_() for t in (q, kl, vl, kg, vg)]
    params = [layer.pool_weight, layer.slot_bias, gate.detach().requires_grad_(), layer.local_scale,
              layer.global_scale]
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = p3d.pack3d_hip_rope(*core, *params, lay.geometry, rope)
    dy = torch.randn(y.shape, generator=torch.Generator().manual_seed(2)).to(gpu, y.dtype)
    got = torch.autograd.grad(y, core + params, dy)

    lay_r = ref.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout="raster_block")
    leaves = [t.detach().cpu().requires_grad_() for t in (q, kl, vl, kg, vg)]
    rot = [ref.axial_rope(t, lay_r.coords) if i in (0, 1, 3) else t for i, t in enumerate(leaves)]
    pcpu = [t.detach().cpu() for t in params]
    rot_in = [t.detach() for t in rot]
    exp_y = ref.pack3d_reference(*rot_in, *pcpu, lay_r.geometry, chunk=4096)
    _compare_one("y", y, exp_y, torch.bfloat16)
    grads = ref.pack3d_reference_grads(*rot_in, *pcpu, lay_r.geometry, dy.cpu(), chunk=2048)
    torch.autograd.backward([rot[0], rot[1], rot[3]], [grads[0], grads[1], grads[3]])
    exp = [leaves[0].grad, leaves[1].grad, grads[2], leaves[3].grad, grads[4], *grads[5:]]
    _compare(got, exp, torch.bfloat16, "c4")


def _compare_one(name, a, e, dtype):
    assert torch.isfinite(a).all(), name
    err = rel_l2(a.float().cpu(), e.float())
    mx = (a.float().cpu() - e.float()).abs().max().item()
    print(f"  {name}: rel_l2={err:.3g} max_abs={mx:.3g}", flush=True)
    assert err < TOL[dtype], (name, err)


from tests.test_gpu_forward import GRIDS  # noqa: E402


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape,block,radius,kind,heads,kv_heads,d", GRIDS)
def test_every_gradient_grid_shapes(gpu, dtype, shape, block, radius, kind, heads, kv_heads, d):
    """Complete-grid layouts of every radius pattern and partial bricks (the
    brick-tiled local backward), against the oracle's autograd."""
    print(f"backward grid {shape} {block} {radius} {kind} h{heads} g{kv_heads} d{d} {dtype}", flush=True)
    lay_h = p3d.build_layout(shape, block, radius=radius, pool_size=1, layout=kind)
    lay_r = ref.build_layout(shape, block, radius=radius, pool_size=1, layout=kind)
    n, vol = math.prod(shape), math.prod(block)
    inputs = random_core_inputs(1, heads, kv_heads, n, d, vol, dtype, seed=n + 3 * d)
    xs = [t.to(gpu).requires_grad_() for t in inputs]
    rs = [t.detach().clone().requires_grad_() for t in inputs]
    y = p3d.pack3d_hip(*xs, lay_h.geometry, temperature=0.9)
    e = ref.pack3d_reference(*rs, lay_r.geometry, temperature=0.9)
    up = torch.randn(e.shape, generator=torch.Generator().manual_seed(17)).to(dtype)
    got = torch.autograd.grad(y, xs, up.to(gpu))
    exp = torch.autograd.grad(e, rs, up)
    _compare(got, exp, dtype, f"grid {shape}")


def _c4_layer(shape, gpu, seed=0):
    """The c4 benchmark layer (bench.py --c4): Xavier projections from
    ``seed``, default pooling, gate and LayerNorm parameters; fp32 parameters
    on the GPU under bf16 autocast, and the oracle layer on the same weights."""
    torch.manual_seed(seed)
    layer = p3d.PACK3DAttention(192, heads=4, kv_heads=4, head_dim=48, block_volume=64)
    for lin in (layer.to_q, layer.to_kv, layer.to_out):
        torch.nn.init.xavier_uniform_(lin.weight)
    oracle = ref.PACK3DAttention(192, heads=4, kv_heads=4, head_dim=48, block_volume=64)
    oracle.load_state_dict(layer.state_dict())
    return layer.to(gpu), oracle


def _autocast_layer_vs_oracle(gpu, shape, what, chunk):
    """The layer under bf16 autocast over an fp32 input, as the c4 step runs
    it (LayerNormTrain, the fused projections, _Pack3DProjections with view
    outputs, OutputResidualWide, the HIP weight gradients): output, dx and
    every parameter gradient against the oracle layer's fp32 gradients, at
    the reference's bf16 relative-L2 bar (tests/test_triton.py:83)."""
    from tests._cases import oracle_layer_grads

    n = math.prod(shape)
    layer, oracle = _c4_layer(shape, gpu)
    lay_h = p3d.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout="raster_block")
    lay_r = ref.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout="raster_block")
    x = torch.randn(1, n, 192, generator=torch.Generator().manual_seed(1))
    dy = torch.randn(1, n, 192, generator=torch.Generator().manual_seed(2))
    xh = x.to(gpu).requires_grad_()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = layer(xh, lay_h)
    y.backward(dy.to(gpu))
    torch.cuda.synchronize()
    exp_y, exp_dx, exp_named = oracle_layer_grads(oracle, x, lay_r, dy, chunk=chunk)
    got = {"y - x": (y.float().cpu() - x), "dx": xh.grad.cpu()}
    exp = {"y - x": exp_y - x, "dx": exp_dx}
    for name, p in layer.named_parameters():
        got[name] = p.grad.cpu()
        exp[name] = exp_named[name]
    for name in got:
        a, e = got[name], exp[name]
        assert a is not None and torch.isfinite(a).all(), (what, name)
        err = rel_l2(a.float(), e.float())
        print(f"  {what} {name}: rel_l2={err:.3g}", flush=True)
        assert err < TOL[torch.bfloat16], (what, name, err)


def test_layer_autocast_gradients_match_oracle(gpu):
    """The c4 path on a small anisotropic grid (8 x 16 x 16)."""
    print("layer autocast backward 8x16x16", flush=True)
    _autocast_layer_vs_oracle(gpu, (8, 16, 16), "autocast 8x16x16", chunk=512)


def test_full_size_c4_layer_gradients(gpu):
    """c4 at full size (32 x 128 x 64, 262,144 tokens): the layer's output,
    dx and the gradients of LayerNorm, to_q, to_kv, the gate, the pooling,
    the scales and to_out against the oracle, whose core is differentiated
    chunk by chunk over query rows."""
    print("full size c4 layer backward", flush=True)
    _autocast_layer_vs_oracle(gpu, (32, 128, 64), "c4 layer", chunk=2048)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape,block,pool,kind", [
    ((4, 6, 10), (1, 1, 2), 5, "raster_block"),          # 2 slots: 32 fine blocks per pooling step
    ((6, 8, 10), (2, 2, 2), 3, "native_block_morton"),   # 8 slots
    ((5, 16, 16), (1, 4, 4), 16, "raster_block"),        # 16 slots, pool 16 (the allen15 preset's)
    ((4, 8, 12), (2, 4, 4), 5, "raster_block"),          # 32 slots, a partial last summary
    ((6, 9, 9), (3, 3, 3), 4, "raster_block"),           # 27 slots: one block per step
])
def test_every_gradient_pooled_grids(gpu, dtype, shape, block, pool, kind):
    """Summaries of several fine blocks (pool_size > 1), with the pooling
    forward and backward packing 64 / V blocks into a 64-lane step when V is
    a power of two: every gradient against the oracle's autograd."""
    print(f"backward pooled {shape} {block} pool {pool} {kind} {dtype}", flush=True)
    lay_h = p3d.build_layout(shape, block, radius=1, pool_size=pool, layout=kind)
    lay_r = ref.build_layout(shape, block, radius=1, pool_size=pool, layout=kind)
    n, vol = math.prod(shape), math.prod(block)
    inputs = random_core_inputs(2, 4, 2, n, 32, vol, dtype, seed=n + vol + pool)
    xs = [t.to(gpu).requires_grad_() for t in inputs]
    rs = [t.detach().clone().requires_grad_() for t in inputs]
    y = p3d.pack3d_hip(*xs, lay_h.geometry, temperature=0.8)
    e = ref.pack3d_reference(*rs, lay_r.geometry, temperature=0.8)
    up = torch.randn(e.shape, generator=torch.Generator().manual_seed(19)).to(dtype)
    got = torch.autograd.grad(y, xs, up.to(gpu))
    exp = torch.autograd.grad(e, rs, up)
    _compare(got, exp, dtype, f"pooled {shape}")


def test_full_size_allen15_layer_gradients_match_oracle(gpu):
    """Forward + backward of the reference benchmark's allen15 preset at the
    size of its published table's first row (dim 512, 8 / 2 heads, head_dim
    64, (1, 4, 4) blocks, pool 16, radius 1, 32 x 128 x 64 = 262,144 tokens,
    bf16 storage): the output, the input gradient and every parameter
    gradient against the oracle layer's autograd on the same (rounded)
    weights and input, relative L2 within the reference's bf16 bar."""
    import oracle.pack3d_oracle as ref_mod
    print("full size allen15 layer gradients vs oracle", flush=True)
    shape, block = (32, 128, 64), (1, 4, 4)
    n = math.prod(shape)
    torch.manual_seed(205)
    layer = p3d.PACK3DAttention(512, heads=8, kv_heads=2, head_dim=64, block_volume=16).to(gpu, torch.bfloat16)
    oracle = ref_mod.PACK3DAttention(512, heads=8, kv_heads=2, head_dim=64, block_volume=16)
    oracle.load_state_dict({k: v.detach().float().cpu() for k, v in layer.state_dict().items()})
    lay = p3d.build_layout(shape, block, radius=1, pool_size=16, layout="raster_block", device=gpu)
    lay_r = ref_mod.build_layout(shape, block, radius=1, pool_size=16, layout="raster_block")
    x = torch.randn(1, n, 512, generator=torch.Generator().manual_seed(12)).to(torch.bfloat16)
    dy = torch.randn(1, n, 512, generator=torch.Generator().manual_seed(13))
    xh = x.to(gpu).requires_grad_()
    xr = x.float().requires_grad_()
    yh = layer(xh, lay)
    yh.backward(dy.to(gpu, torch.bfloat16))
    yr = oracle(xr, lay_r, chunk=512)
    yr.backward(dy)
    checks = [("output", yh, yr), ("input", xh.grad, xr.grad)]
    expected = dict(oracle.named_parameters())
    checks += [(name, prm.grad, expected[name].grad) for name, prm in layer.named_parameters()]
    for name, got, exp in checks:
        assert got is not None and torch.isfinite(got.float()).all(), name
        err = rel_l2(got.float().cpu(), exp)
        print(f"  {name}: rel_l2={err:.3g}", flush=True)
        assert err < TOL[torch.bfloat16], (name, err)
