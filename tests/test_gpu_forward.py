"""Forward parity of the HIP path with the oracle (reference.py / attention.py restated).

Bars: fp32 max-abs <= 1e-5 on the core output and the reference's
assert_close(3e-5) (tests/test_triton.py:91-92); fp16/bf16 max-abs <= 2e-2 on
unit-scale activations and the reference's relative-L2 bars 5e-3 / 3.5e-2
(tests/test_triton.py:83).  Repacks must permute outputs bit-exactly.
"""
import math

import pytest
import torch

import oracle.pack3d_oracle as ref
import pack3d_amd as p3d
from pack3d_amd.rope import axial_rope as hip_axial, packed_rope
from tests._cases import make_case, max_abs, random_core_inputs, rel_l2

pytestmark = pytest.mark.gpu

REL = {torch.float32: 3e-5, torch.float16: 5e-3, torch.bfloat16: 3.5e-2}
ABS = {torch.float32: 1e-5, torch.float16: 2e-2, torch.bfloat16: 2e-2}


def _check(got, exp, dtype, what):
    r, m = rel_l2(got, exp), max_abs(got, exp)
    print(f"  {what}: rel_l2={r:.3g} max_abs={m:.3g}", flush=True)
    assert torch.isfinite(got).all(), what
    assert r < REL[dtype], (what, r)
    assert m <= ABS[dtype], (what, m)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape", [(37, 16, 2, 4, 2, 4, 3), (131, 64, 1, 8, 2, 16, 2), (19, 32, 1, 2, 2, 3, 1),
                                   (21, 128, 1, 2, 1, 4, 4), (67, 48, 1, 4, 4, 8, 1)])
def test_core_custom_graph(gpu, dtype, shape):
    print(f"core custom {shape} {dtype}", flush=True)
    inputs, nb, blocks, pool = make_case(*shape, dtype=dtype)
    og = ref.prepare_geometry(nb, blocks, pool)
    hg = p3d.prepare_geometry(nb.to(gpu), blocks.to(gpu), pool)
    got = p3d.pack3d_hip(*(t.to(gpu) for t in inputs), hg, temperature=0.7)
    exp = ref.pack3d_reference(*inputs, og, temperature=0.7)
    _check(got, exp, dtype, "y")
    if dtype == torch.float32:
        torch.testing.assert_close(got.cpu(), exp, atol=3e-5, rtol=3e-5)


GRIDS = [
    # shape, block, radius, kind, heads, kv_heads, d
    ((8, 8, 8), (4, 4, 4), 2, "raster_block", 4, 4, 48),
    ((8, 8, 8), (4, 4, 4), 2, "native_block_morton", 4, 2, 48),
    ((6, 10, 12), (2, 5, 3), (1, 2, 1), "native_block_morton", 2, 1, 32),
    ((5, 7, 9), (5, 7, 1), (0, 1, 2), "raster_block", 2, 2, 64),
    ((4, 16, 12), (2, 2, 2), 1, "raster_block", 4, 1, 16),
    ((12, 12, 12), (4, 4, 4), 2, "native_block_morton", 2, 2, 128),
    # head_dim 64 with radius <= 1 (10-wide halo planes in 16-bit types):
    # partial bricks on every axis, 4 query heads per kv head; an
    # anisotropic radius; radius 0.
    ((9, 12, 20), (1, 4, 4), 1, "raster_block", 8, 2, 64),
    ((6, 10, 20), (2, 2, 2), (1, 0, 1), "native_block_morton", 4, 2, 64),
    ((3, 8, 8), (1, 4, 4), 0, "raster_block", 2, 1, 64),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape,block,radius,kind,heads,kv_heads,d", GRIDS)
def test_core_grid(gpu, dtype, shape, block, radius, kind, heads, kv_heads, d):
    print(f"core grid {shape} {block} {radius} {kind} h{heads} g{kv_heads} d{d} {dtype}", flush=True)
    lay_h = p3d.build_layout(shape, block, radius=radius, pool_size=1, layout=kind)
    lay_r = ref.build_layout(shape, block, radius=radius, pool_size=1, layout=kind)
    n, vol = math.prod(shape), math.prod(block)
    inputs = random_core_inputs(2, heads, kv_heads, n, d, vol, dtype, seed=n + d)
    got = p3d.pack3d_hip(*(t.to(gpu) for t in inputs), lay_h.geometry, temperature=0.9)
    exp = ref.pack3d_reference(*inputs, lay_r.geometry, temperature=0.9)
    _check(got, exp, dtype, "y")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("kind", ["raster_block", "native_block_morton"])
def test_core_rope_fused(gpu, dtype, kind):
    print(f"core rope fused {kind} {dtype}", flush=True)
    shape, d = (8, 12, 16), 48
    lay_h = p3d.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout=kind)
    lay_r = ref.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout=kind)
    n = math.prod(shape)
    inputs = random_core_inputs(1, 4, 4, n, d, 64, dtype, seed=7)
    rope = hip_axial(d, shape, lay_h.coords)
    got = p3d.pack3d_hip_rope(*(t.to(gpu) for t in inputs), lay_h.geometry, rope)
    rot = [ref.axial_rope(t, lay_r.coords) if i in (0, 1, 3) else t for i, t in enumerate(inputs)]
    exp = ref.pack3d_reference(*rot, lay_r.geometry)
    _check(got, exp, dtype, "y")
    # The same rotation through the custom-graph path (indexed local + rows).
    plain = p3d.prepare_geometry(lay_h.geometry.neighbors, lay_h.geometry.blocks, 1)
    got2 = p3d.pack3d_hip_rope(*(t.to(gpu) for t in inputs), plain, rope)
    _check(got2, exp, dtype, "y (indexed path)")
    # Packed-position control.
    prope = packed_rope(d, n, gpu)
    got3 = p3d.pack3d_hip_rope(*(t.to(gpu) for t in inputs), lay_h.geometry, prope)
    seq = torch.arange(n)
    pc = torch.stack((seq, torch.zeros_like(seq), torch.zeros_like(seq)), -1)
    rot = [ref.axial_rope(t, pc, pairs=(d // 2, 0, 0)) if i in (0, 1, 3) else t for i, t in enumerate(inputs)]
    _check(got3, ref.pack3d_reference(*rot, lay_r.geometry), dtype, "y (packed rope)")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_layer_matches_oracle(gpu, dtype):
    """The whole layer (LayerNorm, projections, gate, core, to_out, residual)
    against the oracle layer in fp32 on the same (rounded) weights and input.
    fp32: assert_close 2e-5.  bf16: max-abs <= 2e-2 plus the output's own
    rounding (half an ulp of |y|, 2^-8 |y| in bf16)."""
    print(f"layer {dtype}", flush=True)
    torch.manual_seed(0)
    shape = (16, 16, 16) if dtype == torch.float32 else (8, 16, 16)
    oracle = ref.PACK3DAttention(192, heads=4, kv_heads=4, head_dim=48, block_volume=64)
    layer = p3d.PACK3DAttention(192, heads=4, kv_heads=4, head_dim=48, block_volume=64)
    layer.load_state_dict(oracle.state_dict())
    layer = layer.to(gpu, dtype)
    oracle = oracle.to(dtype).float()
    lay_h = p3d.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout="raster_block")
    lay_r = ref.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout="raster_block")
    x = torch.randn(1, math.prod(shape), 192, generator=torch.Generator().manual_seed(1)).to(dtype)
    with torch.no_grad():
        got = layer(x.to(gpu), lay_h).float().cpu()
        exp = oracle(x.float(), lay_r)
    if dtype == torch.float32:
        torch.testing.assert_close(got, exp, atol=2e-5, rtol=2e-5)
    else:
        excess = float(((got - exp).abs() - 2 ** -8 * exp.abs()).max())
        print(f"  max_abs={max_abs(got, exp):.3g} beyond rounding={excess:.3g}", flush=True)
        assert excess <= 2e-2


def test_repack_permutes_outputs_exactly(gpu):
    print("repack equivariance", flush=True)
    shape, d = (8, 12, 16), 48
    n = math.prod(shape)
    lay = p3d.build_layout(shape, (4, 4, 4), radius=2, pool_size=1)
    gen = torch.Generator().manual_seed(3)
    blocks_perm = torch.randperm(n // 64, generator=gen)
    slot_perm = torch.stack([torch.randperm(64, generator=gen) for _ in range(n // 64)])
    p = (blocks_perm[:, None] * 64 + slot_perm).reshape(-1)
    other = lay.repack(p)
    for dtype in (torch.float16, torch.bfloat16, torch.float32):
        inputs = [t.to(gpu) for t in random_core_inputs(1, 4, 4, n, d, 64, dtype, seed=11)]
        moved = [t[:, :, p.to(gpu)] if i in (0, 1, 2, 3, 4, 7) else t for i, t in enumerate(inputs)]
        rope_a = hip_axial(d, shape, lay.coords)
        rope_b = hip_axial(d, shape, other.coords)
        y = p3d.pack3d_hip_rope(*inputs, lay.geometry, rope_a)
        yp = p3d.pack3d_hip_rope(*moved, other.geometry, rope_b)
        assert torch.equal(yp, y[:, :, p.to(gpu)]), dtype


def _xavier_layer(shape, batch, dtype, gpu):
    """The benchmark layer of the BASELINE configs: Xavier projections from
    seed 0, mean pooling (w = b = 0), tokens ~ N(0, 1) from seed 1."""
    torch.manual_seed(0)
    layer = p3d.PACK3DAttention(192, heads=4, kv_heads=4, head_dim=48, block_volume=64)
    for lin in (layer.to_q, layer.to_kv, layer.to_out):
        torch.nn.init.xavier_uniform_(lin.weight)
    with torch.no_grad():
        layer.pool_weight.zero_()
        layer.slot_bias.zero_()
    x = torch.randn(batch, math.prod(shape), 192, generator=torch.Generator().manual_seed(1))
    return layer.to(gpu, dtype), x.to(gpu, dtype)


def _oracle_y32(q, kl, vl, kg, vg, weight, bias, gate, sl, sg, geometry, coords):
    """The oracle core on every row, rotating q, kl, kg like the reference,
    with y = sl o_L + gate sg o_G kept in fp32 (the oracle's own output is
    rounded to the storage type, which would add a second rounding)."""
    rot = [ref.axial_rope(t, coords) if i in (0, 1, 3) else t for i, t in enumerate((q, kl, vl, kg, vg))]
    _, ol, og = ref.pack3d_reference(*rot, weight, bias, gate, sl, sg, geometry, chunk=4096,
                                     return_branches=True)
    return sl.float() * ol + gate.float()[..., None] * sg.float() * og


def _core_vs_oracle(layer, x, lay, shape, kind, dtype, what):
    """Core output of the layer at full size against the oracle on every row:
    max-abs <= the dtype's bar and relative L2 below the reference's."""
    with torch.no_grad():
        core = layer.core_inputs(x, lay)
        q, kl, vl, kg, vg, gate, rope = core
        y = p3d.pack3d_hip_rope(q, kl, vl, kg, vg, layer.pool_weight, layer.slot_bias, gate,
                                layer.local_scale, layer.global_scale, lay.geometry, rope)
    lay_r = ref.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout=kind)
    params = [t.detach().cpu() for t in (layer.pool_weight, layer.slot_bias)]
    exp = _oracle_y32(*(t.cpu() for t in (q, kl, vl, kg, vg)), *params, gate.cpu(), layer.local_scale.detach().cpu(),
                      layer.global_scale.detach().cpu(), lay_r.geometry, lay_r.coords)
    _check(y, exp, dtype, what)
    return y, core


def test_full_size_headline(gpu):
    """c2: 64^3 bf16, batch 1, raster: every row against the oracle."""
    print("full size c2", flush=True)
    shape = (64, 64, 64)
    layer, x = _xavier_layer(shape, 1, torch.bfloat16, gpu)
    lay = p3d.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout="raster_block")
    _core_vs_oracle(layer, x, lay, shape, "raster_block", torch.bfloat16, "c2 y")


def test_full_size_c1(gpu):
    """c1: 16 x 64 x 64 bf16, batch 2, raster: every row against the oracle."""
    print("full size c1", flush=True)
    shape = (16, 64, 64)
    layer, x = _xavier_layer(shape, 2, torch.bfloat16, gpu)
    lay = p3d.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout="raster_block")
    _core_vs_oracle(layer, x, lay, shape, "raster_block", torch.bfloat16, "c1 y")


def test_full_size_c3_morton_repack(gpu):
    """c3: 64^3 fp16 in Morton order: every row against the oracle, then a
    seeded pure repack (block permutation + slot shuffle) must permute the
    core output bit for bit."""
    print("full size c3 morton + repack", flush=True)
    shape = (64, 64, 64)
    n = math.prod(shape)
    layer, x = _xavier_layer(shape, 1, torch.float16, gpu)
    lay = p3d.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout="native_block_morton")
    y, (q, kl, vl, kg, vg, gate, _) = _core_vs_oracle(layer, x, lay, shape, "native_block_morton",
                                                      torch.float16, "c3 y")
    gen = torch.Generator().manual_seed(3)
    fine = n // 64
    slots = torch.argsort(torch.rand(fine, 64, generator=gen), dim=1)
    p = (torch.randperm(fine, generator=gen)[:, None] * 64 + slots).reshape(-1)
    other = lay.repack(p)
    pg = p.to(gpu)
    moved = [t[:, :, pg] for t in (q, kl, vl, kg, vg)]
    with torch.no_grad():
        yp = p3d.pack3d_hip_rope(*moved, layer.pool_weight, layer.slot_bias, gate[:, :, pg], layer.local_scale,
                                 layer.global_scale, other.geometry, hip_axial(48, shape, other.coords))
    assert torch.equal(yp, y[:, :, pg])


@pytest.mark.parametrize("grid", [False, True])
def test_core_loose_bound_takes_exact_path(gpu, grid):
    """A summary key far larger than any score it produces (orthogonal to
    every query) makes the Cauchy-Schwarz reference point useless; the
    kernels must fall back to the exact online softmax and still match."""
    print(f"loose bound grid={grid}", flush=True)
    shape, d = (8, 8, 8), 48
    n = math.prod(shape)
    inputs = random_core_inputs(1, 2, 2, n, d, 64, torch.float32, seed=5)
    inputs[0][..., d // 2:] = 0                        # queries live in channels 0..23
    inputs[3][:, :, :64] = 0
    inputs[3][:, :, :64, d // 2:] = 40.0               # block 0: a huge key in channels 24..47
    inputs[5] = torch.zeros(d)                         # mean pooling
    inputs[6] = torch.zeros(64)
    lay_r = ref.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout="raster_block")
    exp = ref.pack3d_reference(*inputs, lay_r.geometry)
    if grid:
        geom = p3d.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout="raster_block").geometry
    else:
        geom = p3d.prepare_geometry(lay_r.geometry.neighbors, lay_r.geometry.blocks, 1)
    got = p3d.pack3d_hip(*(t.to(gpu) for t in inputs), geom)
    _check(got, exp, torch.float32, "y")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("dim", [192, 64, 272, 384, 512])
def test_layer_norm_kernel_matches_torch(gpu, dtype, dim):
    """The layer's LayerNorm kernel against torch's (attention.py:64), parameters
    in the storage type and in fp32."""
    from pack3d_amd.attention import layer_norm
    gen = torch.Generator().manual_seed(dim)
    x = (torch.randn(3, 1000, dim, generator=gen) * 2 + 0.5).to(gpu, dtype)
    for pdtype in (dtype, torch.float32):
        norm = torch.nn.LayerNorm(dim).to(gpu, pdtype)
        with torch.no_grad():
            norm.weight.copy_(torch.randn(dim, generator=gen))
            norm.bias.copy_(torch.randn(dim, generator=gen))
            got = layer_norm(norm, x)
            exp = torch.nn.functional.layer_norm(x.float(), (dim,), norm.weight.float(), norm.bias.float(),
                                                 norm.eps)
        tol = 1e-5 if dtype == torch.float32 else (2e-3 if dtype == torch.float16 else 1.6e-2)
        torch.testing.assert_close(got.float(), exp.to(dtype).float(), atol=tol * 4, rtol=tol)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dim,heads,kv_heads,d", [(192, 4, 4, 48), (64, 2, 1, 32), (128, 4, 2, 16), (256, 2, 2, 64),
                                                (96, 3, 1, 16), (512, 8, 2, 64)])
def test_fused_projections_match_torch(gpu, dtype, dim, heads, kv_heads, d):
    """p3d_project against the separate torch ops it replaces (LayerNorm, the
    three linear maps, the gate softmax), with random LayerNorm affine and
    gate bias; rows not a multiple of the 128-token tile.  With 3 heads of 16
    (q_out 48, kv_out 64) a 32-output block holds the end of q and the start
    of kv, and another the end of kv and the gate logits."""
    from pack3d_amd.attention import fused_projections
    print(f"fused projections {dim} h{heads} g{kv_heads} d{d} {dtype}", flush=True)
    torch.manual_seed(dim + d)
    layer = p3d.PACK3DAttention(dim, heads=heads, kv_heads=kv_heads, head_dim=d, block_volume=64)
    with torch.no_grad():
        layer.norm.weight.uniform_(0.5, 1.5)
        layer.norm.bias.normal_(0.0, 0.1)
        layer.gate.bias.normal_(0.0, 0.5)
    layer = layer.to(gpu, dtype)
    n = 1000
    x = (torch.randn(2, n, dim) * 2.0 + 0.3).to(gpu, dtype)
    with torch.no_grad():
        got = fused_projections(layer, x)
        assert got is not None
        xn = layer.norm(x)
        exp = (layer.to_q(xn), layer.to_kv(xn), layer.gate(xn).view(2, n, heads, 2).softmax(-1)[..., 1])
    tol = {torch.bfloat16: 2 ** -6, torch.float16: 2 ** -9}[dtype]
    for name, g_, e_ in zip(("q", "kv", "gate"), got, exp):
        assert g_.shape == e_.shape, name
        g32, e32 = g_.float(), e_.float()
        # one rounding step of the output, relative to its magnitude (the
        # contraction order differs from hipBLASLt's)
        bound = tol * (e32.abs() + 1.0)
        assert ((g32 - e32).abs() <= bound).all(), (name, float((g32 - e32).abs().max()))
        assert float((g32 - e32).abs().mean()) < tol * 0.1, name


@pytest.mark.gpu
def test_fused_projections_not_used_with_grad(gpu):
    from pack3d_amd.attention import fused_projections
    layer = p3d.PACK3DAttention(192, heads=4, kv_heads=4, head_dim=48, block_volume=64).to(gpu, torch.bfloat16)
    x = torch.randn(1, 64, 192, device=gpu, dtype=torch.bfloat16)
    assert fused_projections(layer, x) is None  # parameters require grad and autograd is on
    with torch.no_grad():
        assert fused_projections(layer, x) is not None
        assert fused_projections(layer.float(), x.float()) is None


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dim,heads,d", [(192, 4, 48), (64, 2, 32), (256, 4, 16)])
def test_fused_out_residual_matches_addmm(gpu, dtype, dim, heads, d):
    """p3d_out_residual against torch.addmm(x, y, Wo^T) (one rounding of the
    fp32 sum); rows not a multiple of the 256-token tile."""
    from pack3d_amd.attention import fused_out_residual
    print(f"fused out residual {dim} h{heads} d{d} {dtype}", flush=True)
    torch.manual_seed(dim + heads)
    layer = p3d.PACK3DAttention(dim, heads=heads, kv_heads=1, head_dim=d, block_volume=64).to(gpu, dtype)
    n = 777
    x = torch.randn(n, dim, device=gpu).to(dtype)
    y = torch.randn(n, heads * d, device=gpu).to(dtype)
    with torch.no_grad():
        got = fused_out_residual(layer, x, y)
        exp = torch.addmm(x, y, layer.to_out.weight.t())
    assert got is not None and got.shape == exp.shape
    tol = {torch.bfloat16: 2 ** -7, torch.float16: 2 ** -10}[dtype]
    g32, e32 = got.float(), exp.float()
    assert ((g32 - e32).abs() <= tol * (e32.abs() + 1.0)).all(), float((g32 - e32).abs().max())


def test_pool_norm_slots_first_and_repeated_call(gpu):
    """The plan's first pooling launch takes the zero-allocated norm slots
    as they are (no clear launch); a repeated launch clears them itself, so
    slots overwritten in between come out the same.  Both equal the maxima of
    the stored summary-key norms, summary m reducing into slot m % 64."""
    from pack3d_amd.core import ForwardPlan

    print("pool norm slots", flush=True)
    torch.manual_seed(0)
    shape = (8, 16, 12)
    n = math.prod(shape)
    layer = p3d.PACK3DAttention(192, heads=4, kv_heads=4, head_dim=48, block_volume=64).to(gpu)
    lay = p3d.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout="raster_block", device=gpu)
    x = torch.randn(1, n, 192, generator=torch.Generator().manual_seed(1)).to(gpu, torch.bfloat16)
    layer = layer.to(torch.bfloat16)
    with torch.inference_mode():
        q, kl, vl, kg, vg, gate, rope = layer.core_inputs(x, lay)
        plan = ForwardPlan(q, kl, vl, kg, vg, layer.pool_weight, layer.slot_bias, gate, layer.local_scale,
                           layer.global_scale, lay.geometry, layer.temperature, rope, rope)
        assert plan.pool_args.norms_cleared == 1
        plan.pool()
        assert plan.pool_args.norms_cleared == 0
        first = plan.sk_norm_max.clone()
        plan.sk_norm_max.fill_(1e30)
        plan.pool()
        torch.cuda.synchronize()
    assert torch.equal(plan.sk_norm_max, first)
    m = lay.geometry.num_summaries
    norms = plan.sk[:, :, :m].float().pow(2).sum(-1).sqrt() * (1 + 1e-6)  # [B, G, M]
    exp = torch.zeros(norms.shape[0], norms.shape[1], 64, device=gpu)
    exp.scatter_reduce_(2, (torch.arange(m, device=gpu) % 64).expand_as(norms), norms, reduce="amax")
    assert torch.allclose(first.view_as(exp), exp, rtol=1e-5, atol=0), (first.view_as(exp) - exp).abs().max()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_pool_32_over_64_slots(gpu, dtype):
    """Summary pool 32 over 64-slot fine blocks at head_dim 64: the reference
    rejects pool_tile * slot_tile * head_dim > 32768 (_validation.py:21-24), a
    register budget of its Triton pooling kernel; this pooling walks the fine
    blocks one at a time and takes it.  Forward and every gradient against the
    oracle, with random pooling weights and a padded last coarse group."""
    print(f"pool 32 x 64 slots {dtype}", flush=True)
    shape, d = (8, 16, 40), 64
    n = math.prod(shape)
    lay_h = p3d.build_layout(shape, (4, 4, 4), radius=1, pool_size=32, layout="native_block_morton")
    lay_r = ref.build_layout(shape, (4, 4, 4), radius=1, pool_size=32, layout="native_block_morton")
    assert lay_h.geometry.blocks.shape == (n // 64, 64) and (n // 64) % 32 != 0
    inputs = random_core_inputs(1, 4, 2, n, d, 64, dtype, seed=32)
    xs = [t.to(gpu).requires_grad_() for t in inputs]
    rs = [t.detach().clone().requires_grad_() for t in inputs]
    y = p3d.pack3d_hip(*xs, lay_h.geometry, temperature=0.6)
    e = ref.pack3d_reference(*rs, lay_r.geometry, temperature=0.6)
    _check(y, e, dtype, "y")
    up = torch.randn(e.shape, generator=torch.Generator().manual_seed(6)).to(dtype)
    got = torch.autograd.grad(y, xs, up.to(gpu))
    exp = torch.autograd.grad(e, rs, up)
    for a, b in zip(got, exp):
        assert rel_l2(a.float(), b.float()) < REL[dtype]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_indexed_local_rotates_and_rounds_q_like_a_prerotated_copy(gpu, dtype):
    """The indexed local kernel rotates q on load and rounds the result to the
    storage type, as rope.py:48 returns it and as the backward (which
    recomputes P on a rounded rotated copy against the saved log-sum-exp)
    sees it: o_L, its log-sum-exp and y are bit-identical to a run on q
    rotated beforehand by p3d_rotate with the identity rotation."""
    from pack3d_amd.core import ForwardPlan, _rotated, brick_tag
    from pack3d_amd.rope import identity_rope

    print(f"indexed local rotate-on-load vs pre-rotated q {dtype}", flush=True)
    shape = (8, 8, 16)
    lay_o = ref.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout="raster_block")
    hg = p3d.prepare_geometry(lay_o.geometry.neighbors.to(gpu), lay_o.geometry.blocks.to(gpu), 1)
    assert brick_tag(hg) is None  # untagged: the indexed local kernel runs
    n = math.prod(shape)
    q, kl, vl, kg, vg, w, b, gate, sl, sg = (t.to(gpu) for t in
                                             random_core_inputs(1, 4, 2, n, 48, 64, dtype, seed=77, scale=2.0))
    coords = lay_o.coords.to(gpu)
    rope = hip_axial(48, shape, coords)
    with torch.no_grad():
        y1, s1 = ForwardPlan(q, kl, vl, kg, vg, w, b, gate, sl, sg, hg, 1.0, rope, rope, save_state=True).run()
        ident = identity_rope(48, gpu)
        y2, s2 = ForwardPlan(_rotated(q, rope), _rotated(kl, rope), vl, kg, vg, w, b, gate, sl, sg, hg, 1.0,
                             ident, rope, save_state=True).run()
        torch.cuda.synchronize()
    assert torch.equal(s1["o_local"], s2["o_local"])
    assert torch.equal(s1["lse_local"], s2["lse_local"])
    assert torch.equal(y1, y2)


def test_full_size_c2_bench_layer_matches_oracle(gpu):
    """The exact layer step bench.py times (c2: 64^3 bf16, batch 1, raster,
    no grad; Xavier projections, mean pooling), asserted to take the fused
    projection pooling (p3d_project_pool: kl stored rotated, kg / vg never
    written), against the oracle layer on the same (rounded) weights and input
    on every row: max-abs <= 2e-2 beyond the output's own rounding to bf16,
    and the attention's share of y (y - x) within the reference's bf16
    relative-L2 bar."""
    import bench
    from pack3d_amd import _lib
    from pack3d_amd.attention import PACK3DAttention

    print("full size c2 bench layer vs oracle", flush=True)
    shape = bench.SHAPE
    n = math.prod(shape)
    layer = bench.build_layer(gpu, torch.bfloat16)
    assert isinstance(layer, PACK3DAttention)
    lay = p3d.build_layout(shape, bench.BLOCK, radius=bench.RADIUS, pool_size=1, layout="raster_block", device=gpu)
    x = torch.randn(1, n, bench.DIM, generator=torch.Generator().manual_seed(1)).to(gpu, torch.bfloat16)
    calls = []
    real = _lib.lib
    _lib.lib = lambda: bench._TimedLib(real(), ("p3d_project_pool", "p3d_attn_fwd_grid"), calls.append)
    try:
        with torch.inference_mode():
            y = layer(x, lay)
        torch.cuda.synchronize()
    finally:
        _lib.lib = real
    assert "p3d_project_pool" in calls and "p3d_attn_fwd_grid" in calls, calls
    oracle = bench.oracle_layer(layer)
    lay_r = ref.build_layout(shape, bench.BLOCK, radius=bench.RADIUS, pool_size=1, layout="raster_block")
    xf = x.float().cpu()
    with torch.inference_mode():
        exp = oracle(xf, lay_r, chunk=512)
    got = y.float().cpu()
    diff = (got - exp).abs()
    beyond = float((diff - 2 ** -8 * exp.abs()).max())
    rel = rel_l2(got - xf, exp - xf)
    print(f"  max_abs={float(diff.max()):.3g} beyond rounding={beyond:.3g} rel_l2(y - x)={rel:.3g}", flush=True)
    assert torch.isfinite(got).all()
    assert beyond <= 2e-2
    assert rel < REL[torch.bfloat16]
    gate = bench.correctness_gate(layer, x, y, shape, exp)
    assert gate["max_abs_beyond_output_rounding"] == round(beyond, 6)


def test_full_size_allen15_layer_matches_oracle(gpu):
    """The reference benchmark's allen15 preset at the size of its published
    table's first row (benchmarks/attention.py:84-91, results table row 1:
    dim 512, 8 / 2 heads, head_dim 64, (1, 4, 4) blocks, pool 16, radius 1,
    32 x 128 x 64 = 262,144 tokens, bf16, no grad): the layer's forward,
    which takes the head_dim-64 attention kernel on 10-wide halo planes and
    the packed pooling steps, against the oracle layer on the same (rounded)
    weights and input on every row: max-abs <= 2e-2 beyond the output's own
    rounding to bf16, and the attention's share of y (y - x) within the
    reference's bf16 relative-L2 bar."""
    print("full size allen15 layer vs oracle", flush=True)
    shape, block = (32, 128, 64), (1, 4, 4)
    n = math.prod(shape)
    torch.manual_seed(205)
    layer = p3d.PACK3DAttention(512, heads=8, kv_heads=2, head_dim=64, block_volume=16).to(gpu, torch.bfloat16)
    lay = p3d.build_layout(shape, block, radius=1, pool_size=16, layout="raster_block", device=gpu)
    x = torch.randn(1, n, 512, generator=torch.Generator().manual_seed(11)).to(gpu, torch.bfloat16)
    with torch.inference_mode():
        y = layer(x, lay)
    torch.cuda.synchronize()
    oracle = ref.PACK3DAttention(512, heads=8, kv_heads=2, head_dim=64, block_volume=16)
    oracle.load_state_dict({k: v.detach().float().cpu() for k, v in layer.state_dict().items()})
    lay_r = ref.build_layout(shape, block, radius=1, pool_size=16, layout="raster_block")
    xf = x.float().cpu()
    with torch.inference_mode():
        exp = oracle(xf, lay_r, chunk=512)
    got = y.float().cpu()
    diff = (got - exp).abs()
    beyond = float((diff - 2 ** -8 * exp.abs()).max())
    rel = rel_l2(got - xf, exp - xf)
    print(f"  max_abs={float(diff.max()):.3g} beyond rounding={beyond:.3g} rel_l2(y - x)={rel:.3g}", flush=True)
    assert torch.isfinite(got).all()
    assert beyond <= 2e-2
    assert rel < REL[torch.bfloat16]
