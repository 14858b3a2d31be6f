"""The HIP backend driven with objects shaped like the reference's own
(``Pack3DGeometry`` / ``TokenLayout`` of src/pack3d/geometry.py:10-50,129-220
of amilworks/Pack3D: ``_radius_one_grid`` and ``_raster_to_packed``, no
``_grid``), and through the registration block of INTEGRATION.md.

Which kernels run is asserted through ``core.brick_tag``: a geometry tagged
by the reference (radius one) or proven by ``adopt_layout`` takes the brick
kernels, any other the indexed ones.  Both must match the oracle.
"""
import math

import pytest
import torch

import oracle.pack3d_oracle as ref
import pack3d_amd as p3d
from pack3d_amd.core import brick_tag
from pack3d_amd.rope import axial_rope as hip_axial
from tests._cases import max_abs, random_core_inputs, rel_l2
from tests._refobjects import ReferenceLayerWithHip, reference_layout

pytestmark = pytest.mark.gpu

REL = {torch.float32: 3e-5, torch.float16: 5e-3, torch.bfloat16: 3.5e-2}
ABS = {torch.float32: 1e-5, torch.float16: 2e-2, torch.bfloat16: 2e-2}


def _check(got, exp, dtype, what):
    r, m = rel_l2(got, exp), max_abs(got, exp)
    print(f"  {what}: rel_l2={r:.3g} max_abs={m:.3g}", flush=True)
    assert torch.isfinite(got).all(), what
    assert r < REL[dtype], (what, r)
    assert m <= ABS[dtype], (what, m)


def _core(gpu, lay_o, lay_ref, d, dtype, heads=4, kv_heads=2, seed=5):
    n = lay_o.geometry.num_tokens
    inputs = random_core_inputs(1, heads, kv_heads, n, d, lay_o.geometry.blocks.shape[1], dtype, seed=seed)
    rope = hip_axial(d, lay_ref.grid_shape, lay_ref.coords)
    got = p3d.pack3d_hip_rope(*(t.to(gpu) for t in inputs), lay_ref.geometry, rope, temperature=0.8)
    rot = [ref.axial_rope(t, lay_o.coords) if i in (0, 1, 3) else t for i, t in enumerate(inputs)]
    exp = ref.pack3d_reference(*rot, lay_o.geometry, temperature=0.8)
    return got, exp


@pytest.mark.parametrize("kind", ["raster_block", "native_block_morton"])
def test_reference_radius_one_tag_takes_brick_kernel(gpu, kind):
    print(f"reference radius-one tag {kind}", flush=True)
    lay_o = ref.build_layout((4, 16, 64), (2, 2, 2), radius=1, pool_size=2, layout=kind)
    lay = reference_layout(lay_o, gpu)
    assert not hasattr(lay.geometry, "_grid") and lay.geometry._radius_one_grid == (4, 16, 64)
    tag = brick_tag(lay.geometry)
    assert tag is not None and tag[0] == (4, 16, 64) and tag[1] == (1, 1, 1)
    assert (tag[2] is None) == (kind == "raster_block")
    for dtype in (torch.float32, torch.bfloat16):
        got, exp = _core(gpu, lay_o, lay, 32, dtype)
        _check(got, exp, dtype, f"y {dtype}")


@pytest.mark.parametrize("kind", ["raster_block", "native_block_morton"])
def test_reference_radius_two_untagged_then_adopted(gpu, kind):
    print(f"reference radius-two layout {kind}", flush=True)
    lay_o = ref.build_layout((8, 8, 16), (4, 4, 4), radius=2, pool_size=1, layout=kind)
    lay = reference_layout(lay_o, gpu)
    assert lay.geometry._radius_one_grid is None and brick_tag(lay.geometry) is None
    for dtype in (torch.float32, torch.bfloat16):
        got_indexed, exp = _core(gpu, lay_o, lay, 48, dtype)
        _check(got_indexed, exp, dtype, f"indexed {dtype}")
    p3d.adopt_layout(lay)
    tag = brick_tag(lay.geometry)
    assert tag is not None and tag[0] == (8, 8, 16) and tag[1] == (2, 2, 2)
    if kind == "raster_block":
        assert tag[2] is None
    else:
        inv = lay_o.order.argsort().to(torch.int32)
        assert torch.equal(tag[2].cpu(), inv)
    for dtype in (torch.float32, torch.bfloat16):
        got, exp = _core(gpu, lay_o, lay, 48, dtype)
        _check(got, exp, dtype, f"brick {dtype}")


def test_adopt_proves_repacked_layout_and_rejects_other_tables(gpu):
    print("adopt repacked and non-stencil tables", flush=True)
    shape = (8, 8, 8)
    lay_o = ref.build_layout(shape, (4, 4, 4), radius=(1, 2, 1), pool_size=1, layout="native_block_morton")
    gen = torch.Generator().manual_seed(11)
    n = math.prod(shape)
    p = (torch.randperm(n // 64, generator=gen)[:, None] * 64
         + torch.stack([torch.randperm(64, generator=gen) for _ in range(n // 64)])).reshape(-1)
    rep_o = lay_o.repack(p)
    lay = reference_layout(rep_o, gpu)
    p3d.adopt_layout(lay)
    tag = brick_tag(lay.geometry)
    assert tag is not None and tag[1] == (1, 2, 1)
    assert torch.equal(tag[2].cpu(), rep_o.order.argsort().to(torch.int32))
    got, exp = _core(gpu, rep_o, lay, 32, torch.float32, kv_heads=1)
    _check(got, exp, torch.float32, "repacked brick")
    # The self edge of one row dropped (the centre column is never -1): a
    # valid graph, but not the complete stencil.
    nb = lay_o.geometry.neighbors.clone()
    assert nb[100, nb.shape[1] // 2] == 100
    nb[100, nb.shape[1] // 2] = -1
    broken = ref.prepare_geometry(nb, lay_o.geometry.blocks, 1)
    lay_b = reference_layout(ref.TokenLayout(shape, lay_o.order, lay_o.coords, broken), gpu)
    p3d.adopt_layout(lay_b)
    assert brick_tag(lay_b.geometry) is None
    # Radii (1, 1, 2), (1, 2, 1) and (2, 1, 1) share the width 45: only the
    # stencil the table holds is proven.
    lay_c = reference_layout(ref.build_layout(shape, (4, 4, 4), radius=(2, 1, 1), pool_size=1), gpu)
    p3d.adopt_layout(lay_c)
    assert brick_tag(lay_c.geometry)[1] == (2, 1, 1)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("dim,heads,kv_heads,d", [(96, 4, 2, 32), (192, 4, 4, 48)])
def test_integration_registration_block(gpu, dtype, dim, heads, kv_heads, d):
    """The reference layer with the hip branch as INTEGRATION.md writes it
    (constructor guards included), on a reference-shaped radius-two layout,
    against the oracle layer: outputs and every gradient.  At the BASELINE
    widths (dim 192, 4 / 4 heads, head_dim 48) the unpatched line 29 of the
    reference's constructor refuses the layer; the patched one builds it."""
    print(f"integration block dim{dim} h{heads} g{kv_heads} d{d} {dtype}", flush=True)
    if d == 48:
        with pytest.raises(ValueError, match="unsupported grouped-head"):
            ReferenceLayerWithHip(dim, heads=heads, kv_heads=kv_heads, head_dim=d, block_volume=64, patched=False)
    torch.manual_seed(0)
    shape = (8, 8, 16)
    lay_o = ref.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout="native_block_morton")
    lay = reference_layout(lay_o, gpu)
    oracle = ref.PACK3DAttention(dim, heads=heads, kv_heads=kv_heads, head_dim=d, block_volume=64)
    layer = ReferenceLayerWithHip(dim, heads=heads, kv_heads=kv_heads, head_dim=d, block_volume=64)
    layer.load_state_dict(oracle.state_dict())
    layer = layer.to(gpu)
    x = torch.randn(1, math.prod(shape), dim, generator=torch.Generator().manual_seed(1))
    dy = torch.randn(1, math.prod(shape), dim, generator=torch.Generator().manual_seed(2))
    xg = x.to(gpu).requires_grad_()
    xo = x.clone().requires_grad_()
    if dtype == torch.float32:
        got = layer(xg, lay)
    else:
        with torch.autocast("cuda", dtype=dtype):
            got = layer(xg, lay)
    exp = oracle(xo, lay_o)
    assert brick_tag(lay.geometry) is not None
    tol = 2e-5 if dtype == torch.float32 else 2e-2
    m = max_abs(got.float(), exp)
    print(f"  y max_abs={m:.3g}", flush=True)
    assert m <= tol
    got.backward(dy.to(gpu).to(got.dtype))
    exp.backward(dy)
    pairs = [("x", xg.grad, xo.grad)] + [(k, a.grad, b.grad) for (k, a), b in
                                         zip(layer.named_parameters(), oracle.parameters())]
    for name, a, b in pairs:
        r = rel_l2(a.float(), b)
        print(f"  d{name}: rel_l2={r:.3g}", flush=True)
        assert r < (1e-4 if dtype == torch.float32 else 5e-2), name


def test_stencil_match_counts_a_duplicated_order_entry(gpu):
    """An order that repeats a raster index is no permutation: some raster
    index is left without a row.  p3d_stencil_match counts it, so no tag is
    recorded even for a neighbour table built to agree with the resulting map
    (whichever of the two rows wins the scatter), and the brick kernels, which
    use the map unchecked, never see it."""
    import types

    from pack3d_amd import _lib
    from pack3d_amd.geometry import grid_tag

    print("stencil match with a duplicated order entry", flush=True)
    shape = (8, 8, 16)
    n = math.prod(shape)
    lay_o = ref.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout="raster_block")
    nb0 = lay_o.geometry.neighbors.long()  # raster order: packed index = raster index
    order = torch.arange(n, dtype=torch.int64)
    order[5] = 6  # rows 5 and 6 both claim raster index 6; raster index 5 has no row
    for winner in (5, 6):
        mapping = torch.arange(n, dtype=torch.int64)
        mapping[5] = -1
        mapping[6] = winner
        nb = torch.where(nb0[order] >= 0, mapping[nb0[order].clamp_min(0)], -1).to(torch.int32)
        nb_g, order_g = nb.to(gpu).contiguous(), order.to(gpu)
        out = torch.empty(n, dtype=torch.int32, device=gpu)
        flags = torch.empty(8, dtype=torch.int32, device=gpu)
        _lib.call("p3d_stencil_match", _lib.i64x3(shape), _lib.i64x3((2, 2, 2)), order_g.data_ptr(),
                  nb_g.data_ptr(), nb.shape[1], out.data_ptr(), flags.data_ptr(), _lib.stream_of(gpu))
        torch.cuda.synchronize()
        assert int(flags[0]) >= 1, (winner, flags.tolist())
        geom = types.SimpleNamespace(neighbors=nb_g, blocks=lay_o.geometry.blocks.to(gpu), tensors=(nb_g,),
                                     _radius_one_grid=None)
        lay = types.SimpleNamespace(grid_shape=shape, order=order_g, geometry=geom)
        p3d.adopt_layout(lay)
        assert grid_tag(geom) is None
