"""The projections with the summary pooling fused in (``p3d_project_pool``)
against the kernels they replace on the same inputs: ``p3d_project`` and then
``p3d_pool_fwd``; and the layer's no-grad forward through the fusion against
the same layer with the fusion switched off.

q, kl, vl and the gate come from the same GEMM code as ``p3d_project``:
bit-exact, with kl (stored rotated, as the layer asks) bit-exact against
``p3d_rotate`` of ``p3d_project``'s kl.  The attention kernels give the same
bits on pre-rotated keys (``kl_rotated``) as on keys they rotate themselves.  The summaries differ from ``p3d_pool_fwd``'s only in the order of
the fp32 sums (two 32-token halves of a fine block added at the end, instead
of one 64-slot sweep; the logits' dot products in two halves).  Both kernels'
summaries are pinned against the oracle's pooling (compression.py restated,
``compress_summaries``) evaluated in fp64 on the same rotated, rounded keys
(rotated by the library's rotation kernel, the table both kernels read):
each stored value within one unit in the last place of the storage type of
the fp64 value (plus 2^-16 of the largest summary, the fp32 sums' own
error), and the key-norm slots within one relative rounding step.
"""
import math

import pytest
import torch

import pack3d_amd as p3d
import pack3d_amd.attention as attention
from pack3d_amd import _lib
from pack3d_amd.core import ForwardPlan, _projection_views

pytestmark = pytest.mark.gpu

STEP = {torch.bfloat16: 2 ** -7, torch.float16: 2 ** -10}


def _layer(dim, heads, kv_heads, d, dtype, gpu, encoding="axial", temperature=0.7):
    torch.manual_seed(dim + 7 * heads + d)
    layer = p3d.PACK3DAttention(dim, heads=heads, kv_heads=kv_heads, head_dim=d, block_volume=64,
                                position_encoding=encoding, temperature=temperature)
    with torch.no_grad():
        layer.norm.weight.uniform_(0.5, 1.5)
        layer.norm.bias.normal_(0.0, 0.1)
        layer.gate.bias.normal_(0.0, 0.5)
        layer.pool_weight.normal_(0.0, 0.5)   # sharp enough slot softmax to matter
        layer.slot_bias.normal_(0.0, 0.5)
    return layer.to(gpu, dtype)


def _plan(layer, made, layout, rope):
    args, qp, kvp, gp = made
    views = _projection_views(qp, kvp, layer.heads, layer.kv_heads)
    return ForwardPlan(*views, layer.pool_weight, layer.slot_bias, gp.transpose(1, 2), layer.local_scale,
                       layer.global_scale, layout.geometry, layer.temperature, rope, rope)


def _summaries(plan, m):
    """sk [B, G, M, d] and the values [B, G, M, d] out of the transposed svt."""
    b, g, mp, d = plan.sk.shape
    sv = plan.svt.permute(0, 1, 2, 4, 3).reshape(b, g, mp, d)
    return plan.sk[:, :, :m].float(), sv[:, :, :m].float()


def _close(got, exp, dtype, what):
    err = (got - exp).abs()
    bound = STEP[dtype] * exp.abs() + 1e-6
    print(f"  {what}: max_abs={float(err.max()):.3g} worst/bound={float((err / bound).max()):.3g}", flush=True)
    assert torch.isfinite(got).all(), what
    assert (err <= bound).all(), what


def _ulps(got, ref64, dtype):
    """|got - ref| in units of the storage type's spacing at ref, with an
    absolute floor of 2^-16 of the largest |ref| (the fp32 sums' error)."""
    eps = torch.finfo(dtype).eps
    _, e = torch.frexp(ref64)
    ulp = eps * torch.ldexp(torch.ones_like(ref64), e - 1)
    ulp = torch.maximum(ulp, torch.full_like(ulp, torch.finfo(dtype).tiny * eps))
    return (got.double() - ref64).abs() / (ulp + 2 ** -16 * float(ref64.abs().max()))


def _oracle_summaries(layer, sep, plan, rope, m):
    """sk (scaled by key_scale) and the values [B, G, M, d] in fp64 from the
    oracle's pooling on the separate path's kg, vg, with kg rotated by the
    library's rotation kernel (the table the fused kernels read; the rotation
    itself is pinned against the oracle's by the rope tests), so that only
    the pooling arithmetic is compared."""
    import oracle.pack3d_oracle as ref
    _, qp, kvp, _ = sep
    _, _, _, kg, vg = _projection_views(qp, kvp, layer.heads, layer.kv_heads)
    b, g, n, d = kg.shape
    kr = torch.empty(kg.shape, dtype=kg.dtype, device=kg.device)
    _lib.call("p3d_rotate", _lib.view(kg), _lib.view(kr), b, g, n, d, _lib.DTYPES[kg.dtype], rope.struct(), 0,
              _lib.stream_of(kg.device))
    geo = plan.geometry_cpu
    w, bias = (t.detach().cpu().double() for t in (layer.pool_weight, layer.slot_bias))
    sk, sv = ref.compress_summaries(kr.cpu().double(), vg.cpu().double(), w, bias, geo,
                                    temperature=layer.temperature)
    return sk[:, :, :m] * plan.key_scale, sv[:, :, :m]


def _rotated(t, rope):
    """p3d_rotate of a [B, G, N, d] view into a new contiguous tensor."""
    b, g, n, d = t.shape
    out = torch.empty(t.shape, dtype=t.dtype, device=t.device)
    _lib.call("p3d_rotate", _lib.view(t), _lib.view(out), b, g, n, d, _lib.DTYPES[t.dtype], rope.struct(), 0,
              _lib.stream_of(t.device))
    return out


def _compare(layer, x, layout, dtype, oracle=True, rotate_kl=1):
    dev = x.device
    stream = _lib.stream_of(dev)
    rope = layer._rope(x, layout)
    with torch.no_grad():
        fused = attention._project_buffers(layer, x)
        plan_f = _plan(layer, fused, layout, rope)
        rc = _lib.lib().p3d_project_pool(fused[0], plan_f.pool_args, rotate_kl, stream)
        assert rc == 0, _lib.lib().p3d_last_error().decode()
        sep = attention._project_buffers(layer, x)
        _lib.call("p3d_project", sep[0], stream)
        plan_s = _plan(layer, sep, layout, rope)
        plan_s.pool()
        h, g = layer.heads, layer.kv_heads
        kl_f = _projection_views(fused[1], fused[2], h, g)[1]
        kl_s = _projection_views(sep[1], sep[2], h, g)[1]
        kl_exp = _rotated(kl_s, rope) if rotate_kl else kl_s
    torch.cuda.synchronize()
    gd = layer.kv_heads * layer.head_dim
    for what, got, exp in (("q", fused[1], sep[1]), ("kl", kl_f.contiguous(), kl_exp.contiguous()),
                           ("vl", fused[2][..., gd:2 * gd], sep[2][..., gd:2 * gd]), ("gate", fused[3], sep[3])):
        diff = (got.float() - exp.float()).abs()
        assert torch.equal(got, exp), (what, int((diff > 0).sum()), float(diff.max()))
    m = layout.geometry.num_summaries
    (kf, vf), (ks, vs) = _summaries(plan_f, m), _summaries(plan_s, m)
    if oracle:
        plan_s.geometry_cpu = layout.geometry.to("cpu")
        k64, v64 = _oracle_summaries(layer, sep, plan_s, rope, m)
        for what, got, r in (("fused keys", kf, k64), ("fused values", vf, v64), ("pool_fwd keys", ks, k64),
                             ("pool_fwd values", vs, v64)):
            u = _ulps(got.cpu(), r, dtype)
            print(f"  {what}: max ulps vs fp64 oracle {float(u.max()):.3g}, "
                  f"{int((u > 0.5).sum())} of {u.numel()} beyond half an ulp", flush=True)
            assert torch.isfinite(got).all() and float(u.max()) <= 1.0, what
    _close(plan_f.sk_norm_max, plan_s.sk_norm_max, dtype, "key-norm slots")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dim,heads,kv_heads,d,shape,batch", [
    (192, 4, 4, 48, (8, 16, 16), 1),      # the headline layer's widths
    (64, 2, 1, 32, (4, 8, 8), 2),         # batch offsets of rows, positions and summaries
    (128, 8, 2, 64, (8, 8, 16), 1),       # grouped heads, d = 64 (the paper adapter's)
    (96, 3, 3, 16, (4, 4, 8), 1),         # kv channels 48: a 16-row last kg / vg block
    (256, 4, 2, 48, (8, 8, 8), 1),        # widest model
])
def test_project_pool_matches_project_then_pool(gpu, dtype, dim, heads, kv_heads, d, shape, batch):
    print(f"project+pool {dim} h{heads} g{kv_heads} d{d} {shape} b{batch} {dtype}", flush=True)
    layer = _layer(dim, heads, kv_heads, d, dtype, gpu)
    layout = p3d.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout="raster_block", device=gpu)
    x = (torch.randn(batch, math.prod(shape), dim, generator=torch.Generator().manual_seed(3)) * 1.5).to(gpu, dtype)
    _compare(layer, x, layout, dtype)


def test_project_pool_packed_rope_and_morton(gpu):
    """The packed rotation (positions along the token order) and a Morton
    layout, whose blocks are also consecutive 64-token runs."""
    print("project+pool packed rope, morton", flush=True)
    dtype = torch.bfloat16
    layer = _layer(192, 4, 4, 48, dtype, gpu, encoding="packed")
    layout = p3d.build_layout((8, 16, 16), (4, 4, 4), radius=2, pool_size=1, layout="native_block_morton",
                              device=gpu)
    x = torch.randn(1, 2048, 192, generator=torch.Generator().manual_seed(4)).to(gpu, dtype)
    _compare(layer, x, layout, dtype)


def test_project_pool_unrotated_kl(gpu):
    """rotate_kl = 0: kl as p3d_project stores it."""
    print("project+pool kl unrotated", flush=True)
    dtype = torch.bfloat16
    layer = _layer(128, 8, 2, 64, dtype, gpu)
    layout = p3d.build_layout((8, 8, 16), (4, 4, 4), radius=2, pool_size=1, layout="raster_block", device=gpu)
    x = torch.randn(1, 1024, 128, generator=torch.Generator().manual_seed(8)).to(gpu, dtype)
    _compare(layer, x, layout, dtype, oracle=False, rotate_kl=0)


@pytest.mark.parametrize("dtype,d,grid", [(torch.bfloat16, 48, True), (torch.bfloat16, 32, True),
                                          (torch.float16, 48, True), (torch.bfloat16, 64, True),
                                          (torch.bfloat16, 48, False)])
def test_attention_on_prerotated_keys(gpu, dtype, d, grid):
    """The core on kl it rotates itself and on kl already rotated (kl_rotated):
    the same bits, on the brick kernel (the plane-DMA path of bf16 d <= 48 and
    the register-staged path of the others) and on an arbitrary graph (the
    indexed path, which then skips its own rotation pass)."""
    print(f"prerotated keys {dtype} d{d} grid={grid}", flush=True)
    torch.manual_seed(9)
    b, h, g, shape = 1, 4, 2, (8, 16, 16)
    layout = p3d.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout="native_block_morton", device=gpu)
    geometry = layout.geometry
    if not grid:
        geometry = p3d.prepare_geometry(geometry.neighbors.clone(), geometry.blocks, pool_size=1)
    n = math.prod(shape)
    q, kl, vl, kg, vg = (torch.randn(b, x, n, d, device=gpu).to(dtype) for x in (h, g, g, g, g))
    gate = torch.rand(b, h, n, device=gpu).to(dtype)
    w, bias = torch.randn(d, device=gpu), torch.randn(64, device=gpu) * 0.3
    sl, sg = torch.rand(d, device=gpu) + 0.5, torch.rand(d, device=gpu) + 0.5
    layer = p3d.PACK3DAttention(h * d, heads=h, kv_heads=g, head_dim=d, block_volume=64).to(gpu)
    rope = layer._rope(torch.empty(b, n, h * d, device=gpu, dtype=dtype), layout)
    with torch.no_grad():
        plain = ForwardPlan(q, kl, vl, kg, vg, w, bias, gate, sl, sg, geometry, 0.7, rope, rope)
        y0, _ = plain.run()
        klr = _rotated(kl, rope)
        pre = ForwardPlan(q, klr, vl, kg, vg, w, bias, gate, sl, sg, geometry, 0.7, rope, rope, kl_rotated=True)
        assert pre.grid == grid
        y1, _ = pre.run()
    torch.cuda.synchronize()
    assert torch.isfinite(y0.float()).all()
    assert torch.equal(y0, y1), float((y0.float() - y1.float()).abs().max())


def test_project_pool_full_size_c2(gpu):
    """c2 (64^3 bf16, the benchmark layer): every summary of the fused kernel
    against p3d_project + p3d_pool_fwd."""
    print("project+pool full size c2", flush=True)
    shape = (64, 64, 64)
    torch.manual_seed(0)
    layer = p3d.PACK3DAttention(192, heads=4, kv_heads=4, head_dim=48, block_volume=64)
    for lin in (layer.to_q, layer.to_kv, layer.to_out):
        torch.nn.init.xavier_uniform_(lin.weight)
    layer = layer.to(gpu, torch.bfloat16)
    layout = p3d.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout="raster_block", device=gpu)
    x = torch.randn(1, math.prod(shape), 192, generator=torch.Generator().manual_seed(1)).to(gpu, torch.bfloat16)
    _compare(layer, x, layout, torch.bfloat16)


def _layer_both(layer, x, layout, monkeypatch):
    """The layer's no-grad output through the fusion and with it switched off;
    asserts which path each run took."""
    taken = []
    real = attention.pooled_core

    def spy(*args):
        out = real(*args)
        taken.append(out is not None)
        return out

    with torch.no_grad():
        monkeypatch.setattr(attention, "pooled_core", spy)
        fused = layer(x, layout)
        monkeypatch.setattr(attention, "pooled_core", lambda *args: None)
        plain = layer(x, layout)
    monkeypatch.setattr(attention, "pooled_core", real)
    return fused, plain, taken


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_layer_through_fusion_matches_unfused(gpu, dtype, monkeypatch):
    """The whole layer with the fused pooling against the same layer on
    p3d_project + the core: equal up to the summaries' last-bit differences
    carried through the attention (relative L2 well below the dtype's own
    rounding)."""
    print(f"layer fused vs unfused {dtype}", flush=True)
    layer = _layer(192, 4, 2, 48, dtype, gpu)
    shape = (8, 16, 16)
    layout = p3d.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout="raster_block", device=gpu)
    x = torch.randn(2, math.prod(shape), 192, generator=torch.Generator().manual_seed(5)).to(gpu, dtype)
    fused, plain, taken = _layer_both(layer, x, layout, monkeypatch)
    assert taken == [True]
    f32, p32 = fused.float(), plain.float()
    rel = float((f32 - p32).norm() / p32.norm())
    print(f"  rel_l2={rel:.3g} max_abs={float((f32 - p32).abs().max()):.3g}", flush=True)
    assert rel < STEP[dtype] / 4
    assert float((f32 - p32).abs().max()) <= 4 * STEP[dtype] * (float(p32.abs().max()) + 1.0)


def test_fusion_declines_shapes_it_does_not_take(gpu, monkeypatch):
    """head_dim 128, and a width whose LDS would not fit (dim 256 with 192 kv
    channels: p3d_project_pool answers P3D_EUNSUPPORTED before launching), take
    the unfused path with the same result; autograd also keeps it off."""
    print("fusion declines", flush=True)
    dtype = torch.bfloat16
    shape = (4, 8, 8)
    layout = p3d.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout="raster_block", device=gpu)
    for dim, heads, kv_heads, d in ((256, 2, 1, 128), (256, 4, 4, 48)):
        layer = _layer(dim, heads, kv_heads, d, dtype, gpu)
        x = torch.randn(1, math.prod(shape), dim, generator=torch.Generator().manual_seed(6)).to(gpu, dtype)
        with torch.no_grad():
            assert attention.pooled_core(layer, x, layout) is None
        fused, plain, taken = _layer_both(layer, x, layout, monkeypatch)
        assert taken == [False]
        assert torch.equal(fused, plain)
    layer = _layer(192, 4, 4, 48, dtype, gpu)
    x = torch.randn(1, math.prod(shape), 192, device=gpu, dtype=dtype)
    assert attention.pooled_core(layer, x, layout) is None  # parameters require grad, autograd on


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape,block,pool,kind", [
    ((4, 6, 10), (1, 1, 2), 5, "raster_block"),             # 2 slots: 32 fine blocks per 64-lane step
    ((6, 8, 10), (2, 2, 2), 3, "native_block_morton"),      # 8 slots, pools of 3 blocks
    ((5, 16, 16), (1, 4, 4), 16, "raster_block"),           # 16 slots, pool 16 (the allen15 preset's)
    ((4, 8, 12), (2, 4, 4), 5, "raster_block"),             # 32 slots, 2 blocks per step, a partial last summary
    ((8, 8, 8), (4, 4, 4), 32, "raster_block"),             # 64 slots: one block per step
    ((6, 9, 9), (3, 3, 3), 4, "raster_block"),              # 27 slots (not a power of two): one block per step
    ((4, 4, 8), (1, 1, 1), 32, "native_block_morton"),      # 1 slot: 32 blocks in one step
])
def test_pool_fwd_packed_steps_match_fp64_oracle(gpu, dtype, shape, block, pool, kind):
    """p3d_pool_fwd packs 64 / V fine blocks into each 64-lane step when the
    slot count V is a power of two up to 32 (a per-block slot softmax, the
    weighted sums over all 64 lanes).  Its summaries against the oracle's
    pooling in fp64 on the same rotated, rounded keys: within one unit in the
    last place of the storage type, as in the tests above; the key-norm slots
    against the norms of the stored keys."""
    import oracle.pack3d_oracle as ref
    vol = math.prod(block)
    print(f"pool packed {shape} block {block} (V={vol}) pool {pool} {kind} {dtype}", flush=True)
    torch.manual_seed(vol + pool)
    layer = p3d.PACK3DAttention(64, heads=2, kv_heads=2, head_dim=32, block_volume=vol, temperature=0.7)
    with torch.no_grad():
        layer.norm.weight.uniform_(0.5, 1.5)
        layer.pool_weight.normal_(0.0, 0.5)
        layer.slot_bias.normal_(0.0, 0.5)
    layer = layer.to(gpu, dtype)
    layout = p3d.build_layout(shape, block, radius=1, pool_size=pool, layout=kind, device=gpu)
    x = (torch.randn(2, math.prod(shape), 64, generator=torch.Generator().manual_seed(5)) * 1.5).to(gpu, dtype)
    rope = layer._rope(x, layout)
    with torch.no_grad():
        sep = attention._project_buffers(layer, x)
        _lib.call("p3d_project", sep[0], _lib.stream_of(gpu))
        plan = _plan(layer, sep, layout, rope)
        plan.pool()
    torch.cuda.synchronize()
    m = layout.geometry.num_summaries
    ks, vs = _summaries(plan, m)
    plan.geometry_cpu = layout.geometry.to("cpu")
    k64, v64 = _oracle_summaries(layer, sep, plan, rope, m)
    for what, got, r in (("keys", ks, k64), ("values", vs, v64)):
        u = _ulps(got.cpu(), r, dtype)
        print(f"  {what}: max ulps vs fp64 oracle {float(u.max()):.3g}", flush=True)
        assert torch.isfinite(got).all() and float(u.max()) <= 1.0, what
    # Key-norm slots: slot s of (batch, kv head) holds the largest norm of
    # the stored keys of summaries m = s mod 64 (times 1 + 1e-6).
    norms = ks.cpu().double().norm(dim=-1)
    b, g = norms.shape[:2]
    exp = torch.zeros(b, g, 64, dtype=torch.float64)
    for mm in range(m):
        exp[:, :, mm % 64] = torch.maximum(exp[:, :, mm % 64], norms[:, :, mm])
    got = plan.sk_norm_max.cpu().double().view(b, g, 64)
    assert torch.allclose(got, exp * (1 + 1e-6), rtol=1e-5, atol=0), float((got - exp).abs().max())
