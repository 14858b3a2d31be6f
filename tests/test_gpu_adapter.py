"""The paper adapter's core call on the HIP backend.

``StreamedPACK3D.forward`` (reproduce/paper_backend/hypernsa/attention/
streamed_adapter.py:94-96 of amilworks/Pack3D) calls

    pack3d_streamed(q, kl, vl, kg, vg, l.atom_logits.weight[0],
                    l.atom_rel_bias[:, 0], gates[..., 1], sl, sg, self.geometry,
                    temperature=max(l.atom_temperature, 1e-6))

with q, kl, kg already rotated by the historical layer, a geometry from the
reference's ``prepare_geometry`` over the historical neighbour table (built
in itertools.product offset order, layout.py:428-475, absent entries -1) and
block table, ``gates`` a softmax over three branch logits laid out
[B, H, N, 3] by a permute, the Allen-15 shapes (head_dim 64, 8 query / 2 kv
heads, radius 1, (1, 4, 4) raster blocks, summary pool 16).  ``pack3d_hip``
takes the same call; here against the oracle, forward and all ten gradients,
first on the indexed kernels (the geometry carries no tag) and again after
``adopt_layout`` proves the stencil.  The adapter itself (hypernsa) is not
run: its inputs are built with the same shapes, strides and dtypes.
"""
import math
from types import SimpleNamespace

import pytest
import torch

import oracle.pack3d_oracle as ref
import pack3d_amd as p3d
from pack3d_amd.core import brick_tag
from tests._cases import rel_l2
from tests._refobjects import reference_layout

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 3e-5, torch.bfloat16: 3.5e-2}


def _adapter_inputs(n, dtype, seed=0):
    gen = torch.Generator().manual_seed(seed)
    b, h, g, d, v = 1, 8, 2, 64, 16
    q = torch.randn(b, h, n, d, generator=gen) * 0.5
    kl, vl, kg, vg = (torch.randn(b, g, n, d, generator=gen) * 0.5 for _ in range(4))
    atom_logits = torch.randn(1, d, generator=gen) * 0.2          # nn.Linear(d, 1).weight
    atom_rel_bias = torch.randn(v, 1, generator=gen) * 0.2        # [slots, num_atoms]
    logits = torch.randn(b, n, h, 3, generator=gen).permute(0, 2, 1, 3)
    gates = logits.softmax(-1)                                    # [B, H, N, 3], permuted strides
    scale = torch.tensor([1.0, 0.25, 0.0])[:, None] + 0.1 * torch.randn(3, d, generator=gen)
    return [t.to(dtype) for t in (q, kl, vl, kg, vg)], atom_logits, atom_rel_bias, gates, scale


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_adapter_call(gpu, dtype):
    print(f"adapter call {dtype}", flush=True)
    shape = (8, 16, 32)
    n = math.prod(shape)
    lay_o = ref.build_layout(shape, (1, 4, 4), radius=1, pool_size=16, layout="raster_block")
    lay = reference_layout(lay_o, gpu)
    # The adapter's geometry comes from prepare_geometry over the raw tables:
    # no radius-one tag, unlike the layout build_layout would return.
    g0 = lay.geometry
    geometry = type(g0)(g0.neighbors, g0.reverse_neighbors, g0.blocks, 16, n)
    assert brick_tag(geometry) is None
    qkv, atom_logits, atom_rel_bias, gates, scale = _adapter_inputs(n, dtype)
    temperature = max(0.5, 1e-6)

    def call(core, tensors, params, geom):
        w, bias, gts, sc = params
        sl, sg = sc[:2].to(tensors[0].dtype).unbind(0)
        return core(*tensors, w[0], bias[:, 0], gts[..., 1], sl, sg, geom, temperature=temperature)

    for tagged in (False, True):
        if tagged:
            # What the adapter would add at its construction (streamed_adapter.py:32):
            # prove the table is the radius-one stencil of the historical grid.
            p3d.adopt_layout(SimpleNamespace(grid_shape=shape, order=lay.order, geometry=geometry))
            assert brick_tag(geometry) is not None
        xs = [t.to(gpu).requires_grad_() for t in qkv]
        ps = [t.to(gpu).requires_grad_() for t in (atom_logits, atom_rel_bias, gates, scale)]
        assert not ps[2][..., 1].is_contiguous()
        y = call(p3d.pack3d_hip, xs, ps, geometry)
        rs = [t.detach().clone().requires_grad_() for t in qkv]
        rp = [t.detach().clone().requires_grad_() for t in (atom_logits, atom_rel_bias, gates, scale)]
        e = call(ref.pack3d_reference, rs, rp, lay_o.geometry)
        up = torch.randn(e.shape, generator=torch.Generator().manual_seed(4)).to(dtype)
        got = torch.autograd.grad(y, xs + ps, up.to(gpu))
        exp = torch.autograd.grad(e, rs + rp, up)
        for name, a, b_ in zip(["y", "q", "kl", "vl", "kg", "vg", "atom_logits", "atom_rel_bias", "gates",
                                "branch_scale"], [y, *got], [e, *exp]):
            assert torch.isfinite(a).all(), name
            err = rel_l2(a.float(), b_.float())
            print(f"  tagged={tagged} {name}: rel_l2={err:.3g}", flush=True)
            assert err < TOL[dtype], (tagged, name, err)
            if dtype == torch.float32:
                torch.testing.assert_close(a.cpu(), b_, atol=3e-5, rtol=3e-5)
