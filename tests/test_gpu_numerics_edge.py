"""Numerical edge cases of the HIP core against the oracle.

* The summary softmax's fixed reference point with a bound 14-24 log2 units
  above the best score (tests/test_bound_emulation.py shows the inputs
  discriminate), in every dtype, through the brick and the rows kernel.
* Extreme finite logits: q, kl, vl x 8, pooling weight x 30, temperature
  0.03 (tests/test_triton.py:217-231 of amilworks/Pack3D), in every dtype.
* fp16 score gradients beyond fp16's range while the local VJPs fit
  (tests/test_triton.py:361-380): brick and indexed backward against each
  other and the oracle.
* Saved state: linear in N, nothing of size N x M, deterministic gradients
  (tests/test_triton.py:197-214).
"""
import math

import pytest
import torch

import oracle.pack3d_oracle as ref
import pack3d_amd as p3d
from tests._cases import make_case, max_abs, rel_l2
from tests.test_bound_emulation import SHAPE, loose_bound_case, oracle_geometry

pytestmark = pytest.mark.gpu

REL = {torch.float32: 3e-5, torch.float16: 5e-3, torch.bfloat16: 3.5e-2}
ABS = {torch.float32: 1e-5, torch.float16: 2e-2, torch.bfloat16: 2e-2}
NAMES = ["q", "kl", "vl", "kg", "vg", "pool_weight", "slot_bias", "gate", "local_scale", "global_scale"]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("grid", [True, False])
def test_loose_bound_band(gpu, dtype, grid):
    print(f"loose bound band grid={grid} {dtype}", flush=True)
    inputs = loose_bound_case(dtype)
    og = oracle_geometry()
    exp = ref.pack3d_reference(*inputs, og)
    if grid:
        geom = p3d.build_layout(SHAPE, (4, 4, 4), radius=2, pool_size=1, layout="raster_block").geometry
    else:
        geom = p3d.prepare_geometry(og.neighbors.to(gpu), og.blocks.to(gpu), 1)
    got = p3d.pack3d_hip(*(t.to(gpu) for t in inputs), geom)
    r = rel_l2(got, exp)
    # y = o_G here, with |o_G| up to ~2: max-abs is measured relative to max |y|.
    m = max_abs(got, exp) / max(1.0, float(exp.float().abs().max()))
    print(f"  rel_l2={r:.3g} scaled max_abs={m:.3g}", flush=True)
    assert torch.isfinite(got).all()
    assert r < REL[dtype] and m <= ABS[dtype]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_extreme_finite_logits(gpu, dtype):
    """Output and every gradient; fp32 at the reference's assert_close(2e-4),
    16-bit types at the relative-L2 bars of tests/test_triton.py:83."""
    print(f"extreme logits {dtype}", flush=True)
    inputs, nb, blocks, pool = make_case(n=97, b=1, h=4, g=2, volume=16, pool=4)
    for i in (0, 1, 2):
        inputs[i] = inputs[i] * 8
    inputs[5] = inputs[5] * 30
    inputs = [t.to(dtype) for t in inputs]
    og = ref.prepare_geometry(nb, blocks, pool)
    hg = p3d.prepare_geometry(nb.to(gpu), blocks.to(gpu), pool)
    xs = [t.to(gpu).requires_grad_() for t in inputs]
    rs = [t.detach().clone().requires_grad_() for t in inputs]
    y = p3d.pack3d_hip(*xs, hg, temperature=0.03)
    e = ref.pack3d_reference(*rs, og, temperature=0.03)
    up = torch.randn(e.shape, generator=torch.Generator().manual_seed(4)).to(dtype)
    got = torch.autograd.grad(y, xs, up.to(gpu))
    exp = torch.autograd.grad(e, rs, up)
    for name, a, b in zip(["y", *NAMES], [y, *got], [e, *exp]):
        assert torch.isfinite(a).all(), name
        err = rel_l2(a.float(), b.float())
        print(f"  {name}: rel_l2={err:.3g} max_abs={max_abs(a.float(), b.float()):.3g}", flush=True)
        if dtype == torch.float32:
            torch.testing.assert_close(a.cpu(), b, atol=2e-4, rtol=2e-4)
        else:
            assert err < REL[dtype], (name, err)


def test_fp16_large_score_gradients(gpu):
    """Tiny q and k, values +-1024 and upstream 1024: dS reaches ~6e5, beyond
    fp16, while dq, dk and dv fit.  The brick backward (which rescales dS
    before its fp16 MFMAs) must agree with the indexed fp32 backward and with
    the oracle."""
    print("fp16 large score gradients", flush=True)
    torch.manual_seed(27)
    lay = p3d.build_layout((8, 16, 32), layout="raster_block")
    geom = lay.geometry
    n, d = geom.num_tokens, 16
    q, k = [(torch.randn(1, 1, n, d) * .001).half() for _ in range(2)]
    sign = (torch.arange(n) % 2) * 2 - 1
    v = (sign.half() * 1024).view(1, 1, n, 1).expand(1, 1, n, d).contiguous()
    rest = [torch.zeros(1, 1, n, d).half(), torch.zeros(1, 1, n, d).half(), torch.zeros(d).half(),
            torch.zeros(8).half(), torch.zeros(1, 1, n).half(), torch.ones(d).half(), torch.zeros(d).half()]
    dy = torch.full((1, 1, n, d), 1024.).half()
    indexed = p3d.prepare_geometry(geom.neighbors, geom.blocks, geom.pool_size)
    results = []
    for g in (geom, indexed):
        xs = [t.to(gpu).requires_grad_() for t in (q, k, v)]
        y = p3d.pack3d_hip(*xs, *(t.to(gpu) for t in rest), g)
        results.append(torch.autograd.grad(y, xs, dy.to(gpu)))
    rs = [t.clone().requires_grad_() for t in (q, k, v)]
    lay_r = ref.build_layout((8, 16, 32), layout="raster_block")
    e = ref.pack3d_reference(*rs, *rest, lay_r.geometry)
    exp = torch.autograd.grad(e, rs, dy)
    for name, a, b, c in zip(("dq", "dk", "dv"), results[0], results[1], exp):
        assert torch.isfinite(a).all() and torch.isfinite(b).all(), name
        ab = rel_l2(a.float(), b.float())
        ac = rel_l2(a.float(), c.float())
        print(f"  {name}: brick vs indexed {ab:.3g}, brick vs oracle {ac:.3g}", flush=True)
        assert ab < 1e-3 and ac < 1e-3, name


def test_saved_state_is_linear_and_deterministic(gpu, monkeypatch):
    """The autograd function saves the ten inputs and seven states (sk, svt,
    the norm slots, o_L, o_G and the two log-sum-exps); the geometry stays on
    the context and is re-checked in backward.  Nothing saved has both an N
    and an M dimension, and two backward passes agree bit for bit."""
    print("saved state", flush=True)

    def forbidden(*args, **kwargs):
        raise AssertionError("the hip backend called torch's SDPA")

    monkeypatch.setattr(torch.nn.functional, "scaled_dot_product_attention", forbidden)
    inputs, nb, blocks, pool = make_case(n=2053, b=1, h=2, g=1, d=16)
    hg = p3d.prepare_geometry(nb.to(gpu), blocks.to(gpu), pool)
    xs = [t.to(gpu).requires_grad_() for t in inputs]
    saved = []

    def record(t):
        saved.append(tuple(t.shape))
        return t

    with torch.autograd.graph.saved_tensors_hooks(record, lambda t: t):
        y = p3d.pack3d_hip(*xs, hg)
    n, m = hg.num_tokens, hg.num_summaries
    assert len(saved) == 17, saved
    assert all(not (n in s and m in s) for s in saved), saved
    assert sum(math.prod(s) for s in saved) < 40 * n * 16
    dy = torch.randn_like(y)
    g1 = torch.autograd.grad(y, xs, dy, retain_graph=True)
    g2 = torch.autograd.grad(y, xs, dy)
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)
