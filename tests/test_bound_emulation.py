"""The summary pass's fixed softmax reference point, emulated on the CPU.

The attention kernels score summaries against B_q = |q| max_m |sk_m|
(Cauchy-Schwarz) instead of a running max, round p = 2^(s - B_q) to the
storage type and feed it to the PV and denominator MFMAs.  This file builds
inputs whose bound lies 14-24 log2 units above the true maximum score and
shows, with an emulation of that arithmetic in float64 (p rounded to the
storage type), that the inputs discriminate: fp16 probabilities fall into
fp16's subnormal range and the bounded algorithm misses the fp16 bar, while
bf16 keeps its 8 significant bits and stays far inside its bar.  The GPU
test (tests/test_gpu_numerics_edge.py) runs the kernels on the same inputs;
fp16 must therefore take the running-max softmax to pass.
"""
import math

import torch

import oracle.pack3d_oracle as ref
from tests._cases import rel_l2

SHAPE = (8, 16, 32)
D = 48


def loose_bound_case(dtype, seed=0, c=1.2, q_norm=22.0, sigma_k=6.0):
    """Core inputs (q, kl, kg pre-rotated) on a raster 8 x 16 x 32 grid with 4^3
    blocks (64 summaries).  Queries (norm q_norm) and keys live in channels
    0..23, except fine block 0, whose keys are the constant c in channels
    24..47: its summary is orthogonal to every query but has a large norm, so
    the bound overshoots the best score.  Mean pooling; y = o_G (sl = 0,
    gate = sg = 1)."""
    gen = torch.Generator().manual_seed(seed)
    n = math.prod(SHAPE)
    half = D // 2
    q = torch.zeros(1, 2, n, D)
    u = torch.randn(1, 2, n, half, generator=gen)
    q[..., :half] = u / u.norm(dim=-1, keepdim=True) * q_norm
    kg = torch.zeros(1, 2, n, D)
    kg[..., :half] = torch.randn(1, 2, n, half, generator=gen) * sigma_k
    kg[:, :, :64] = 0
    kg[:, :, :64, half:] = c
    kl = torch.randn(1, 2, n, D, generator=gen) * 0.5
    vl = torch.randn(1, 2, n, D, generator=gen) * 0.5
    vg = torch.randn(1, 2, n, D, generator=gen) * 4.0
    inputs = [q, kl, vl, kg, vg, torch.zeros(D), torch.zeros(64), torch.ones(1, 2, n), torch.zeros(D),
              torch.ones(D)]
    return [t.to(dtype) for t in inputs]


def oracle_geometry():
    return ref.build_layout(SHAPE, (4, 4, 4), radius=2, pool_size=1, layout="raster_block").geometry


def emulate_bounded(inputs, geometry, dtype):
    """o_G of the bounded summary pass in float64, with the kernel's rounding
    points: pooled keys stored in ``dtype`` pre-scaled by log2(e)/sqrt(d),
    pooled values stored in ``dtype``, p = 2^(s - B) rounded to ``dtype``, the
    denominator summed from the rounded p.  Also returns the bound gap
    B - max s per query in log2 units."""
    q, _, _, kg, vg = (t.double() for t in inputs[:5])
    sk, sv = ref.compress_summaries(kg, vg, inputs[5].double(), inputs[6].double(), geometry)
    scale = math.log2(math.e) / math.sqrt(D)
    sk = (sk * scale).to(dtype).double()
    sv = sv.to(dtype).double()
    bound = q.norm(dim=-1, keepdim=True) * sk.norm(dim=-1).amax(-1)[..., None, None]
    s = q @ sk.transpose(-1, -2)
    p = torch.exp2(s - bound).to(dtype).double()
    og = (p @ sv) / p.sum(-1, keepdim=True)
    gap = (bound[..., 0] - s.amax(-1))
    return og, gap


def test_bound_gap_lies_in_band_and_discriminates():
    geometry = oracle_geometry()
    for dtype, expect_bad in ((torch.float16, True), (torch.bfloat16, False)):
        inputs = loose_bound_case(dtype)
        exp = ref.pack3d_reference(*inputs, geometry).double()
        og, gap = emulate_bounded(inputs, geometry, dtype)
        in_band = ((gap >= 14) & (gap <= 24)).double().mean().item()
        assert in_band > 0.95, in_band
        assert torch.isfinite(og).all()  # no query underflows completely (no fallback)
        err = rel_l2(og, exp)
        if expect_bad:
            assert err > 2 * 5e-3, err     # misses the fp16 relative-L2 bar by a margin
        else:
            assert err < 3.5e-2 / 4, err   # bf16: well inside its bar
