"""Pins for the oracle's RoPE, pooling, core and layer restatements (CPU).

Each check is chosen so that a plausible slip (wrong pair/axis assignment,
a transposed operand, a wrong softmax axis, a dropped mask or scale, a wrong
GQA head map, the count of the coarse mean) fails at least one of them:

* RoPE: balanced_pairs known answers (tests/test_rope.py:6-7), an exact
  closed-form rotation computed with ``math`` in fp64, zero angle = identity,
  the relative-position identity and norm preservation (test_rope.py:10-18).
* Pooling: brute force with Python floats, the w=0/b=0 arithmetic mean,
  empty fine blocks excluded from the count, the relative-logit identity
  (tests/test_compression.py:7-21).
* Core: brute-force fp64 Python loops over a ragged asymmetric graph
  (the make_case generator of tests/test_triton.py:27-49), chunking and
  row sampling invariance, fp64 gradcheck (test_triton.py:52-55), the
  singleton-summary special case (test_triton.py:262-271).
* Layer: repack equivariance of outputs and all gradients at 1e-10 in fp64
  with the packed-position control (tests/test_repacking.py:5-23).
"""
import math

import pytest
import torch

from oracle.pack3d_oracle import (PACK3DAttention, axial_rope, balanced_pairs, build_layout,
                                  compress_summaries, pack3d_reference, pack3d_reference_grads,
                                  prepare_geometry)


def test_balanced_pairs_known_answers():
    assert balanced_pairs(64) == (11, 11, 10)
    assert balanced_pairs(48) == (8, 8, 8)
    assert balanced_pairs(16) == (3, 3, 2)
    with pytest.raises(ValueError):
        balanced_pairs(15)


def test_rope_closed_form():
    d = 48
    coords = torch.tensor([[3, 5, 7], [0, 0, 0], [60, 1, 33]])
    x = torch.randn(1, 2, 3, d, dtype=torch.float64, generator=torch.Generator().manual_seed(0))
    out = axial_rope(x, coords)
    pairs = balanced_pairs(d)
    for t in range(3):
        off = 0
        for axis, cnt in enumerate(pairs):
            for j in range(cnt):
                ang = float(coords[t, axis]) * 10000.0 ** (-j / cnt)
                c, s = math.cos(ang), math.sin(ang)
                for h in range(2):
                    a, b = float(x[0, h, t, off + 2 * j]), float(x[0, h, t, off + 2 * j + 1])
                    assert abs(float(out[0, h, t, off + 2 * j]) - (a * c - b * s)) < 1e-12
                    assert abs(float(out[0, h, t, off + 2 * j + 1]) - (a * s + b * c)) < 1e-12
            off += 2 * cnt
    # Zero coordinates are the exact identity, also after the fp32 round trip.
    xb = torch.randn(1, 1, 4, d).to(torch.bfloat16)
    assert torch.equal(axial_rope(xb, torch.zeros(4, 3, dtype=torch.long)), xb)


def test_rope_relative_identity_and_norm():
    torch.manual_seed(3)
    q, k = torch.randn(2, 1, 1, 7, 48, dtype=torch.float64)
    c, d = torch.randn(2, 7, 3, dtype=torch.float64)
    qr, kr = axial_rope(q, c), axial_rope(k, d)
    assert (qr - q).abs().max() > 0.01
    torch.testing.assert_close((qr * kr).sum(-1), (q * axial_rope(k, d - c)).sum(-1), atol=1e-12, rtol=1e-12)
    torch.testing.assert_close(q.square().sum(-1), qr.square().sum(-1), atol=1e-12, rtol=1e-12)


@pytest.mark.parametrize("pairs", [(0, 0, 0), (8, 0, -1), (3, 3, 3), (True, 3, 4)])
def test_rope_rejects_bad_pairs(pairs):
    with pytest.raises(ValueError):
        axial_rope(torch.randn(1, 1, 4, 16), torch.zeros(4, 3), pairs=pairs)


def make_case(n=37, d=16, b=2, h=4, g=2, volume=4, pool=3, dtype=torch.float32, seed=18):
    """Ragged asymmetric graph with an all-masked row and a padded last block.

    Same construction as the generator at tests/test_triton.py:27-49 of the
    reference (edges {i, i+1 mod n, max(i-2,0)}, row 0 empty).
    """
    gen = torch.Generator().manual_seed(seed)
    nb = torch.full((n, 5), -1, dtype=torch.int32)
    for i in range(n):
        edges = sorted({i, (i + 1) % n, max(i - 2, 0)})
        nb[i, :len(edges)] = torch.tensor(edges)
    nb[0] = -1
    blocks = torch.full(((n + volume - 1) // volume, volume), -1, dtype=torch.int32)
    blocks.view(-1)[:n] = torch.arange(n)
    geometry = prepare_geometry(nb, blocks, pool)
    shapes = [(b, h, n, d)] + [(b, g, n, d)] * 4 + [(d,), (volume,), (b, h, n), (d,), (d,)]
    inputs = []
    for index, shape in enumerate(shapes):
        t = torch.randn(shape, generator=gen) * (0.2 if index in (5, 6) else 0.5)
        if index == 7:
            t = t.sigmoid()
        if index == 8:
            t = t + 1
        if index == 9:
            t = t + 0.25
        inputs.append(t.to(dtype))
    return inputs, geometry


def brute_core(inputs, geometry, tau):
    """fp64 Python-loop evaluation of the core contract."""
    q, kl, vl, kg, vg, w, bias, gate, sl, sg = [t.double().tolist() for t in inputs]
    B, H, N, D = inputs[0].shape
    G = inputs[1].shape[1]
    blocks = geometry.blocks.tolist()
    P = geometry.pool_size
    nb = geometry.neighbors.tolist()
    # Pooling per (b, g): fine softmax pooling, then mean over non-empty fine blocks.
    sk = [[[] for _ in range(G)] for _ in range(B)]
    sv = [[[] for _ in range(G)] for _ in range(B)]
    for bb in range(B):
        for gg in range(G):
            fine = []
            for row in blocks:
                mem = [(s, t) for s, t in enumerate(row) if t >= 0]
                if not mem:
                    fine.append(None)
                    continue
                lg = [sum(kg[bb][gg][t][c] * w[c] for c in range(D)) / tau + bias[s] for s, t in mem]
                mx = max(lg)
                e = [math.exp(v - mx) for v in lg]
                tot = sum(e)
                fk = [sum(e[i] / tot * kg[bb][gg][t][c] for i, (s, t) in enumerate(mem)) for c in range(D)]
                fv = [sum(e[i] / tot * vg[bb][gg][t][c] for i, (s, t) in enumerate(mem)) for c in range(D)]
                fine.append((fk, fv))
            for start in range(0, len(fine), P):
                grp = [f for f in fine[start:start + P] if f is not None]
                sk[bb][gg].append([sum(f[0][c] for f in grp) / len(grp) for c in range(D)])
                sv[bb][gg].append([sum(f[1][c] for f in grp) / len(grp) for c in range(D)])
    out = torch.zeros(B, H, N, D, dtype=torch.float64)
    root = math.sqrt(D)
    for bb in range(B):
        for hh in range(H):
            gg = hh // (H // G)
            for i in range(N):
                qi = q[bb][hh][i]
                sc = [sum(qi[c] * k[c] for c in range(D)) / root for k in sk[bb][gg]]
                mx = max(sc)
                e = [math.exp(s - mx) for s in sc]
                og = [sum(e[m] * sv[bb][gg][m][c] for m in range(len(e))) / sum(e) for c in range(D)]
                valid = [j for j in nb[i] if j >= 0]
                if valid:
                    sc = [sum(qi[c] * kl[bb][gg][j][c] for c in range(D)) / root for j in valid]
                    mx = max(sc)
                    e = [math.exp(s - mx) for s in sc]
                    ol = [sum(e[t] * vl[bb][gg][j][c] for t, j in enumerate(valid)) / sum(e) for c in range(D)]
                else:
                    ol = [0.0] * D
                for c in range(D):
                    out[bb, hh, i, c] = sl[c] * ol[c] + gate[bb][hh][i] * sg[c] * og[c]
    return out


@pytest.mark.parametrize("shape", [(37, 16, 2, 4, 2, 4, 3), (19, 32, 1, 2, 2, 3, 1), (21, 48, 1, 2, 1, 4, 4)])
def test_core_matches_brute_force(shape):
    inputs, geometry = make_case(*shape, dtype=torch.float64)
    got = pack3d_reference(*inputs, geometry, temperature=0.7, chunk=5)
    ref = brute_core(inputs, geometry, 0.7)
    torch.testing.assert_close(got, ref, atol=1e-12, rtol=1e-12)


def test_core_rows_and_chunks_invariant():
    inputs, geometry = make_case(n=67, d=48, dtype=torch.float64)
    full = pack3d_reference(*inputs, geometry, chunk=1000)
    rows = torch.tensor([0, 5, 66, 31])
    part = pack3d_reference(*inputs, geometry, rows=rows, chunk=3)
    torch.testing.assert_close(part, full[:, :, rows], atol=1e-14, rtol=1e-14)


def test_core_gradcheck():
    inputs, geometry = make_case(n=3, b=1, h=1, g=1, volume=2, pool=2, dtype=torch.float64)
    inputs = [t.requires_grad_() for t in inputs]
    assert torch.autograd.gradcheck(lambda *a: pack3d_reference(*a, geometry, temperature=0.7),
                                    tuple(inputs), fast_mode=True)


def test_singleton_summary_is_its_value():
    inputs, geometry = make_case(n=1, b=1, h=1, g=1, volume=1, pool=1, dtype=torch.float64)
    inputs = [t.requires_grad_() for t in inputs]
    y, ol, og = pack3d_reference(*inputs, geometry, return_branches=True)
    torch.testing.assert_close(og[0, 0, 0], inputs[4][0, 0, 0].detach(), atol=1e-15, rtol=0)
    assert torch.equal(ol, torch.zeros_like(ol))
    grads = torch.autograd.grad(y, inputs, torch.randn_like(y))
    for index in (0, 1, 2, 3, 5, 6):
        assert torch.count_nonzero(grads[index]) == 0


def test_pool_mean_and_empty_blocks():
    torch.manual_seed(1)
    n, d = 24, 16
    nb = torch.arange(n)[:, None].int()
    blocks = torch.full((7, 4), -1, dtype=torch.int32)
    perm = torch.randperm(n)
    blocks[0, :3] = perm[:3].int()
    blocks[2] = perm[3:7].int()
    blocks[3, 1:] = perm[7:10].int()
    blocks[4] = perm[10:14].int()
    blocks[5] = perm[14:18].int()
    blocks[6, :2] = perm[18:20].int()
    blocks[1, :4] = perm[20:24].int()
    geom = prepare_geometry(nb, blocks, 2)
    k, v = torch.randn(2, 1, 2, n, d, dtype=torch.float64)
    sk, sv = compress_summaries(k, v, torch.zeros(d, dtype=torch.float64),
                                torch.zeros(4, dtype=torch.float64), geom)
    assert sk.shape == (1, 2, 4, d)
    for m in range(4):
        fines = []
        for f in range(2 * m, min(2 * m + 2, 7)):
            mem = [t for t in blocks[f].tolist() if t >= 0]
            if mem:
                fines.append((k[:, :, mem].mean(2), v[:, :, mem].mean(2)))
        torch.testing.assert_close(sk[:, :, m], sum(f[0] for f in fines) / len(fines), atol=1e-14, rtol=0)
        torch.testing.assert_close(sv[:, :, m], sum(f[1] for f in fines) / len(fines), atol=1e-14, rtol=0)
    # An empty fine block (not a group) contributes neither mass nor count.
    blocks2 = torch.cat((torch.full((1, 4), -1, dtype=torch.int32), blocks[1:]))
    blocks2 = torch.cat((blocks2, blocks[:1]))
    geom2 = prepare_geometry(nb, blocks2, 2)
    sk2, _ = compress_summaries(k, v, torch.zeros(d, dtype=torch.float64),
                                torch.zeros(4, dtype=torch.float64), geom2)
    mem = [t for t in blocks[1].tolist() if t >= 0]
    torch.testing.assert_close(sk2[:, :, 0], k[:, :, mem].mean(2), atol=1e-14, rtol=0)


def test_pool_relative_logit_identity():
    torch.manual_seed(4)
    layout = build_layout((2, 2, 4), pool_size=2)
    q, k, v = torch.randn(3, 1, 1, 16, 16, dtype=torch.float64)
    w, bias = torch.randn(16, dtype=torch.float64), torch.randn(8, dtype=torch.float64)
    rotated = axial_rope(k, layout.coords)
    sk, _ = compress_summaries(rotated, v, w, bias, layout.geometry, temperature=.7)
    index = layout.geometry.blocks.long()
    a = ((rotated[:, :, index] * w).sum(-1) / .7 + bias).softmax(-1)
    effective = a.flatten(-2) / 2
    for i in (0, 7, 15):
        relative = axial_rope(k, layout.coords - layout.coords[i])
        rhs = ((q[:, :, i, None] * relative).sum(-1) * effective).sum(-1)
        lhs = (axial_rope(q, layout.coords)[:, :, i] * sk[:, :, 0]).sum(-1)
        torch.testing.assert_close(lhs, rhs, atol=1e-12, rtol=1e-12)


def test_layer_repack_equivariance_fp64():
    torch.manual_seed(21)
    layout = build_layout((4, 4, 4), pool_size=2)
    p = torch.randperm(64)
    other = layout.repack(p)
    layer = PACK3DAttention(16, heads=2, kv_heads=1, head_dim=16).double()
    x = torch.randn(1, 64, 16, dtype=torch.float64, requires_grad=True)
    xp = x.detach()[:, p].clone().requires_grad_()
    y, yp = layer(x, layout), layer(xp, other)
    torch.testing.assert_close(y, yp[:, p.argsort()], atol=1e-10, rtol=1e-10)
    dy = torch.randn_like(y)
    gs = torch.autograd.grad(y, (x, *layer.parameters()), dy)
    gps = torch.autograd.grad(yp, (xp, *layer.parameters()), dy[:, p])
    torch.testing.assert_close(gs[0], gps[0][:, p.argsort()], atol=1e-10, rtol=1e-10)
    for a, b in zip(gs[1:], gps[1:]):
        torch.testing.assert_close(a, b, atol=1e-10, rtol=1e-10)
    layer.position_encoding = "packed"
    assert (layer(x, layout) - layer(xp, other)[:, p.argsort()]).abs().max() > 1e-4


def test_layer_shapes_d48_and_state_dict_names():
    torch.manual_seed(12)
    layout = build_layout((4, 4, 4), (4, 4, 4), radius=2, pool_size=1, layout="raster_block")
    layer = PACK3DAttention(192, heads=4, kv_heads=4, head_dim=48, block_volume=64).double()
    x = torch.randn(1, 64, 192, dtype=torch.float64, requires_grad=True)
    y = layer(x, layout)
    assert y.shape == x.shape
    y.square().sum().backward()
    assert all(p.grad is not None and torch.isfinite(p.grad).all() for p in layer.parameters())
    assert set(layer.state_dict()) == {"norm.weight", "norm.bias", "to_q.weight", "to_kv.weight",
                                        "pool_weight", "slot_bias", "gate.weight", "gate.bias",
                                        "local_scale", "global_scale", "to_out.weight"}


@pytest.mark.parametrize("case", ["ragged", "grid_gqa"])
def test_chunked_backward_equals_autograd(case):
    """pack3d_reference_grads (one autograd graph per chunk of query rows)
    against torch.autograd.grad through pack3d_reference, in fp64: every
    gradient to 1e-12, with chunks that do not divide the token count."""
    if case == "ragged":
        inputs, geometry = make_case(n=37, d=16, b=2, h=4, g=2, volume=4, pool=3, dtype=torch.float64)
        tau = 0.7
    else:
        layout = build_layout((4, 6, 4), (2, 2, 2), radius=(1, 2, 1), pool_size=2)
        gen = torch.Generator().manual_seed(5)
        n = 96
        shapes = [(1, 4, n, 16)] + [(1, 2, n, 16)] * 4 + [(16,), (8,), (1, 4, n), (16,), (16,)]
        inputs = [torch.randn(s, generator=gen, dtype=torch.float64) for s in shapes]
        inputs[7] = inputs[7].sigmoid()
        geometry, tau = layout.geometry, 0.6
    xs = [t.clone().requires_grad_() for t in inputs]
    y = pack3d_reference(*xs, geometry, temperature=tau)
    dy = torch.randn(y.shape, generator=torch.Generator().manual_seed(9), dtype=torch.float64)
    exp = torch.autograd.grad(y, xs, dy)
    got = pack3d_reference_grads(*inputs, geometry, dy, temperature=tau, chunk=7)
    for a, b in zip(got, exp):
        torch.testing.assert_close(a, b, atol=1e-12, rtol=1e-12)
