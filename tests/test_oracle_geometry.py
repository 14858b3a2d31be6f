"""Pins for the oracle's geometry restatement (CPU).

The reference holds no geometry fixtures; these checks pin the restatement
with brute force over explicit coordinate loops, the closed-form Morton bit
layout, the known answers of the reference docs (docs/method.md:25-28) and
the invariants of the reference tests (tests/test_geometry.py).
"""
import itertools
import math

import pytest
import torch

from oracle.pack3d_oracle import (build_layout, grid_coordinates, morton_codes, neighbor_offsets,
                                  prepare_geometry, reverse_adjacency)


def _interleave(z, y, x, nbits):
    code = 0
    for b in range(nbits):
        for axis, c in enumerate((z, y, x)):
            code |= ((c >> b) & 1) << (3 * b + axis)
    return code


def brute_layout(shape, block, radius, kind):
    """Pure-Python construction of order / neighbours from coordinates."""
    Z, Y, X = shape
    pts = [(z, y, x) for z in range(Z) for y in range(Y) for x in range(X)]
    if kind == "raster_block":
        order = list(range(len(pts)))
    else:
        slots = [tuple(c % b for c, b in zip(p, block)) for p in pts]
        blks = [tuple(c // b for c, b in zip(p, block)) for p in pts]
        sbits = max(max(s) for s in slots).bit_length()
        bbits = max(max(b) for b in blks).bit_length()
        scode = [_interleave(*s, sbits) for s in slots]
        bcode = [_interleave(*b, bbits) for b in blks]
        mult = max(scode) + 1
        order = sorted(range(len(pts)), key=lambda i: bcode[i] * mult + scode[i])
    pos = {pts[r]: i for i, r in enumerate(order)}
    offsets = list(itertools.product(*(range(-r, r + 1) for r in radius)))
    nb = []
    for r in order:
        z, y, x = pts[r]
        nb.append([pos.get((z + dz, y + dy, x + dx), -1) for dz, dy, dx in offsets])
    return order, [pts[r] for r in order], nb


@pytest.mark.parametrize("shape,block,radius,kind", [
    ((4, 4, 4), (2, 2, 2), 1, "native_block_morton"),
    ((4, 4, 4), (2, 2, 2), 2, "raster_block"),
    ((4, 6, 8), (2, 2, 4), (1, 2, 0), "native_block_morton"),
    ((3, 5, 4), (1, 5, 2), 2, "raster_block"),
    ((8, 4, 4), (4, 4, 4), 2, "native_block_morton"),
    ((2, 8, 6), (2, 4, 3), (0, 1, 1), "native_block_morton"),
])
def test_build_layout_matches_brute_force(shape, block, radius, kind):
    rad = (radius,) * 3 if isinstance(radius, int) else radius
    layout = build_layout(shape, block, radius=radius, pool_size=1, layout=kind)
    order, coords, nb = brute_layout(shape, block, rad, kind)
    assert layout.order.tolist() == order
    assert layout.coords.tolist() == [list(c) for c in coords]
    assert layout.geometry.neighbors.tolist() == nb
    vol = math.prod(block)
    assert layout.geometry.blocks.tolist() == [list(range(i, i + vol)) for i in range(0, len(order), vol)]
    # Reverse adjacency: row j lists ascending the rows i that use j.
    n = len(order)
    users = [[] for _ in range(n)]
    for i, row in enumerate(nb):
        for j in row:
            if j >= 0:
                users[j].append(i)
    width = max(1, max(len(u) for u in users))
    assert layout.geometry.reverse_neighbors.tolist() == [u + [-1] * (width - len(u)) for u in users]


def test_known_answers_from_method_doc():
    # docs/method.md:25-28: first native block of a 4^3 grid with 2^3 blocks,
    # 8 valid neighbours at the corner and 27 at (1,1,1).
    layout = build_layout((4, 4, 4), (2, 2, 2), pool_size=2)
    first = layout.coords[layout.geometry.blocks[0].long()].tolist()
    assert first == [[0, 0, 0], [1, 0, 0], [0, 1, 0], [1, 1, 0], [0, 0, 1], [1, 0, 1], [0, 1, 1], [1, 1, 1]]
    valid = (layout.geometry.neighbors >= 0).sum(1)
    corner = (layout.coords == torch.tensor([0, 0, 0])).all(1)
    inner = (layout.coords == torch.tensor([1, 1, 1])).all(1)
    assert int(valid[corner]) == 8 and int(valid[inner]) == 27
    assert layout.geometry.neighbors.shape == (64, 27)
    assert layout.geometry.num_summaries == 4


def test_morton_closed_form_and_centre_column():
    c = grid_coordinates((5, 7, 9))
    codes = morton_codes(c)
    for i in range(0, c.shape[0], 17):
        z, y, x = c[i].tolist()
        assert int(codes[i]) == _interleave(z, y, x, 4)
    # Column ((dz+r)(2r+1)+(dy+r))(2r+1)+(dx+r); the centre column is the query itself.
    offs = neighbor_offsets((2, 2, 2))
    assert offs[62] == (0, 0, 0) and offs[0] == (-2, -2, -2) and offs[1] == (-2, -2, -1)
    layout = build_layout((8, 8, 8), (4, 4, 4), radius=2, pool_size=1, layout="raster_block")
    assert torch.equal(layout.geometry.neighbors[:, 62].long(), torch.arange(512))
    with pytest.raises(ValueError, match="Morton"):
        morton_codes(torch.tensor([[1 << 20, 0, 0]]))


def test_edge_count_closed_form():
    # Valid edges per axis of extent n >= 4 at radius 2 total 5n - 6; the
    # stencil is a product, so E = prod(5n_a - 6).
    for shape in ((16, 16, 16), (4, 9, 5)):
        layout = build_layout(shape, (4, 1, 1) if shape[0] % 4 == 0 else (1, 1, 1), radius=2,
                              pool_size=1, layout="raster_block")
        expect = math.prod(5 * s - 6 for s in shape)
        assert int((layout.geometry.neighbors >= 0).sum()) == expect


def test_pack_unpack_and_repack_transport():
    layout = build_layout((4, 4, 8), pool_size=2)
    grid = torch.randn(2, 4, 4, 8, 3)
    torch.testing.assert_close(layout.unpack(layout.pack(grid)), grid)
    p = torch.randperm(128, generator=torch.Generator().manual_seed(5))
    new = layout.repack(p)
    torch.testing.assert_close(new.pack(grid), layout.pack(grid)[:, p])
    torch.testing.assert_close(new.unpack(new.pack(grid)), grid)
    torch.testing.assert_close(new.coords[new.geometry.blocks.long()],
                               layout.coords[layout.geometry.blocks.long()])
    # The neighbour relation is transported: same coordinates in the same columns.
    def nb_coords(lay):
        idx = lay.geometry.neighbors.long()
        return torch.where(idx[..., None] >= 0, lay.coords[idx.clamp_min(0)], -1)
    inv = p.argsort()
    torch.testing.assert_close(nb_coords(new)[inv], nb_coords(layout))
    assert torch.equal(new.geometry.raster_to_packed.long(), new.order.argsort())
    back = new.repack(new.order.argsort())
    assert back.geometry.raster_to_packed is None and back.geometry.grid == layout.geometry.grid


@pytest.mark.parametrize("kwargs", [{"grid_shape": (3, 4, 4)}, {"radius": -1},
                                    {"block_shape": (0, 2, 2)}, {"layout": "unknown"},
                                    {"pool_size": True}, {"radius": 3}])
def test_bad_layout_rejected(kwargs):
    args = {"grid_shape": (4, 4, 4), **kwargs}
    with pytest.raises(ValueError):
        build_layout(**args)


def test_prepare_geometry_guards_and_mutation():
    nb = torch.tensor([[0, 1], [1, -1], [2, 0]], dtype=torch.int32)
    blocks = torch.tensor([[0, 1], [2, -1]], dtype=torch.int32)
    geom = prepare_geometry(nb, blocks, 1)
    assert geom.reverse_neighbors.tolist() == [[0, 2], [0, 1], [2, -1]]
    with pytest.raises(ValueError, match="out-of-range"):
        prepare_geometry(nb + 5, blocks, 1)
    with pytest.raises(ValueError, match="duplicate"):
        prepare_geometry(torch.tensor([[0, 0], [1, -1], [2, -1]]), blocks, 1)
    with pytest.raises(ValueError, match="partition"):
        prepare_geometry(nb, torch.zeros_like(blocks), 1)
    with pytest.raises(ValueError, match="empty coarse"):
        prepare_geometry(nb, torch.tensor([[0, 1], [-1, -1], [2, -1]]), 1)
    with pytest.raises(ValueError, match="pool_size"):
        prepare_geometry(nb, blocks, 33)
    layout = build_layout((2, 2, 2))
    with pytest.raises(ValueError, match="permutation"):
        layout.repack(torch.zeros(8, dtype=torch.int64))
    layout.coords[0, 0] += 1
    with pytest.raises(RuntimeError, match="changed"):
        layout.pack(torch.zeros(1, 2, 2, 2, 1))


def test_reverse_adjacency_asymmetric():
    nb = torch.tensor([[-1, -1, -1], [1, 2, 0], [2, 0, -1], [0, 3, 1]])
    rev = reverse_adjacency(nb)
    assert rev.tolist() == [[1, 2, 3], [1, 3, -1], [1, 2, -1], [3, -1, -1]]
