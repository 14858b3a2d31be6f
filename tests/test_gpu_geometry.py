"""Bit-exact parity of the HIP geometry kernels with the oracle (geometry.py restated)."""
import math

import pytest
import torch

import oracle.pack3d_oracle as ref
import pack3d_amd as p3d
from tests._cases import make_case

pytestmark = pytest.mark.gpu


def _same(layout, expected):
    cpu = layout.to("cpu")
    assert torch.equal(cpu.order, expected.order)
    assert torch.equal(cpu.coords, expected.coords)
    assert torch.equal(cpu.geometry.neighbors, expected.geometry.neighbors)
    assert torch.equal(cpu.geometry.blocks, expected.geometry.blocks)
    assert torch.equal(cpu.geometry.reverse_neighbors, expected.geometry.reverse_neighbors)
    m_got, m_exp = cpu.geometry._raster_to_packed, expected.geometry.raster_to_packed
    assert (m_got is None) == (m_exp is None)
    if m_got is not None:
        assert torch.equal(m_got, m_exp)


LAYOUTS = [
    ((16, 16, 16), (4, 4, 4), 2, "raster_block"),      # c0 geometry
    ((16, 16, 16), (4, 4, 4), 2, "native_block_morton"),
    ((16, 64, 64), (4, 4, 4), 2, "raster_block"),      # c1 geometry
    ((8, 32, 16), (4, 4, 4), 2, "native_block_morton"),
    ((4, 4, 8), (1, 2, 2), 1, "native_block_morton"),
    ((7, 11, 55), (1, 1, 5), 1, "raster_block"),
    ((6, 10, 12), (2, 5, 3), (0, 1, 2), "native_block_morton"),
    ((3, 3, 3), (1, 1, 1), 2, "native_block_morton"),
    ((2, 8, 6), (2, 4, 3), (3, 1, 1), "raster_block"),
]


@pytest.mark.parametrize("shape,block,radius,kind", LAYOUTS)
def test_build_layout_bit_exact(gpu, shape, block, radius, kind):
    print(f"build_layout {shape} {block} {radius} {kind}", flush=True)
    got = p3d.build_layout(shape, block, radius=radius, pool_size=1, layout=kind)
    _same(got, ref.build_layout(shape, block, radius=radius, pool_size=1, layout=kind))


@pytest.mark.parametrize("shape,kind", [((64, 64, 64), "raster_block"), ((32, 128, 64), "native_block_morton")])
def test_build_layout_bit_exact_full_size(gpu, shape, kind):
    print(f"build_layout full {shape} {kind}", flush=True)
    got = p3d.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout=kind)
    _same(got, ref.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout=kind))


def test_repack_bit_exact(gpu):
    print("repack", flush=True)
    shape = (8, 12, 16)
    gen = torch.Generator().manual_seed(3)
    lay = p3d.build_layout(shape, (4, 4, 4), radius=2, pool_size=1)
    exp = ref.build_layout(shape, (4, 4, 4), radius=2, pool_size=1)
    for _ in range(2):
        p = torch.randperm(math.prod(shape), generator=gen)
        lay, exp = lay.repack(p), exp.repack(p)
        _same(lay, exp)
    back = lay.repack(lay.order.argsort().cpu())
    exp = exp.repack(exp.order.argsort())
    _same(back, exp)
    assert back.geometry._raster_to_packed is None
    with pytest.raises(ValueError, match="permutation"):
        lay.repack(torch.zeros(math.prod(shape), dtype=torch.int64))


@pytest.mark.parametrize("n,volume,pool", [(37, 4, 3), (131, 16, 2), (2053, 8, 2), (1, 1, 1)])
def test_prepare_geometry_bit_exact(gpu, n, volume, pool):
    print(f"prepare_geometry {n}", flush=True)
    _, nb, blocks, _ = make_case(n=n, volume=volume, pool=pool)
    got = p3d.prepare_geometry(nb, blocks, pool).to("cpu")
    exp = ref.prepare_geometry(nb, blocks, pool)
    for a, b in zip(got.tensors, exp.tensors):
        assert torch.equal(a, b)
    # int64 inputs and device inputs give the same tables.
    got64 = p3d.prepare_geometry(nb.long().to(gpu), blocks.long(), pool).to("cpu")
    for a, b in zip(got64.tensors, exp.tensors):
        assert torch.equal(a, b)


def test_prepare_geometry_errors(gpu):
    print("prepare_geometry errors", flush=True)
    _, nb, blocks, pool = make_case()
    with pytest.raises(ValueError, match="partition"):
        p3d.prepare_geometry(nb, torch.zeros_like(blocks), 3)
    with pytest.raises(ValueError, match="out-of-range"):
        p3d.prepare_geometry(nb + 1000, blocks, 3)
    dup = nb.clone()
    dup[3, 1] = dup[3, 0]
    with pytest.raises(ValueError, match="duplicate"):
        p3d.prepare_geometry(dup, blocks, 3)
    empty = torch.cat((torch.full((3, blocks.shape[1]), -1, dtype=torch.int32), blocks))
    with pytest.raises(ValueError, match="empty coarse"):
        p3d.prepare_geometry(nb, empty, 3)
    geom = p3d.prepare_geometry(nb, blocks, pool)
    geom.blocks[0, 0] = 0
    with pytest.raises(RuntimeError, match="changed"):
        geom.check_unmodified()


def test_layout_validation_and_mutation(gpu):
    print("layout validation", flush=True)
    lay = p3d.build_layout((4, 4, 4), (2, 2, 2), radius=1, pool_size=2)
    same = p3d.TokenLayout(lay.grid_shape, lay.order, lay.coords, lay.geometry)
    assert torch.equal(same.order, lay.order)
    bad = lay.coords.clone()
    bad[0, 0] += 1
    with pytest.raises(ValueError, match="permutation|agree"):
        p3d.TokenLayout(lay.grid_shape, lay.order, bad, lay.geometry)
    grid = torch.randn(2, 4, 4, 4, 3, device=gpu)
    torch.testing.assert_close(lay.unpack(lay.pack(grid)), grid)
    lay.coords[0, 0] += 1
    with pytest.raises(RuntimeError, match="changed"):
        lay.pack(grid)
