"""CPU restatement of the reference geometry (test infrastructure only).

Follows ``src/pack3d/geometry.py`` of amilworks/Pack3D:

* ``prepare_geometry``  -- geometry.py:53-101
* ``grid_coordinates``  -- geometry.py:112-115
* ``morton_codes``      -- geometry.py:118-126
* ``TokenLayout``       -- geometry.py:129-220
* ``build_layout``      -- geometry.py:223-266

The tensors produced here are the bit-exact targets of the HIP geometry
kernels in ``pack3d_amd``.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from itertools import product

import torch
from torch import Tensor

_SEAL = object()


def _versions_of(tensors):
    return tuple(t._version for t in tensors if t is not None)


@dataclass(frozen=True)
class Pack3DGeometry:
    """Validated neighbour table, reverse adjacency and fine-block membership.

    Mirrors ``Pack3DGeometry`` (geometry.py:10-50).  ``grid`` records the
    complete coordinate stencil a layout was built from (shape and per-axis
    radius); ``raster_to_packed`` maps a raster index to its packed row
    (``None`` means the identity).
    """

    neighbors: Tensor
    reverse_neighbors: Tensor
    blocks: Tensor
    pool_size: int
    num_tokens: int
    grid: tuple | None = None
    raster_to_packed: Tensor | None = None
    _seal: object = field(default=None, repr=False)
    _versions: tuple = field(default=(), repr=False)

    def __post_init__(self):
        if self._seal is not _SEAL:
            raise ValueError("Use prepare_geometry() to validate indices before launching kernels")
        object.__setattr__(self, "_versions", _versions_of(self._all()))

    def _all(self):
        return (self.neighbors, self.reverse_neighbors, self.blocks, self.raster_to_packed)

    @property
    def tensors(self):
        return self.neighbors, self.reverse_neighbors, self.blocks

    @property
    def num_summaries(self):
        return math.ceil(self.blocks.shape[0] / self.pool_size)

    def check_unmodified(self):
        if _versions_of(self._all()) != self._versions:
            raise RuntimeError("Geometry changed after validation; prepare it again")

    def with_grid(self, grid, raster_to_packed):
        return Pack3DGeometry(self.neighbors, self.reverse_neighbors, self.blocks, self.pool_size,
                              self.num_tokens, grid, raster_to_packed, _seal=_SEAL)


def reverse_adjacency(nb: Tensor) -> Tensor:
    """Row j lists, ascending, the rows i whose neighbour list contains j.

    geometry.py:88-99: a stable argsort of the destinations of all valid
    edges taken in row-major order, then a scatter into -1 padded rows of
    width max(1, max in-degree).
    """
    n, width = nb.shape
    source = torch.arange(n).repeat_interleave(width).view(n, width)
    valid = nb >= 0
    src, dst = source[valid], nb[valid]
    perm = torch.sort(dst, stable=True).indices
    src, dst = src[perm], dst[perm]
    degree = torch.bincount(dst, minlength=n)
    rwidth = max(1, int(degree.max())) if degree.numel() else 1
    if rwidth > 128:
        raise ValueError("reverse local degree exceeds 128")
    start = torch.cumsum(degree, 0) - degree
    slot = torch.arange(dst.numel()) - start[dst]
    out = torch.full((n, rwidth), -1, dtype=torch.int32)
    out[dst, slot] = src.to(torch.int32)
    return out


def prepare_geometry(neighbors: Tensor, blocks: Tensor, pool_size: int) -> Pack3DGeometry:
    """Validate a local graph and a fine-block partition (geometry.py:53-101)."""
    for name, t in (("neighbors", neighbors), ("blocks", blocks)):
        if t.ndim != 2 or t.dtype not in (torch.int32, torch.int64):
            raise ValueError(f"{name} must be a rank-two integer tensor")
        if min(t.shape) == 0:
            raise ValueError(f"{name} must be nonempty")
    if type(pool_size) is not int or not 1 <= pool_size <= 32:
        raise ValueError("pool_size must be an integer in [1,32]")
    nb = neighbors.detach().to("cpu", torch.int64).contiguous().clone()
    members = blocks.detach().to("cpu", torch.int64).contiguous().clone()
    n = nb.shape[0]
    if nb.shape[1] > 128 or members.shape[1] > 64:
        raise ValueError("at most 128 neighbors and 64 fine-block slots are supported")
    if max(nb.numel(), members.numel()) >= 2 ** 31:
        raise ValueError("geometry exceeds the 32-bit kernel indexing limit")
    for name, t in (("neighbors", nb), ("blocks", members)):
        if bool(((t < -1) | (t >= n)).any()):
            raise ValueError(f"{name} contains an out-of-range token")
    ordered = nb.sort(dim=1).values
    if bool(((ordered[:, 1:] == ordered[:, :-1]) & (ordered[:, 1:] >= 0)).any()):
        raise ValueError("duplicate local edges are not supported")
    hits = torch.bincount(members[members >= 0], minlength=n)
    if hits.numel() != n or not bool((hits == 1).all()):
        raise ValueError("fine blocks must partition every token exactly once")
    fine_valid = (members >= 0).any(dim=1)
    groups = math.ceil(len(members) / pool_size)
    padded = torch.zeros(groups * pool_size, dtype=torch.bool)
    padded[: len(members)] = fine_valid
    if not bool(padded.view(groups, pool_size).any(dim=1).all()):
        raise ValueError("an entirely empty coarse group is unsupported")
    rev = reverse_adjacency(nb)
    return Pack3DGeometry(nb.to(torch.int32), rev, members.to(torch.int32), pool_size, n, _seal=_SEAL)


def triple(value, name, *, allow_zero=False):
    """geometry.py:104-109."""
    values = (value,) * 3 if type(value) is int else tuple(value)
    low = 0 if allow_zero else 1
    if len(values) != 3 or any(type(v) is not int or v < low for v in values):
        raise ValueError(f"{name} must contain three integers >= {low}")
    return values


def grid_coordinates(shape) -> Tensor:
    """Raster-order (z, y, x) int64 coordinates [Z*Y*X, 3] (geometry.py:112-115)."""
    z, y, x = triple(shape, "shape")
    zz, yy, xx = torch.meshgrid(torch.arange(z), torch.arange(y), torch.arange(x), indexing="ij")
    return torch.stack((zz, yy, xx), -1).reshape(-1, 3)


def morton_codes(coords: Tensor) -> Tensor:
    """Interleave coordinate bits: bit b of axis a goes to bit 3b+a (geometry.py:118-126).

    The number of interleaved bits is the bit length of the largest coordinate
    over all axes; more than 20 bits is rejected.
    """
    nbits = int(coords.max()).bit_length()
    if nbits > 20:
        raise ValueError("Morton coordinates exceed the supported int64 range")
    code = torch.zeros(coords.shape[0], dtype=torch.int64)
    for b in range(nbits):
        for axis in range(3):
            code |= ((coords[:, axis] >> b) & 1) << (3 * b + axis)
    return code


@dataclass(frozen=True)
class TokenLayout:
    """Packed token order, coordinates and geometry (geometry.py:129-220)."""

    grid_shape: tuple
    order: Tensor
    coords: Tensor
    geometry: Pack3DGeometry
    _versions: tuple = field(default=(), repr=False)

    def __post_init__(self):
        shape = triple(self.grid_shape, "grid_shape")
        n = math.prod(shape)
        if self.order.shape != (n,) or self.order.dtype != torch.int64:
            raise ValueError("order must be an int64 permutation of the grid")
        if self.coords.shape != (n, 3) or self.coords.dtype != torch.int64:
            raise ValueError("coords must be int64 [tokens, 3]")
        if not torch.equal(self.order.sort().values, torch.arange(n)):
            raise ValueError("order must be a permutation")
        if not torch.equal(self.coords, grid_coordinates(shape)[self.order]):
            raise ValueError("coordinates do not agree with order")
        if n != self.geometry.num_tokens:
            raise ValueError("layout and geometry must agree on token count and device")
        object.__setattr__(self, "_versions", (self.order._version, self.coords._version))

    def check_unmodified(self):
        self.geometry.check_unmodified()
        if self._versions != (self.order._version, self.coords._version):
            raise RuntimeError("layout changed in place; construct a new layout")

    def pack(self, grid: Tensor) -> Tensor:
        """[batch, Z, Y, X, C] -> [batch, tokens, C] (geometry.py:174-179)."""
        self.check_unmodified()
        if grid.ndim != 5 or tuple(grid.shape[1:4]) != tuple(self.grid_shape):
            raise ValueError("input must match [batch,Z,Y,X,channels]")
        return grid.flatten(1, 3).index_select(1, self.order)

    def unpack(self, packed: Tensor) -> Tensor:
        """Inverse of ``pack`` (geometry.py:181-187)."""
        self.check_unmodified()
        if packed.ndim != 3 or packed.shape[1] != self.geometry.num_tokens:
            raise ValueError("packed input must have shape [batch,tokens,channels]")
        flat = packed.index_select(1, self.order.argsort())
        return flat.reshape(packed.shape[0], *self.grid_shape, packed.shape[-1])

    def repack(self, permutation) -> "TokenLayout":
        """New row i is old row permutation[i]; the graph is transported (geometry.py:189-220)."""
        self.check_unmodified()
        n = self.geometry.num_tokens
        p = torch.as_tensor(permutation).detach().cpu()
        if p.dtype not in (torch.int32, torch.int64) or p.shape != (n,):
            raise ValueError("permutation must be an integer vector with one entry per token")
        p = p.long()
        if not torch.equal(p.sort().values, torch.arange(n)):
            raise ValueError("permutation must contain every token exactly once")
        inv = p.argsort()
        nb = self.geometry.neighbors.long()[p]
        nb = torch.where(nb >= 0, inv[nb.clamp_min(0)], -1)
        blk = self.geometry.blocks.long()
        blk = torch.where(blk >= 0, inv[blk.clamp_min(0)], -1)
        geom = prepare_geometry(nb, blk, self.geometry.pool_size)
        if self.geometry.grid is not None:
            old = self.geometry.raster_to_packed
            mapping = inv if old is None else inv[old.long()]
            identity = torch.equal(mapping, torch.arange(n))
            geom = geom.with_grid(self.geometry.grid, None if identity else mapping.to(torch.int32))
        return TokenLayout(self.grid_shape, self.order[p].clone(), self.coords[p].clone(), geom)


def neighbor_offsets(radius):
    """Offsets in ``itertools.product`` order: z slowest, x fastest (geometry.py:254)."""
    return list(product(*(range(-r, r + 1) for r in radius)))


def build_layout(grid_shape, block_shape=(2, 2, 2), *, radius=1, pool_size=4,
                 layout="native_block_morton") -> TokenLayout:
    """Complete grid layout with a coordinate stencil (geometry.py:223-266).

    Unlike the reference, every layout records its grid and radius (the
    reference tags only radius-one grids, geometry.py:262-265); the tag is
    what the HIP brick kernels need, and it does not change any tensor.
    """
    shape = triple(grid_shape, "grid_shape")
    block = triple(block_shape, "block_shape")
    rad = triple(radius, "radius", allow_zero=True)
    if any(s % b for s, b in zip(shape, block)):
        raise ValueError("build_layout requires an unpadded grid divisible by block_shape")
    if math.prod(block) > 64 or math.prod(2 * r + 1 for r in rad) > 128:
        raise ValueError("layout exceeds supported block or neighborhood width")
    raster = grid_coordinates(shape)
    n = raster.shape[0]
    if layout == "native_block_morton":
        bshape = torch.tensor(block)
        slot_code = morton_codes(raster % bshape)
        key = morton_codes(raster // bshape) * (int(slot_code.max()) + 1) + slot_code
        order = key.argsort()
    elif layout == "raster_block":
        order = torch.arange(n)
    else:
        raise ValueError("layout must be raster_block or native_block_morton")
    coords = raster[order]
    inv = order.argsort()
    extent = torch.tensor(shape)
    stride = torch.tensor([shape[1] * shape[2], shape[2], 1])
    columns = []
    for off in neighbor_offsets(rad):
        target = coords + torch.tensor(off)
        inside = ((target >= 0) & (target < extent)).all(-1)
        flat = (target * stride).sum(-1).clamp(0, n - 1)
        columns.append(torch.where(inside, inv[flat], -1))
    members = torch.arange(n).reshape(-1, math.prod(block))
    geom = prepare_geometry(torch.stack(columns, 1), members, pool_size)
    mapping = None if layout == "raster_block" else inv.to(torch.int32)
    geom = geom.with_grid((shape, rad), mapping)
    return TokenLayout(shape, order, coords, geom)
