"""Objects with exactly the attribute set of the reference's geometry and
layout classes, and the reference layer with the HIP branch that
INTEGRATION.md registers (not collected by pytest).

``RefGeometry`` carries the fields of ``Pack3DGeometry`` in
``src/pack3d/geometry.py:10-50`` of amilworks/Pack3D -- neighbors,
reverse_neighbors, blocks, pool_size, num_tokens, _radius_one_grid,
_raster_to_packed, _versions, with ``tensors``, ``num_summaries``, ``to``
and ``check_unmodified`` -- and no ``_grid``.  ``reference_layout`` tags a
layout the way the reference's ``build_layout`` does (geometry.py:262-265:
radius one, n >= 4096, Z >= 2, Y >= 2, X >= 4), from the oracle's tables.
"""
from __future__ import annotations

import math
from dataclasses import InitVar, dataclass, field

import torch
from torch import Tensor

from oracle.pack3d_oracle import PACK3DAttention as OracleLayer
from oracle.pack3d_oracle import balanced_pairs


@dataclass(frozen=True)
class RefGeometry:
    neighbors: Tensor
    reverse_neighbors: Tensor
    blocks: Tensor
    pool_size: int
    num_tokens: int
    _seal: InitVar[object] = None
    _radius_one_grid: tuple | None = field(default=None, kw_only=True, repr=False)
    _raster_to_packed: Tensor | None = field(default=None, kw_only=True, repr=False)
    _versions: tuple = field(init=False, repr=False)

    def __post_init__(self, _seal):
        object.__setattr__(self, "_versions", self._tensor_versions())

    def _tensor_versions(self):
        versions = tuple(t._version for t in self.tensors)
        return versions if self._raster_to_packed is None else (*versions, self._raster_to_packed._version)

    @property
    def tensors(self):
        return self.neighbors, self.reverse_neighbors, self.blocks

    @property
    def num_summaries(self):
        return math.ceil(self.blocks.shape[0] / self.pool_size)

    def to(self, device):
        m = self._raster_to_packed
        return RefGeometry(*(t.to(device) for t in self.tensors), self.pool_size, self.num_tokens,
                           _radius_one_grid=self._radius_one_grid,
                           _raster_to_packed=None if m is None else m.to(device))

    def check_unmodified(self):
        if self._tensor_versions() != self._versions:
            raise RuntimeError("Geometry changed after validation; prepare it again")


@dataclass(frozen=True)
class RefLayout:
    grid_shape: tuple
    order: Tensor
    coords: Tensor
    geometry: RefGeometry

    def check_unmodified(self):
        self.geometry.check_unmodified()

    def to(self, device):
        return RefLayout(self.grid_shape, self.order.to(device), self.coords.to(device), self.geometry.to(device))


def reference_layout(oracle_layout, device=None):
    """The oracle's layout as the reference would hold it: the same tables,
    tagged only where the reference's build_layout tags (and its repack keeps
    the tag)."""
    g = oracle_layout.geometry
    shape = tuple(oracle_layout.grid_shape)
    n = math.prod(shape)
    tagged = (g.grid is not None and tuple(g.grid[1]) == (1, 1, 1) and n >= 4096 and shape[0] >= 2
              and shape[1] >= 2 and shape[2] >= 4)
    geom = RefGeometry(g.neighbors.to(torch.int32), g.reverse_neighbors.to(torch.int32), g.blocks.to(torch.int32),
                       g.pool_size, g.num_tokens, _radius_one_grid=shape if tagged else None,
                       _raster_to_packed=g.raster_to_packed if tagged else None)
    layout = RefLayout(shape, oracle_layout.order.clone(), oracle_layout.coords.clone(), geom)
    return layout if device is None else layout.to(device)


# attention.py:29 of the reference, and the whitelist INTEGRATION.md's patch
# of that line gives the hip backend.
REFERENCE_HEAD_DIMS = (16, 32, 64, 128)
PATCHED_HEAD_DIMS = (16, 32, 48, 64, 128)


class ReferenceLayerWithHip(OracleLayer):
    """The reference layer's constructor guards (attention.py:27-36, with
    line 29 patched as INTEGRATION.md writes it unless ``patched`` is False)
    and forward (attention.py:53-89) with the third, explicit ``hip`` branch
    of INTEGRATION.md in place of its dispatch."""

    def __init__(self, dim, *, heads=4, kv_heads=2, head_dim=32, block_volume=8, backend="hip",
                 position_encoding="axial", temperature=1.0, patched=True):
        if any(type(v) is not int or v <= 0 for v in (dim, heads, kv_heads, head_dim, block_volume)):
            raise ValueError("dimensions must be positive integers")
        widths = PATCHED_HEAD_DIMS if patched and backend == "hip" else REFERENCE_HEAD_DIMS
        if heads % kv_heads or head_dim not in widths or block_volume > 64:
            raise ValueError("unsupported grouped-head dimensions or block volume")
        if backend not in (("reference", "triton", "hip") if patched else ("reference", "triton")):
            raise ValueError("backend must be explicitly reference, triton or hip")
        super().__init__(dim, heads=heads, kv_heads=kv_heads, head_dim=head_dim, block_volume=block_volume,
                         position_encoding=position_encoding, temperature=temperature)
        self.backend = backend

    def forward(self, x, layout):
        layout.check_unmodified()
        residual, b, n = x, x.shape[0], x.shape[1]
        x = self.norm(x)
        q = self.to_q(x).reshape(b, n, self.heads, self.head_dim).transpose(1, 2)
        kl, vl, kg, vg = (t.reshape(b, n, self.kv_heads, self.head_dim).transpose(1, 2)
                          for t in self.to_kv(x).chunk(4, -1))
        packed = self.position_encoding == "packed"
        pairs = (self.head_dim // 2, 0, 0) if packed else balanced_pairs(self.head_dim)
        coords = layout.coords
        if self.backend == "hip":
            # ---- the registered branch, as INTEGRATION.md writes it ----
            import functools
            from pack3d_amd import adopt_layout
            from pack3d_amd.core import pack3d_hip_rope
            from pack3d_amd.rope import axial_rope as hip_rope, packed_rope
            adopt_layout(layout)  # proves the brick-kernel tag once per geometry object
            rope = (packed_rope(self.head_dim, n, x.device) if packed
                    else hip_rope(self.head_dim, layout.grid_shape, coords, pairs))
            core = functools.partial(pack3d_hip_rope, rope=rope)  # q, kl, kg stay unrotated
        else:
            raise ValueError("only the hip branch is registered here")
        gates = self.gate(x).reshape(b, n, self.heads, 2).softmax(-1)
        gate = gates[..., 1].transpose(1, 2)
        out = core(q, kl, vl, kg, vg, self.pool_weight, self.slot_bias, gate,
                   self.local_scale, self.global_scale, layout.geometry, temperature=self.temperature)
        return residual + self.to_out(out.transpose(1, 2).reshape(b, n, -1))
