"""Host side of the fused axial RoPE: pair allocation and (cos, sin) tables.

The kernels rotate on load (``p3d_rope`` in ``include/pack3d_hip.h``).  The
tables are built here with the same fp32 arithmetic as ``rope.py:42-44`` of
amilworks/Pack3D (frequency ``base**(-j/p)``, angle ``position * frequency``)
and indexed by coordinate, so a token's rotation does not depend on where it
is stored.
"""
from __future__ import annotations

import threading
from collections import OrderedDict

import torch

from . import _lib


def balanced_pairs(head_dim):
    """Split head_dim/2 rotary pairs over (z, y, x), remainder first (rope.py:7-12)."""
    if type(head_dim) is not int or head_dim <= 0 or head_dim % 2:
        raise ValueError("head_dim must be a positive even integer")
    total = head_dim // 2
    return tuple(total // 3 + (1 if axis < total % 3 else 0) for axis in range(3))


class RopeSpec:
    """Device tables plus the coordinates a kernel needs to rotate on load."""

    def __init__(self, table, pairs, coords, packed):
        self.table, self.pairs, self.coords, self.packed = table, pairs, coords, int(packed)
        self.identity = False

    def struct(self):
        return _lib.Rope(self.table.data_ptr(), self.pairs.data_ptr(),
                         None if self.coords is None else self.coords.data_ptr(), self.packed,
                         self.table.shape[0])


_cache: "OrderedDict[tuple, tuple]" = OrderedDict()
_cache_lock = threading.Lock()


def _cached(key, make):
    with _cache_lock:
        hit = _cache.get(key)
        if hit is not None:
            _cache.move_to_end(key)
            return hit
    value = make()
    with _cache_lock:
        _cache[key] = value
        while len(_cache) > 32:
            _cache.popitem(last=False)
    return value


def _tables(pairs, extents, head_dim, device, base=10000.0):
    """(table, pair descriptors) for per-axis pair counts and axis extents.

    Entry (axis, coordinate, pair j) sits at descriptor base_j + stride *
    coordinate.  The stride is the axis' pair count rounded up to an odd
    number (pad entries hold the identity (1, 0)): lanes that read the same
    pair at consecutive coordinates, as a fine block of a raster row does,
    then hit distinct LDS banks.
    """
    parts, desc, offset = [], [], 0
    for axis, (count, extent) in enumerate(zip(pairs, extents)):
        if count == 0:
            continue
        stride = count | 1
        freq = base ** (-torch.arange(count, dtype=torch.float32) / count)
        angle = torch.arange(extent, dtype=torch.float32)[:, None] * freq
        cs = torch.stack((angle.cos(), angle.sin()), -1)
        if stride > count:
            pad = torch.tensor([1.0, 0.0]).expand(extent, stride - count, 2)
            cs = torch.cat((cs, pad), 1)
        parts.append(cs.reshape(-1, 2))
        desc.extend([offset + j, stride, axis] for j in range(count))
        offset += extent * stride
    assert len(desc) == head_dim // 2
    table = torch.cat(parts).contiguous().to(device)
    return table, torch.tensor(desc, dtype=torch.int32).to(device)


def identity_rope(head_dim, device) -> RopeSpec:
    """The exact identity: every pair reads entry 0 = (cos 0, sin 0) = (1, 0)."""
    def make():
        table = torch.tensor([[1.0, 0.0]], dtype=torch.float32, device=device)
        return table, torch.zeros(head_dim // 2, 3, dtype=torch.int32, device=device)
    table, desc = _cached(("identity", head_dim, str(device)), make)
    spec = RopeSpec(table, desc, None, packed=True)
    spec.identity = True
    return spec


def axial_rope(head_dim, grid_shape, coords, pairs=None) -> RopeSpec:
    """Rotation at (z, y, x) coordinates ``coords`` [N, 3] of a grid (rope.py:35-48)."""
    pairs = balanced_pairs(head_dim) if pairs is None else tuple(pairs)
    if len(pairs) != 3 or 2 * sum(pairs) != head_dim or any(p < 0 for p in pairs):
        raise ValueError("pairs must allocate every rotary pair across three axes")
    device = coords.device
    key = ("axial", head_dim, tuple(pairs), tuple(grid_shape), str(device))
    table, desc = _cached(key, lambda: _tables(pairs, grid_shape, head_dim, device))
    return RopeSpec(table, desc, coords, packed=False)


def packed_rope(head_dim, tokens, device) -> RopeSpec:
    """The packed-position control: pairs (d/2, 0, 0) at positions (row, 0, 0)."""
    pairs = (head_dim // 2, 0, 0)
    key = ("packed", head_dim, tokens, str(device))
    table, desc = _cached(key, lambda: _tables(pairs, (tokens, 1, 1), head_dim, device))
    return RopeSpec(table, desc, None, packed=True)
