"""CPU restatement of the reference axial RoPE (test infrastructure only).

Follows ``src/pack3d/rope.py:7-48`` of amilworks/Pack3D.
"""
from __future__ import annotations

import math

import torch
from torch import Tensor


def balanced_pairs(head_dim):
    """Split head_dim/2 rotary pairs over (z, y, x), remainder to the first axes (rope.py:7-12)."""
    if type(head_dim) is not int or head_dim <= 0 or head_dim % 2:
        raise ValueError("head_dim must be a positive even integer")
    total = head_dim // 2
    return tuple(total // 3 + (1 if axis < total % 3 else 0) for axis in range(3))


def frequencies(count, dtype=torch.float32):
    """Per-axis frequencies base**(-j/count), j < count, computed in ``dtype`` (rope.py:42)."""
    return 10000.0 ** (-torch.arange(count, dtype=dtype) / count)


def axial_rope(tensor: Tensor, coords: Tensor, *, pairs=None, base=10000.0) -> Tensor:
    """Rotate channel pairs of [B, H, N, d] by their token's per-axis angle (rope.py:15-48).

    Axis a owns channels [off_a, off_a + 2 p_a); pair j of that axis is
    channels (off_a + 2j, off_a + 2j + 1) rotated by angle coord_a * f_j.
    Computation runs in fp32 (fp64 for fp64 input) and rounds back.
    """
    if tensor.ndim != 4 or not tensor.is_floating_point():
        raise ValueError("tensor must be floating [batch,heads,tokens,head_dim]")
    pairs = balanced_pairs(tensor.shape[-1]) if pairs is None else tuple(pairs)
    if (len(pairs) != 3 or any(type(p) is not int or p < 0 for p in pairs)
            or 2 * sum(pairs) != tensor.shape[-1]):
        raise ValueError("pairs must allocate every rotary pair across three axes")
    if coords.shape != (tensor.shape[2], 3) or coords.device != tensor.device:
        raise ValueError("coords must be [tokens,3] on the tensor device")
    if coords.is_complex() or (coords.is_floating_point() and not bool(torch.isfinite(coords).all())):
        raise ValueError("coordinates must be real and finite")
    if not math.isfinite(base) or base <= 1:
        raise ValueError("base must be finite and greater than one")
    work = torch.float64 if tensor.dtype == torch.float64 else torch.float32
    pos = coords.to(work)
    out, start = [], 0
    for axis, count in enumerate(pairs):
        if count == 0:
            continue
        seg = tensor[..., start:start + 2 * count].to(work)
        even, odd = seg[..., 0::2], seg[..., 1::2]
        freq = base ** (-torch.arange(count, dtype=work) / count)
        angle = pos[:, axis, None] * freq
        c, s = angle.cos(), angle.sin()
        rot = torch.stack((even * c - odd * s, even * s + odd * c), -1)
        out.append(rot.flatten(-2))
        start += 2 * count
    return torch.cat(out, -1).to(tensor.dtype)
