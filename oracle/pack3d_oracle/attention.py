"""CPU restatement of the reference PACK3D layer (test infrastructure only).

Follows ``src/pack3d/attention.py:24-89`` of amilworks/Pack3D, with the
``reference`` backend only, head_dim widened to any multiple of 16 up to 128.
Parameter names, shapes and initialisation order match the reference so a
``state_dict`` moves unchanged between this layer and ``pack3d_amd``'s.
"""
from __future__ import annotations

import math

import torch
from torch import nn

from .core import pack3d_reference
from .rope import axial_rope, balanced_pairs


class PACK3DAttention(nn.Module):
    def __init__(self, dim, *, heads=4, kv_heads=2, head_dim=32, block_volume=8,
                 backend="reference", position_encoding="axial", temperature=1.0):
        super().__init__()
        if any(type(v) is not int or v <= 0 for v in (dim, heads, kv_heads, head_dim, block_volume)):
            raise ValueError("dimensions must be positive integers")
        if heads % kv_heads or head_dim % 16 or head_dim > 128 or block_volume > 64:
            raise ValueError("unsupported grouped-head dimensions or block volume")
        if backend != "reference":
            raise ValueError("the oracle layer implements only the reference backend")
        if position_encoding not in ("axial", "packed"):
            raise ValueError("position_encoding must be axial or packed")
        if not math.isfinite(temperature) or temperature <= 0:
            raise ValueError("temperature must be finite and positive")
        self.dim, self.heads, self.kv_heads, self.head_dim = dim, heads, kv_heads, head_dim
        self.backend, self.position_encoding = backend, position_encoding
        self.temperature = float(temperature)
        # Creation order fixes the RNG stream (attention.py:40-51).
        self.norm = nn.LayerNorm(dim)
        self.to_q = nn.Linear(dim, heads * head_dim, bias=False)
        self.to_kv = nn.Linear(dim, 4 * kv_heads * head_dim, bias=False)
        self.pool_weight = nn.Parameter(torch.empty(head_dim))
        nn.init.uniform_(self.pool_weight, -1 / math.sqrt(head_dim), 1 / math.sqrt(head_dim))
        self.slot_bias = nn.Parameter(torch.empty(block_volume))
        nn.init.normal_(self.slot_bias, std=0.02)
        self.gate = nn.Linear(dim, heads * 2)
        nn.init.zeros_(self.gate.bias)
        self.local_scale = nn.Parameter(torch.ones(head_dim))
        self.global_scale = nn.Parameter(torch.full((head_dim,), 0.25))
        self.to_out = nn.Linear(heads * head_dim, dim, bias=False)

    def project(self, x, layout):
        """LayerNorm, projections, RoPE and gate (attention.py:63-86).

        Returns the core inputs (q, kl, vl, kg, vg, gate) with q, kl, kg rotated.
        """
        b, n = x.shape[0], x.shape[1]
        xn = self.norm(x)
        q = self.to_q(xn).reshape(b, n, self.heads, self.head_dim).transpose(1, 2)
        kl, vl, kg, vg = (t.reshape(b, n, self.kv_heads, self.head_dim).transpose(1, 2)
                          for t in self.to_kv(xn).chunk(4, -1))
        if self.position_encoding == "packed":
            pairs = (self.head_dim // 2, 0, 0)
            seq = torch.arange(n, device=x.device)
            coords = torch.stack((seq, torch.zeros_like(seq), torch.zeros_like(seq)), -1)
        else:
            pairs = balanced_pairs(self.head_dim)
            coords = layout.coords
        q, kl, kg = (axial_rope(t, coords, pairs=pairs) for t in (q, kl, kg))
        gate = self.gate(xn).reshape(b, n, self.heads, 2).softmax(-1)[..., 1].transpose(1, 2)
        return q, kl, vl, kg, vg, gate

    def forward(self, x, layout, **core_kwargs):
        layout.check_unmodified()
        if x.ndim != 3 or x.shape[0] == 0 or tuple(x.shape[1:]) != (layout.geometry.num_tokens, self.dim):
            raise ValueError("x must be [batch,layout_tokens,dim] with a nonempty batch")
        if layout.geometry.blocks.shape[1] != len(self.slot_bias):
            raise ValueError("layout canonical slot count must match block_volume")
        b, n = x.shape[0], x.shape[1]
        q, kl, vl, kg, vg, gate = self.project(x, layout)
        out = pack3d_reference(q, kl, vl, kg, vg, self.pool_weight, self.slot_bias, gate,
                               self.local_scale, self.global_scale, layout.geometry,
                               temperature=self.temperature, **core_kwargs)
        rows = core_kwargs.get("rows")
        residual = x if rows is None else x[:, torch.as_tensor(rows, dtype=torch.long)]
        return residual + self.to_out(out.transpose(1, 2).reshape(b, residual.shape[1], -1))
