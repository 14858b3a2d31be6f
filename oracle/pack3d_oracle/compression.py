"""CPU restatement of the reference two-stage summary pooling (test infrastructure only).

Follows ``src/pack3d/compression.py:7-44`` of amilworks/Pack3D, without its
size guard (compression.py:26-27).
"""
from __future__ import annotations

import math

import torch


def compress_summaries(keys, values, weight, bias, geometry, *, temperature=1.0):
    """Pool rotated keys and plain values [B, G, N, d] -> [B, G, M, d].

    Fine stage (compression.py:28-38): for fine block f and slot s with
    member t = blocks[f, s] >= 0, logit = (k_t . w) / tau + bias_s; a softmax
    over the valid slots gives weights a applied to keys and values alike.
    Empty fine blocks get zero weight.  Coarse stage (compression.py:39-43):
    the sum of fine summaries in each group of ``pool_size`` consecutive fine
    blocks divided by the number of non-empty fine blocks in the group.
    Arithmetic runs in fp32 (fp64 for fp64 inputs).
    """
    geometry.check_unmodified()
    if keys.ndim != 4 or values.shape != keys.shape or keys.shape[2] != geometry.num_tokens:
        raise ValueError("keys/values must match [batch,kv_heads,tokens,head_dim]")
    if not keys.is_floating_point() or values.dtype != keys.dtype:
        raise ValueError("keys and values must have matching floating dtypes")
    if weight.shape != (keys.shape[-1],) or bias.shape != (geometry.blocks.shape[1],):
        raise ValueError("pool weight or canonical slot bias has the wrong shape")
    if not math.isfinite(temperature) or temperature <= 0:
        raise ValueError("temperature must be finite and positive")
    work = torch.float64 if keys.dtype == torch.float64 else torch.float32
    idx = geometry.blocks.long()
    ok = idx >= 0
    safe = idx.clamp_min(0)
    k = keys.to(work)[:, :, safe]          # [B, G, F, V, d]
    v = values.to(work)[:, :, safe]
    logit = (k * weight.to(work)).sum(-1) / temperature + bias.to(work)
    logit = logit.masked_fill(~ok, -torch.inf)
    nonempty = ok.any(-1)
    logit = torch.where(nonempty[None, None, :, None], logit, torch.zeros_like(logit))
    a = logit.softmax(-1) * ok
    fine_k = (a[..., None] * k).sum(-2)   # [B, G, F, d]
    fine_v = (a[..., None] * v).sum(-2)
    f, p = idx.shape[0], geometry.pool_size
    groups = math.ceil(f / p)
    pad = groups * p - f
    if pad:
        fine_k = torch.cat((fine_k, fine_k.new_zeros(*fine_k.shape[:2], pad, fine_k.shape[-1])), 2)
        fine_v = torch.cat((fine_v, fine_v.new_zeros(*fine_v.shape[:2], pad, fine_v.shape[-1])), 2)
        nonempty = torch.cat((nonempty, nonempty.new_zeros(pad)))
    count = nonempty.view(groups, p).sum(-1).to(work)
    shape = (*fine_k.shape[:2], groups, p, fine_k.shape[-1])
    sk = fine_k.reshape(shape).sum(3) / count[:, None]
    sv = fine_v.reshape(shape).sum(3) / count[:, None]
    return sk, sv
