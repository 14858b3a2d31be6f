"""CPU restatement of the reference PACK3D core (test infrastructure only).

Follows ``src/pack3d/reference.py:8-31`` and ``src/pack3d/_validation.py:4-37``
of amilworks/Pack3D.  Differences: no dense guards (reference.py:13-15); the
head_dim whitelist (``_validation.py:17``) is widened to any even head_dim;
queries are processed in chunks, and ``rows`` restricts the evaluation to a
subset of query rows (the summaries still pool every token).
"""
from __future__ import annotations

import math

import torch

from .compression import compress_summaries


def validate_inputs(q, kl, vl, kg, vg, weight, bias, gate, sl, sg, geometry, temperature):
    """The core contract (_validation.py:4-37), head_dim widened to any even value."""
    geometry.check_unmodified()
    if q.ndim != 4 or min(q.shape) < 1:
        raise ValueError("Q must have shape [batch, query_heads, tokens, head_dim]")
    b, h, n, d = q.shape
    if kl.ndim != 4 or kl.shape[0] != b or tuple(kl.shape[2:]) != (n, d):
        raise ValueError("local K has incompatible dimensions")
    if not 0 < kl.shape[1] <= h or h % kl.shape[1]:
        raise ValueError("query heads must be divisible by KV heads")
    if any(t.shape != kl.shape for t in (vl, kg, vg)):
        raise ValueError("all branch K/V tensors must have matching shapes")
    if any(t.dtype != q.dtype for t in (kl, vl, kg, vg)):
        raise ValueError("Q/K/V must have the same dtype")
    if d % 2:
        raise ValueError("head_dim must be even")
    if weight.shape != (d,) or bias.shape != (geometry.blocks.shape[1],):
        raise ValueError("pool scorer/slot bias shape mismatch")
    if gate.shape != (b, h, n) or sl.shape != (d,) or sg.shape != (d,):
        raise ValueError("gate or channelwise branch scale shape mismatch")
    if n != geometry.num_tokens:
        raise ValueError("geometry token count does not match Q")
    if any(not t.is_floating_point() for t in (q, kl, vl, kg, vg, weight, bias, gate, sl, sg)):
        raise ValueError("attention inputs must be floating point")
    if not math.isfinite(temperature) or temperature <= 0:
        raise ValueError("temperature must be finite and positive")


def pack3d_reference(q, kl, vl, kg, vg, weight, bias, gate, sl, sg, geometry, *,
                     temperature=1.0, rows=None, chunk=2048, return_branches=False):
    """``y = sl * o_L + gate * sg * o_G`` in fp32 (fp64 for fp64), cast to q.dtype.

    reference.py:16-31.  Global branch: softmax over all M summaries of
    q.sk/sqrt(d), times sv.  Local branch: softmax over the valid entries of
    the neighbour row of q.k/sqrt(d), times v; an all-masked row gives 0.
    Query head h reads KV head h // (H/G).

    ``rows`` (1-D LongTensor) evaluates only those query rows; the result is
    then [B, H, len(rows), d].  ``return_branches`` also returns (o_L, o_G)
    in the working precision.
    """
    validate_inputs(q, kl, vl, kg, vg, weight, bias, gate, sl, sg, geometry, temperature)
    b, h, n, d = q.shape
    g = kl.shape[1]
    rep = h // g
    work = torch.float64 if q.dtype == torch.float64 else torch.float32
    qf, klf, vlf, kgf, vgf = (t.to(work) for t in (q, kl, vl, kg, vg))
    sk, sv = compress_summaries(kgf, vgf, weight, bias, geometry, temperature=temperature)
    sk, sv = sk.repeat_interleave(rep, 1), sv.repeat_interleave(rep, 1)
    klr, vlr = klf.repeat_interleave(rep, 1), vlf.repeat_interleave(rep, 1)
    nb = geometry.neighbors.long()
    if rows is None:
        rows = torch.arange(n)
    rows = torch.as_tensor(rows, dtype=torch.long)
    root = math.sqrt(d)
    ol_parts, og_parts = [], []
    for start in range(0, rows.numel(), chunk):
        r = rows[start:start + chunk]
        qc = qf[:, :, r]
        og_parts.append(((qc @ sk.transpose(-1, -2)) / root).softmax(-1) @ sv)
        idx = nb[r]
        ok = idx >= 0
        safe = idx.clamp_min(0)
        lk, lv = klr[:, :, safe], vlr[:, :, safe]          # [B, H, c, W, d]
        s = (qc[..., None, :] * lk).sum(-1) / root
        s = s.masked_fill(~ok, -torch.inf)
        s = torch.where(ok.any(-1)[None, None, :, None], s, torch.zeros_like(s))
        p = s.softmax(-1) * ok
        ol_parts.append((p[..., None] * lv).sum(-2))
    ol = torch.cat(ol_parts, 2)
    og = torch.cat(og_parts, 2)
    gr = gate.to(work)[:, :, rows]
    y = (sl.to(work) * ol + gr[..., None] * sg.to(work) * og).to(q.dtype)
    return (y, ol, og) if return_branches else y
