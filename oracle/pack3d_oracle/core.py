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


def _rows_branches(qf, klr, vlr, sk, sv, nb, r, root):
    """(o_L, o_G) of query rows r: reference.py:20-30 on one chunk of rows.

    qf [B, H, N, d]; klr, vlr, sk, sv already repeated to the H query heads.
    Global: softmax over all summaries of q.sk/sqrt(d), times sv.  Local:
    softmax over the valid entries of the neighbour row, times v; an
    all-masked row gives 0.
    """
    qc = qf[:, :, r]
    og = ((qc @ sk.transpose(-1, -2)) / root).softmax(-1) @ sv
    idx = nb[r]
    ok = idx >= 0
    safe = idx.clamp_min(0)
    lk, lv = klr[:, :, safe], vlr[:, :, safe]          # [B, H, c, W, d]
    s = (qc[..., None, :] * lk).sum(-1) / root
    s = s.masked_fill(~ok, -torch.inf)
    s = torch.where(ok.any(-1)[None, None, :, None], s, torch.zeros_like(s))
    p = s.softmax(-1) * ok
    ol = (p[..., None] * lv).sum(-2)
    return ol, og


def _prepared(q, kl, vl, kg, vg, weight, bias, geometry, temperature, work):
    g, h = kl.shape[1], q.shape[1]
    rep = h // g
    qf, klf, vlf, kgf, vgf = (t.to(work) for t in (q, kl, vl, kg, vg))
    sk, sv = compress_summaries(kgf, vgf, weight, bias, geometry, temperature=temperature)
    return qf, klf.repeat_interleave(rep, 1), vlf.repeat_interleave(rep, 1), sk, sv, rep


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
    n, d = q.shape[2], q.shape[3]
    work = torch.float64 if q.dtype == torch.float64 else torch.float32
    qf, klr, vlr, sk, sv, rep = _prepared(q, kl, vl, kg, vg, weight, bias, geometry, temperature, work)
    sk, sv = sk.repeat_interleave(rep, 1), sv.repeat_interleave(rep, 1)
    nb = geometry.neighbors.long()
    if rows is None:
        rows = torch.arange(n)
    rows = torch.as_tensor(rows, dtype=torch.long)
    root = math.sqrt(d)
    ol_parts, og_parts = [], []
    for start in range(0, rows.numel(), chunk):
        ol, og = _rows_branches(qf, klr, vlr, sk, sv, nb, rows[start:start + chunk], root)
        ol_parts.append(ol)
        og_parts.append(og)
    ol = torch.cat(ol_parts, 2)
    og = torch.cat(og_parts, 2)
    gr = gate.to(work)[:, :, rows]
    y = (sl.to(work) * ol + gr[..., None] * sg.to(work) * og).to(q.dtype)
    return (y, ol, og) if return_branches else y


def pack3d_reference_grads(q, kl, vl, kg, vg, weight, bias, gate, sl, sg, geometry, dy, *,
                           temperature=1.0, chunk=2048):
    """The ten input gradients of ``pack3d_reference`` for the upstream
    gradient ``dy`` (the reference's autograd of reference.py:16-31), each in
    its input's dtype, evaluated so that no autograd graph spans more than
    one chunk of query rows.  The summaries are computed once.  Each chunk
    differentiates the same ``_rows_branches`` math on leaf copies of the
    rows it touches -- its queries and gates, the neighbours it gathers
    (remapped to a local table), the summaries -- and the leaves' gradients
    are added into full-size accumulators; the summaries' gradients then go
    through the pooling's graph once.  The same values as
    ``torch.autograd.grad`` of ``pack3d_reference`` (up to summation order),
    at the memory cost of one chunk, so it runs at 262,144 tokens.
    """
    validate_inputs(q, kl, vl, kg, vg, weight, bias, gate, sl, sg, geometry, temperature)
    n, d = q.shape[2], q.shape[3]
    work = torch.float64 if q.dtype == torch.float64 else torch.float32
    inputs = (q, kl, vl, kg, vg, weight, bias, gate, sl, sg)
    qf, klf, vlf, kgf, vgf, w, b, gt, slf, sgf = (t.detach().to(work) for t in inputs)
    pooled = [t.requires_grad_() for t in (kgf, vgf, w, b)]
    slf.requires_grad_()
    sgf.requires_grad_()
    dq, dkl, dvl, dgate = (torch.zeros_like(t) for t in (qf, klf, vlf, gt))
    nb = geometry.neighbors.long()
    root = math.sqrt(d)
    dyw = dy.detach().to(work)
    with torch.enable_grad():
        sk, sv = compress_summaries(*pooled, geometry, temperature=temperature)
        rep = q.shape[1] // kl.shape[1]
        sk_leaf, sv_leaf = sk.detach().requires_grad_(), sv.detach().requires_grad_()
        skr, svr = sk_leaf.repeat_interleave(rep, 1), sv_leaf.repeat_interleave(rep, 1)
        for start in range(0, n, chunk):
            r = torch.arange(start, min(n, start + chunk))
            idx = nb[r]
            ok = idx >= 0
            uniq, inv = torch.unique(idx.clamp_min(0), return_inverse=True)
            local_nb = torch.where(ok, inv, -1)
            qc = qf[:, :, r].requires_grad_()
            gc = gt[:, :, r].requires_grad_()
            kc = klf[:, :, uniq].requires_grad_()
            vc = vlf[:, :, uniq].requires_grad_()
            ol, og = _rows_branches(qc, kc.repeat_interleave(rep, 1), vc.repeat_interleave(rep, 1), skr, svr,
                                    local_nb, torch.arange(r.numel()), root)
            y = slf * ol + gc[..., None] * sgf * og
            # The summary repeat nodes are shared by every chunk's graph.
            torch.autograd.backward(y, dyw[:, :, r], retain_graph=start + chunk < n)
            dq[:, :, r] = qc.grad
            dgate[:, :, r] = gc.grad
            dkl.index_add_(2, uniq, kc.grad)
            dvl.index_add_(2, uniq, vc.grad)
        torch.autograd.backward([sk, sv], [sk_leaf.grad, sv_leaf.grad])
    grads = (dq, dkl, dvl, pooled[0].grad, pooled[1].grad, pooled[2].grad, pooled[3].grad, dgate, slf.grad,
             sgf.grad)
    return [g.to(t.dtype) for g, t in zip(grads, inputs)]
