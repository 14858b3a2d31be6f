"""The layer's linear maps under autograd in fp16 / bf16, with the weight
gradients from the HIP kernel ``p3d_weight_grad``.

For y = x W^T the weight gradient dW = dy^T x contracts over every token
(262,144 at 64^3) into a small matrix; the library GEMM runs it with a
handful of workgroups.  ``p3d_weight_grad`` splits the tokens over the whole
GPU and sums fp32 partials in a fixed order.  The three input projections
run as one kernel over the normalised tokens (``p3d_project_linear``), their
input gradient as one contraction (``p3d_input_grad``); the output
projection's products stay torch GEMMs.  These functions replace the to_q, to_kv,
gate (attention.py:64-67,85 of amilworks/Pack3D) and to_out + residual
(attention.py:89) steps of ``PACK3DAttention.forward`` when it runs in a
16-bit compute type with autograd active; weight gradients are accumulated
in fp32 (torch's autocast path rounds them to the compute type first).
"""
from __future__ import annotations

import torch

from . import _lib

# The kernel's workgroups own up to 256 output rows, up to 256 input columns
# and a range of rows of dy / x; splits are chosen for at most WORKGROUPS
# workgroups in all (one per compute unit: from 128 input columns on, one
# workgroup fills a compute unit's LDS, and a second round for a few
# workgroups would double the pass), with at least MIN_ROWS_PER_SPLIT rows
# each.  The fp32 partials ([splits, out, in]) stay below half of the bytes
# of dy and x at 64^3.
WG_ROWS = 256
WG_COLS = 256
WORKGROUPS = 256
MIN_ROWS_PER_SPLIT = 512


def splits_for(rows, out_features, in_features):
    blocks = -(-out_features // WG_ROWS) * max(1, in_features // WG_COLS)
    return max(1, min(max(1, WORKGROUPS // blocks), rows // MIN_ROWS_PER_SPLIT))


def compute_dtype(x):
    """The 16-bit type the layer's linear maps run in: the autocast type when
    autocast is on for x's device, else x's own type (None when that is not
    fp16 / bf16)."""
    if x.is_cuda and torch.is_autocast_enabled("cuda"):
        dt = torch.get_autocast_dtype("cuda")
    else:
        dt = x.dtype
    return dt if dt in (torch.float16, torch.bfloat16) else None


def weight_grad_supported(out_features, in_features):
    cols_ok = (in_features % 32 == 0 and 32 <= in_features <= 256) or (
        in_features % 256 == 0 and 256 < in_features <= 2048)
    return out_features >= 8 and out_features % 8 == 0 and cols_ok


INPUT_GRAD_DIMS = (64, 96, 128, 192, 256, 384, 512)


def input_grad(dys, ws):
    """dq Wq + dkv Wkv + dgl Wg for the three 16-bit gradients dys [rows, *]
    and the weights ws [*, dim] of the same type, as one contraction summed in
    fp32 (``p3d_input_grad``); None where the kernel does not take the shapes
    (the caller then runs the three products)."""
    if any(dy is None for dy in dys):
        return None
    dt, rows, dim = ws[0].dtype, dys[0].shape[0], ws[0].shape[1]
    outs = [w.shape[0] for w in ws]
    if (dt not in (torch.float16, torch.bfloat16) or dim not in INPUT_GRAD_DIMS or any(o % 8 for o in outs)
            or any(dy.dtype != dt or dy.shape != (rows, o) or dy.stride(1) != 1 or dy.stride(0) % 8
                   or dy.data_ptr() % 16 for dy, o in zip(dys, outs))):
        return None
    k = sum(outs)
    k_pad = -(-k // 64) * 64
    wt = torch.zeros(dim, k_pad, dtype=dt, device=ws[0].device)
    wt[:, :k] = torch.cat(ws, 0).t()
    dx = torch.empty(rows, dim, dtype=dt, device=ws[0].device)
    _lib.call("p3d_input_grad", dys[0].data_ptr(), dys[0].stride(0), outs[0], dys[1].data_ptr(), dys[1].stride(0),
              outs[1], dys[2].data_ptr(), dys[2].stride(0), outs[2], wt.data_ptr(), k_pad, dx.data_ptr(), rows, dim,
              _lib.DTYPES[dt], _lib.stream_of(dx.device))
    return dx


PROJECT_DIMS = (64, 96, 128, 192, 256, 384, 512)


def project_linear(x16, ws, bg):
    """(x Wq^T, x Wkv^T, x Wg^T + bg) for x16 [rows, dim] and the weights ws
    [*, dim] of one 16-bit type, from one pass over x16 (``p3d_project_linear``:
    each output summed in fp32 and rounded once, as the torch products); None
    where the kernel does not take the shapes (the caller then runs the three
    products)."""
    dt, (rows, dim) = x16.dtype, x16.shape
    q_out, kv_out, g_out = (w.shape[0] for w in ws)
    if (dt not in (torch.float16, torch.bfloat16) or dim not in PROJECT_DIMS or q_out % 16 or kv_out % 16
            or g_out % 2 or not x16.is_contiguous() or x16.data_ptr() % 16
            or any(w.dtype != dt or w.shape[1] != dim or not w.is_contiguous() or w.data_ptr() % 16 for w in ws)
            or bg.numel() != g_out):
        return None
    bg = bg.to(dt).contiguous()  # the bias in dt, as torch.addmm(bg.to(dt), ...) adds it
    q = torch.empty(rows, q_out, dtype=dt, device=x16.device)
    kv = torch.empty(rows, kv_out, dtype=dt, device=x16.device)
    gl = torch.empty(rows, g_out, dtype=dt, device=x16.device)
    args = _lib.ProjectArgs(x=x16.data_ptr(), ln_weight=None, ln_bias=None, wq=ws[0].data_ptr(),
                            wkv=ws[1].data_ptr(), wg=ws[2].data_ptr(), gate_bias=bg.data_ptr(), q=q.data_ptr(),
                            kv=kv.data_ptr(), gate=gl.data_ptr(), rows=rows, dim=dim, q_out=q_out, kv_out=kv_out,
                            heads=g_out // 2, dtype=_lib.DTYPES[dt], ln_dtype=_lib.DTYPES[dt],
                            gate_bias_dtype=_lib.DTYPES[bg.dtype], eps=0.0)
    _lib.call("p3d_project_linear", args, _lib.stream_of(x16.device))
    return q, kv, gl


def weight_grad(dy, x):
    """dW = dy^T x in fp32 for dy [rows, out], x [rows, in] of one 16-bit type
    (``p3d_weight_grad``; torch's product in fp32 where the kernel does not
    take the shape)."""
    rows, out_f = dy.shape
    in_f = x.shape[1]
    if not weight_grad_supported(out_f, in_f) or dy.dtype != x.dtype or dy.dtype not in (torch.float16,
                                                                                           torch.bfloat16):
        return torch.mm(dy.t().float(), x.float())
    dy = dy if dy.stride(1) == 1 and dy.stride(0) % 8 == 0 else dy.contiguous()
    x = x if x.stride(1) == 1 and x.stride(0) % 8 == 0 else x.contiguous()
    if dy.data_ptr() % 16 or x.data_ptr() % 16:
        dy, x = dy.clone(), x.clone()
    splits = splits_for(rows, out_f, in_f)
    dw = torch.empty(out_f, in_f, dtype=torch.float32, device=dy.device)
    work = torch.empty(splits, out_f, in_f, dtype=torch.float32, device=dy.device)
    _lib.call("p3d_weight_grad", dy.data_ptr(), dy.stride(0), x.data_ptr(), x.stride(0), dw.data_ptr(),
              work.data_ptr(), rows, out_f, in_f, splits, _lib.DTYPES[dy.dtype], _lib.stream_of(dy.device))
    return dw


def weight_grads3(dys, x):
    """dW of three linear maps sharing the input x: [dy0^T x; dy1^T x;
    dy2^T x] in fp32 from one pass over x (``p3d_weight_grad3``), as three
    tensors; None where the kernel does not take the shapes (the caller
    then takes them one at a time)."""
    rows, in_f = x.shape
    outs = [dy.shape[1] for dy in dys]
    dt = x.dtype
    if (dt not in (torch.float16, torch.bfloat16) or not all(weight_grad_supported(o, in_f) for o in outs)
            or x.stride(1) != 1 or x.stride(0) % 8 or x.data_ptr() % 16
            or any(dy.dtype != dt or dy.shape[0] != rows or dy.stride(1) != 1 or dy.stride(0) % 8
                   or dy.data_ptr() % 16 for dy in dys)):
        return None
    total = sum(outs)
    splits = splits_for(rows, total, in_f)
    dw = torch.empty(total, in_f, dtype=torch.float32, device=x.device)
    work = torch.empty(splits, total, in_f, dtype=torch.float32, device=x.device)
    _lib.call("p3d_weight_grad3", dys[0].data_ptr(), dys[0].stride(0), outs[0], dys[1].data_ptr(), dys[1].stride(0),
              outs[1], dys[2].data_ptr(), dys[2].stride(0), outs[2], x.data_ptr(), x.stride(0), dw.data_ptr(),
              work.data_ptr(), rows, in_f, splits, _lib.DTYPES[dt], _lib.stream_of(x.device))
    return torch.split(dw, outs, 0)


def _rows(t):
    return t.reshape(-1, t.shape[-1])


def layer_norm_train_supported(norm, x):
    """Whether LayerNormTrain takes this nn.LayerNorm and input."""
    dim = x.shape[-1]
    ep = 16 // x.element_size()
    return (x.dtype in _lib.DTYPES and norm.weight is not None and norm.bias is not None
            and norm.weight.dtype in _lib.DTYPES and norm.bias.dtype in _lib.DTYPES
            and norm.weight.dtype == norm.bias.dtype and tuple(norm.normalized_shape) == (dim,)
            and dim % ep == 0 and dim <= 512
            and not norm._forward_hooks and not norm._forward_pre_hooks)


class LayerNormTrain(torch.autograd.Function):
    """nn.LayerNorm of the layer input (attention.py:64) for 16-bit training,
    on ``p3d_layer_norm_train`` / ``p3d_layer_norm_bwd``: fp32 statistics, the
    output rounded straight to the compute type dt (the value the next
    linear maps would cast it to), and a backward that returns dx in x's
    dtype and the affine gradients summed in fp32.

    With residual=True the forward also returns x rounded to dt as a
    [rows, dim] tensor, written from the same read of x: the residual operand
    of the output product (OutputResidual with x_owned=True).  With
    residual="pass" it returns x itself as [rows, dim] (the unrounded residual
    of autocast over a wider x, for OutputResidualWide).  Either way the
    backward adds that output's gradient into dx inside the kernel, where
    autograd would otherwise sum the two gradients of x in a separate pass."""

    @staticmethod
    def forward(ctx, x, weight, bias, eps, dt, residual=False):
        x2 = _rows(x).contiguous()
        rows, dim = x2.shape
        dev = x.device
        y = torch.empty(rows, dim, dtype=dt, device=dev)
        xc = torch.empty(rows, dim, dtype=dt, device=dev) if residual else None
        mean = torch.empty(rows, dtype=torch.float32, device=dev)
        rstd = torch.empty(rows, dtype=torch.float32, device=dev)
        _lib.call("p3d_layer_norm_train", x2.data_ptr(), weight.data_ptr(), bias.data_ptr(), _lib.DTYPES[weight.dtype],
                  y.data_ptr(), 0 if xc is None else xc.data_ptr(), mean.data_ptr(), rstd.data_ptr(), rows, dim,
                  _lib.DTYPES[x2.dtype], _lib.DTYPES[dt], float(eps), _lib.stream_of(dev))
        ctx.save_for_backward(x2, weight, mean, rstd)
        ctx.meta = (x.shape, bias.dtype)
        ctx.set_materialize_grads(False)
        if residual == "pass":
            return y.view(x.shape), x2
        if residual:
            return y.view(x.shape), xc
        return y.view(x.shape)

    @staticmethod
    def backward(ctx, dy, dres=None):
        x2, weight, mean, rstd = ctx.saved_tensors
        shape, b_dt = ctx.meta
        rows, dim = x2.shape
        if dy is None:
            dy = torch.zeros(rows, dim, dtype=torch.float32, device=x2.device)
        dy2 = _rows(dy).contiguous()
        if dy2.dtype not in _lib.DTYPES:
            dy2 = dy2.float()
        dx = torch.empty_like(x2)
        dr = None if dres is None else _rows(dres).to(dx.dtype).contiguous()
        parts = max(1, min(1024, rows // 256))
        part = torch.empty(parts, 2, dim, dtype=torch.float32, device=x2.device)
        _lib.call("p3d_layer_norm_bwd", dy2.data_ptr(), 0 if dr is None else dr.data_ptr(), x2.data_ptr(),
                  weight.data_ptr(), _lib.DTYPES[weight.dtype], mean.data_ptr(), rstd.data_ptr(), dx.data_ptr(),
                  part.data_ptr(), rows, dim, _lib.DTYPES[dy2.dtype], _lib.DTYPES[x2.dtype], _lib.DTYPES[dx.dtype],
                  parts, _lib.stream_of(x2.device))
        sums = part.sum(0)
        return dx.view(shape), sums[0].to(weight.dtype), sums[1].to(b_dt), None, None, None


class InputProjections(torch.autograd.Function):
    """(x Wq^T, x Wkv^T, x Wg^T + bg) of the normalised tokens x in the 16-bit
    type dt (attention.py:64-67,85): x is rounded to dt once and shared by
    the three products; the backward returns dx in x's dtype (the three
    input gradients summed in fp32) and fp32 weight gradients cast to the
    parameters' dtypes."""

    @staticmethod
    def forward(ctx, x, wq, wkv, wg, bg, dt):
        x16 = _rows(x).to(dt).contiguous()
        ws = [w.to(dt) for w in (wq, wkv, wg)]
        made = project_linear(x16, ws, bg)
        if made is not None:
            q, kv, gl = made
        else:
            q = torch.mm(x16, ws[0].t())
            kv = torch.mm(x16, ws[1].t())
            gl = torch.addmm(bg.to(dt), x16, ws[2].t())
        ctx.save_for_backward(x16, *ws)
        ctx.meta = (x.shape, x.dtype, wq.dtype, wkv.dtype, wg.dtype, bg.dtype)
        lead = x.shape[:-1]
        return q.view(*lead, -1), kv.view(*lead, -1), gl.view(*lead, -1)

    @staticmethod
    def backward(ctx, dq, dkv, dgl):
        x16, wq, wkv, wg = ctx.saved_tensors
        shape, x_dt, wq_dt, wkv_dt, wg_dt, bg_dt = ctx.meta
        # dx = dq Wq + dkv Wkv + dgl Wg: for an fp32 x (autocast) the three
        # products are summed in fp32 as autograd would; for a 16-bit x the
        # GEMMs accumulate into one buffer of that type.
        wide = x_dt == torch.float32
        dys = [None if dy is None else _rows(dy).to(x16.dtype) for dy in (dq, dkv, dgl)]
        # One kernel for the three products where it takes the shapes (16-bit x).
        dx = None if wide else input_grad(dys, (wq, wkv, wg))
        fused = dx is not None
        if wide:
            dx = torch.zeros(x16.shape, dtype=torch.float32, device=x16.device)
        # The three weight gradients from one pass over x16 where the kernel takes them.
        dws = None if any(dy is None for dy in dys) else weight_grads3(dys, x16)
        grads = []
        for i, (dy, w, w_dt) in enumerate(zip(dys, (wq, wkv, wg), (wq_dt, wkv_dt, wg_dt))):
            if dy is None:
                grads.append(None)
                continue
            if wide:
                dx.add_(torch.mm(dy, w))
            elif dx is None:
                dx = torch.mm(dy, w)
            elif not fused:
                dx.addmm_(dy, w)  # in place: no copy of dx into a new result
            grads.append((weight_grad(dy, x16) if dws is None else dws[i]).to(w_dt))
        if dx is None:
            dx = torch.zeros(x16.shape, dtype=x16.dtype, device=x16.device)
        dbg = None if dgl is None else _rows(dgl).float().sum(0).to(bg_dt)
        return dx.view(shape).to(x_dt), grads[0], grads[1], grads[2], dbg, None


def wide_residual_supported(x, k, dim, dt):
    """Whether p3d_out_residual takes an fp32 residual x [.., dim] for the
    product of width k in the 16-bit type dt."""
    return (x.is_cuda and x.dtype == torch.float32 and dt in (torch.float16, torch.bfloat16)
            and k in (64, 96, 128, 192, 256, 384, 512) and dim % 32 == 0 and dim <= 512)


class OutputResidualWide(torch.autograd.Function):
    """x + y Wo^T under autocast over an fp32 input (attention.py:89): the
    product in the 16-bit type dt, rounded to dt, added to the unrounded fp32
    residual x [rows, dim], as the reference's ``residual + to_out(...)`` sums
    an fp32 tensor and a 16-bit one; y [rows, k].  One kernel
    (``p3d_out_residual`` with an fp32 residual) instead of the product, a
    16-bit intermediate and a torch add.  The backward gives dx = dout
    (fp32), dy = dout Wo and an fp32 weight gradient, as OutputResidual's."""

    @staticmethod
    def forward(ctx, x, y, wo, dt):
        y16 = y.to(dt).contiguous()
        wo16 = wo.to(dt).contiguous()
        x2 = x.contiguous()
        rows, dim = x2.shape
        out = torch.empty_like(x2)
        _lib.call("p3d_out_residual", y16.data_ptr(), wo16.data_ptr(), x2.data_ptr(), out.data_ptr(), rows,
                  y16.shape[1], dim, _lib.DTYPES[dt], _lib.DTYPES[torch.float32], _lib.stream_of(x2.device))
        ctx.save_for_backward(y16, wo16)
        ctx.meta = (y.dtype, wo.dtype)
        return out

    @staticmethod
    def backward(ctx, dout):
        y16, wo16 = ctx.saved_tensors
        y_dt, wo_dt = ctx.meta
        d16 = dout.to(y16.dtype)
        dy = torch.mm(d16, wo16).to(y_dt)
        return dout, dy, weight_grad(d16, y16).to(wo_dt), None


class OutputResidual(torch.autograd.Function):
    """x + y Wo^T in the 16-bit type dt (attention.py:89 with a 16-bit x):
    x [rows, dim], y [rows, k].  The product accumulates into the residual in
    place: into x itself when the caller owns it (x_owned: x is already a dt
    copy, such as the one LayerNormTrain returns; it is marked dirty and
    returned), else into a dt copy of x (addmm with a full matrix would copy
    it into a new result first).  With x None it returns the product y Wo^T
    alone, rounded to dt: the caller adds a residual of a wider type itself,
    as the reference's ``residual + to_out(...)`` does under autocast.  The
    backward gives dx = dout (in x's dtype), dy = dout Wo and an fp32 weight
    gradient."""

    @staticmethod
    def forward(ctx, x, y, wo, dt, x_owned=False):
        y16 = y.to(dt).contiguous()
        wo16 = wo.to(dt)
        if x is None:
            out = torch.mm(y16, wo16.t())
        elif x_owned and x.dtype == dt and x.dim() == 2 and x.is_contiguous():
            ctx.mark_dirty(x)
            out = x
            out.addmm_(y16, wo16.t())
        else:
            out = x.to(dt, copy=True)
            out.addmm_(y16, wo16.t())
        ctx.save_for_backward(y16, wo16)
        ctx.meta = (None if x is None else x.dtype, y.dtype, wo.dtype)
        return out

    @staticmethod
    def backward(ctx, dout):
        y16, wo16 = ctx.saved_tensors
        x_dt, y_dt, wo_dt = ctx.meta
        d16 = dout.to(y16.dtype)
        dy = torch.mm(d16, wo16).to(y_dt)
        dx = None if x_dt is None else dout.to(x_dt)
        return dx, dy, weight_grad(d16, y16).to(wo_dt), None, None
