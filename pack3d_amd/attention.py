"""The PACK3D attention layer with the MI355X HIP backend.

Same constructor, parameters (names, shapes, initialisation order) and
forward as ``PACK3DAttention`` of amilworks/Pack3D (``src/pack3d/attention.py``),
with ``backend="hip"``.  In the no-grad forward (fp16 / bf16) LayerNorm,
to_q, to_kv, the gate map and its softmax run as one kernel
(``p3d_project``); on layouts whose fine blocks are consecutive 64-token runs
with pool_size 1 (this package's ``build_layout``) that kernel also pools the
summaries from the kg / vg values it computes (``p3d_project_pool``), and kg /
vg never reach memory.  With autograd active in fp16 / bf16, and under
autocast, LayerNorm is ``linear.LayerNormTrain`` and the linear maps are
``linear.InputProjections`` (``p3d_project_linear``) and
``linear.OutputResidual`` / ``OutputResidualWide``, with weight gradients from
``p3d_weight_grad``; for fp32 models without autocast they are the torch
modules (LayerNorm on the HIP kernel when no gradient is needed).  The
rotation, pooling, local and global attention and their fusion run in
``libpack3d_hip.so``, and so does ``x + to_out(y)`` in the no-grad fp16 /
bf16 forward and under autocast over an fp32 input (``p3d_out_residual``;
otherwise one GEMM with the residual as its C operand).  The projections are
consumed as strided views, without copies.
"""
from __future__ import annotations

import math

import torch
from torch import nn

from . import _lib
from .core import SUPPORTED_HEAD_DIMS, ForwardPlan, _projection_views, _validate_inputs, pack3d_hip_projections
from .linear import (InputProjections, LayerNormTrain, OutputResidual, OutputResidualWide, compute_dtype,
                     layer_norm_train_supported, wide_residual_supported)
from .geometry import TokenLayout, blocks_consecutive
from .rope import axial_rope, balanced_pairs, packed_rope


def layer_norm(norm: nn.LayerNorm, x):
    """``norm(x)`` on the HIP LayerNorm kernel when no gradient is needed.

    With autograd active the differentiable torch op runs instead; shapes
    the kernel does not take (a channel count that is not a whole number of
    16-byte pieces, or above 512) do too.
    """
    dim = x.shape[-1]
    dtypes = _lib.DTYPES
    ep = 16 // x.element_size()
    usable = (x.is_cuda and x.dtype in dtypes and norm.weight is not None and norm.bias is not None
              and norm.weight.dtype == norm.bias.dtype and norm.weight.dtype in dtypes
              and dim % ep == 0 and dim <= 512 and len(norm.normalized_shape) == 1)
    if not usable or (torch.is_grad_enabled() and (x.requires_grad or norm.weight.requires_grad
                                                   or norm.bias.requires_grad)):
        return norm(x)
    xc = x.contiguous()
    y = torch.empty_like(xc)
    _lib.call("p3d_layer_norm", xc.data_ptr(), norm.weight.data_ptr(), norm.bias.data_ptr(),
              dtypes[norm.weight.dtype], y.data_ptr(), xc.numel() // dim, dim, dtypes[x.dtype], float(norm.eps),
              _lib.stream_of(x.device))
    return y


PROJECT_DIMS = (64, 96, 128, 192, 256, 384, 512)


def _project_buffers(layer, x):
    """(argument block, q [B,N,H*d], kv [B,N,4*G*d], gate [B,N,H]) for the
    fused projection kernels, or None when they do not apply (autograd
    active, fp32 or mixed dtypes, a model width the kernels do not take)."""
    norm, lin = layer.norm, (layer.to_q, layer.to_kv, layer.gate)
    dt = x.dtype
    params = [norm.weight, norm.bias, *(m.weight for m in lin), layer.gate.bias]
    if any(p is None for p in params):
        return None
    if torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in params)):
        return None
    if (not x.is_cuda or dt not in (torch.float16, torch.bfloat16) or layer.dim not in PROJECT_DIMS
            or tuple(norm.normalized_shape) != (layer.dim,) or any(m.weight.dtype != dt for m in lin)
            or any(not m.weight.is_contiguous() for m in lin) or norm.weight.dtype != norm.bias.dtype
            or norm.weight.dtype not in _lib.DTYPES or layer.gate.bias.dtype not in _lib.DTYPES):
        return None
    b, n = x.shape[0], x.shape[1]
    h, g, d = layer.heads, layer.kv_heads, layer.head_dim
    xc = x.contiguous()
    q = torch.empty(b, n, h * d, dtype=dt, device=x.device)
    kv = torch.empty(b, n, 4 * g * d, dtype=dt, device=x.device)
    gate = torch.empty(b, n, h, dtype=dt, device=x.device)
    args = _lib.ProjectArgs(xc.data_ptr(), norm.weight.data_ptr(), norm.bias.data_ptr(),
                            layer.to_q.weight.data_ptr(), layer.to_kv.weight.data_ptr(), layer.gate.weight.data_ptr(),
                            layer.gate.bias.data_ptr(), q.data_ptr(), kv.data_ptr(), gate.data_ptr(), b * n, layer.dim,
                            h * d, 4 * g * d, h, _lib.DTYPES[dt], _lib.DTYPES[norm.weight.dtype],
                            _lib.DTYPES[layer.gate.bias.dtype], float(norm.eps))
    args._keep = xc
    return args, q, kv, gate


def fused_projections(layer, x):
    """(q [B,N,H*d], kv [B,N,4*G*d], gate [B,N,H]) of the no-grad forward from
    one kernel (``p3d_project``): LayerNorm, to_q, to_kv, the gate map and its
    pair softmax.  None when it does not apply (autograd active, fp32 or mixed
    dtypes, a model width the kernel does not take); the caller then runs the
    separate ops, which compute the same values."""
    made = _project_buffers(layer, x)
    if made is None:
        return None
    args, q, kv, gate = made
    _lib.call("p3d_project", args, _lib.stream_of(x.device))
    return q, kv, gate


POOLED_HEAD_DIMS = (16, 32, 48, 64)
POOLED_DIMS = (64, 96, 128, 192, 256)


def pooled_core(layer, x, layout):
    """The core's output [B, H, N, d] (a transposed view of a [B, N, H, d]
    buffer) of the no-grad forward with the summary pooling fused into the
    projections (``p3d_project_pool``): q, kl, vl, the gate and the summaries
    come from one kernel, kg and vg are never written, kl is stored rotated
    (the attention kernels then rotate only q), and the attention kernels
    follow.  The same values as the projections, ``p3d_pool_fwd`` and the
    attention, up to the order of fp32 sums in the pooling.  None
    when it does not apply: autograd active, fp32, pool_size other than 1,
    fine blocks that are not the consecutive 64-token runs of
    ``build_layout``, or shapes the kernel does not take; the caller then runs
    the projections and the core separately."""
    geometry = layout.geometry
    h, g, d = layer.heads, layer.kv_heads, layer.head_dim
    pool_params = (layer.pool_weight, layer.slot_bias, layer.local_scale, layer.global_scale)
    if torch.is_grad_enabled() and any(p.requires_grad for p in pool_params):
        return None
    if (geometry.pool_size != 1 or d not in POOLED_HEAD_DIMS or g * d > 192 or layer.dim not in POOLED_DIMS
            or not x.is_cuda or x.dtype not in (torch.float16, torch.bfloat16) or x.shape[1] % 64):
        return None
    made = _project_buffers(layer, x)
    if made is None or not blocks_consecutive(geometry):
        return None
    args, qp, kvp, gp = made
    q, kl, vl, kg, vg = _projection_views(qp, kvp, h, g)
    inputs = (q, kl, vl, kg, vg, *pool_params[:2], gp.transpose(1, 2), *pool_params[2:])
    _validate_inputs(*inputs, geometry, layer.temperature)
    rope = layer._rope(x, layout)
    # kl is stored rotated by the projections, so the attention kernels do
    # not rotate every halo key again for each brick that reads it.
    rotate = not rope.identity
    plan = ForwardPlan(*inputs, geometry, layer.temperature, rope, rope, kl_rotated=rotate)
    m = geometry.num_summaries
    if m % 32:
        # Padding summaries up to the next multiple of 32: zero, as
        # p3d_pool_fwd writes them (the fused kernel writes real ones only).
        plan.sk[:, :, m:].zero_()
        plan.svt[:, :, -1, :, m % 32:].zero_()
    rc = _lib.lib().p3d_project_pool(args, plan.pool_args, int(rotate), _lib.stream_of(x.device))
    if rc == _lib.P3D_EUNSUPPORTED:
        return None
    if rc != 0:
        raise RuntimeError(f"p3d_project_pool failed ({rc}): {_lib.lib().p3d_last_error().decode()}")
    plan.attention()
    return plan.y


def fused_out_residual(layer, x, y):
    """x + to_out(y) of the no-grad forward from one kernel (``p3d_out_residual``)
    for y [B*N, H*d]; None when it does not apply (autograd active, fp32 or
    mixed dtypes, widths the kernel does not take)."""
    w = layer.to_out.weight
    if torch.is_grad_enabled() and (x.requires_grad or y.requires_grad or w.requires_grad):
        return None
    dt = x.dtype
    k = layer.heads * layer.head_dim
    if (not x.is_cuda or dt not in (torch.float16, torch.bfloat16) or w.dtype != dt or y.dtype != dt
            or k not in PROJECT_DIMS or layer.dim % 32 or layer.dim > 512 or not w.is_contiguous()
            or not y.is_contiguous()):
        return None
    xc = x.contiguous()
    out = torch.empty_like(xc)
    _lib.call("p3d_out_residual", y.data_ptr(), w.data_ptr(), xc.data_ptr(), out.data_ptr(), y.shape[0], k,
              layer.dim, _lib.DTYPES[dt], _lib.DTYPES[dt], _lib.stream_of(x.device))
    return out


class PACK3DAttention(nn.Module):
    """Local residual plus gated compressed attention and an outer residual (attention.py:10-21)."""

    def __init__(self, dim, *, heads=4, kv_heads=2, head_dim=32, block_volume=8,
                 backend="hip", position_encoding="axial", temperature=1.0):
        super().__init__()
        if any(type(v) is not int or v <= 0 for v in (dim, heads, kv_heads, head_dim, block_volume)):
            raise ValueError("dimensions must be positive integers")
        if heads % kv_heads or head_dim not in SUPPORTED_HEAD_DIMS or block_volume > 64:
            raise ValueError("unsupported grouped-head dimensions or block volume")
        if backend != "hip":
            raise ValueError("backend must be explicitly hip (this package has no other backend)")
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

    def core_inputs(self, x, layout: TokenLayout):
        """Unrotated q, kl, vl, kg, vg (views of the projections), gate, and the rotation."""
        b, n = x.shape[0], x.shape[1]
        qp, kvp, gate, _ = self._projections(x)
        q = qp.view(b, n, self.heads, self.head_dim).transpose(1, 2)
        kl, vl, kg, vg = (t.view(b, n, self.kv_heads, self.head_dim).transpose(1, 2)
                          for t in kvp.view(b, n, 4, self.kv_heads * self.head_dim).unbind(2))
        return q, kl, vl, kg, vg, gate, self._rope(x, layout)

    def _rope(self, x, layout):
        n = x.shape[1]
        if self.position_encoding == "packed":
            return packed_rope(self.head_dim, n, x.device)
        return axial_rope(self.head_dim, layout.grid_shape, layout.coords, balanced_pairs(self.head_dim))

    def _projections(self, x):
        """qp [B, N, H*d], kvp [B, N, 4*G*d] (kl | vl | kg | vg), the gate
        [B, H, N], and the residual operand of the output product when
        LayerNormTrain wrote it (x rounded to the compute type, [B*N, dim];
        else None)."""
        b, n = x.shape[0], x.shape[1]
        res = None
        fused = fused_projections(self, x)
        if fused is not None:
            qp, kvp, gp = fused
            gate = gp.transpose(1, 2)
        elif self._hip_linear(x):
            dt = compute_dtype(x)
            if layer_norm_train_supported(self.norm, x):
                if x.dtype == dt:  # the residual copy is the output product's accumulator
                    xn, res = LayerNormTrain.apply(x, self.norm.weight, self.norm.bias, self.norm.eps, dt, True)
                elif wide_residual_supported(x, self.heads * self.head_dim, self.dim, dt):
                    # x itself, for the output product's fp32 residual (one consumer of x)
                    xn, res = LayerNormTrain.apply(x, self.norm.weight, self.norm.bias, self.norm.eps, dt, "pass")
                else:
                    xn = LayerNormTrain.apply(x, self.norm.weight, self.norm.bias, self.norm.eps, dt)
            else:
                xn = layer_norm(self.norm, x)
            qp, kvp, gl = InputProjections.apply(xn, self.to_q.weight, self.to_kv.weight, self.gate.weight,
                                                 self.gate.bias, dt)
            gate = gl.view(b, n, self.heads, 2).softmax(-1)[..., 1].transpose(1, 2)
        else:
            xn = layer_norm(self.norm, x)
            qp, kvp, gl = self.to_q(xn), self.to_kv(xn), self.gate(xn)
            gate = gl.view(b, n, self.heads, 2).softmax(-1)[..., 1].transpose(1, 2)
        return qp, kvp, gate, res

    def forward(self, x, layout: TokenLayout):
        layout.check_unmodified()
        if x.ndim != 3 or x.shape[0] == 0 or tuple(x.shape[1:]) != (layout.geometry.num_tokens, self.dim):
            raise ValueError("x must be [batch,layout_tokens,dim] with a nonempty batch")
        if x.device != layout.coords.device:
            raise ValueError("x and layout are on different devices; move both with .to(device)")
        if layout.geometry.blocks.shape[1] != len(self.slot_bias):
            raise ValueError("layout canonical slot count must match block_volume")
        if self.backend != "hip":
            raise ValueError("unknown backend; implicit fallback is disabled")
        b, n = x.shape[0], x.shape[1]
        out, res = pooled_core(self, x, layout), None
        if out is None:
            qp, kvp, gate, res = self._projections(x)
            out = pack3d_hip_projections(qp, kvp, self.heads, self.kv_heads, self.pool_weight, self.slot_bias,
                                         gate, self.local_scale, self.global_scale, layout.geometry,
                                         self._rope(x, layout), temperature=self.temperature)
        # x + to_out(out): one kernel in the no-grad forward, else one GEMM with the
        # residual as its C operand (to_out has no bias), with a HIP weight gradient
        # in 16-bit training.
        o = out.transpose(1, 2).reshape(b * n, -1)
        fused = fused_out_residual(self, x, o)
        if fused is not None:
            return fused.view(b, n, self.dim)
        if self._hip_linear(x):
            dt = compute_dtype(x)
            if x.dtype != dt:
                # Autocast over a wider x: the residual keeps x's type and is
                # not rounded, as in the reference's sum (attention.py:89).
                if res is not None:  # x as LayerNormTrain passed it through (fp32)
                    return OutputResidualWide.apply(res, o, self.to_out.weight, dt).view(b, n, self.dim)
                return x + OutputResidual.apply(None, o, self.to_out.weight, dt).view(b, n, self.dim)
            if res is not None:  # LayerNormTrain's dt copy of x, owned by this step
                return OutputResidual.apply(res, o, self.to_out.weight, dt, True).view(b, n, self.dim)
            return OutputResidual.apply(x.reshape(b * n, self.dim), o, self.to_out.weight, dt).view(b, n, self.dim)
        if x.is_cuda and torch.is_autocast_enabled("cuda") and x.dtype != torch.get_autocast_dtype("cuda"):
            return x + self.to_out(o).view(b, n, self.dim)
        return torch.addmm(x.reshape(b * n, self.dim), o, self.to_out.weight.t()).view(b, n, self.dim)

    def _hip_linear(self, x):
        """Whether the linear maps run as InputProjections / OutputResidual
        (weight gradients from p3d_weight_grad) and LayerNorm as LayerNormTrain:
        autograd active, or autocast on (the no-grad forward under autocast,
        whose fp32 parameters or input the fused projection kernel does not
        take); a CUDA input and a 16-bit compute type, the gate with a bias,
        and no hooks or parametrisations on the linear modules that the
        functions would skip."""
        mods = (self.to_q, self.to_kv, self.gate, self.to_out)
        params = [m.weight for m in mods] + [self.gate.bias]
        grad = torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in params))
        return ((grad or torch.is_autocast_enabled("cuda")) and x.is_cuda and compute_dtype(x) is not None
                and self.gate.bias is not None and self.to_q.bias is None and self.to_kv.bias is None
                and self.to_out.bias is None
                and all(type(m) is nn.Linear and not m._forward_hooks and not m._forward_pre_hooks for m in mods))
