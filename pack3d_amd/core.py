"""The PACK3D core on MI355X: validation, dispatch to the HIP kernels, autograd.

``pack3d_hip`` has the core contract of ``pack3d_reference`` /
``pack3d_streamed`` of amilworks/Pack3D (``src/pack3d/reference.py:8-9``,
``src/pack3d/backends/triton/autograd.py:40-64``): rotated q, kl, kg.
``pack3d_hip_rope`` takes the unrotated projections and fuses the axial
rotation into the kernels' loads; the layer uses it.

There is no fallback: inputs that the HIP kernels cannot take raise.
"""
from __future__ import annotations

import math

import torch
from torch.autograd.function import once_differentiable

from . import _lib
from .geometry import grid_tag
from .rope import RopeSpec, identity_rope

SUPPORTED_HEAD_DIMS = (16, 32, 48, 64, 128)


def _validate_inputs(q, kl, vl, kg, vg, weight, bias, gate, sl, sg, geometry, temperature):
    """The core contract (``_validation.py:4-37``); head_dim 48 is also accepted."""
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
    if d not in SUPPORTED_HEAD_DIMS:
        raise ValueError("supported head dimensions are 16, 32, 48, 64 and 128")
    if q.numel() >= 2 ** 31 or b * kl.shape[1] * 32 * geometry.num_summaries * d >= 2 ** 31:
        raise ValueError("shape exceeds the 32-bit kernel indexing limit")
    if weight.shape != (d,) or bias.shape != (geometry.blocks.shape[1],):
        raise ValueError("pool scorer/slot bias shape mismatch")
    if gate.shape != (b, h, n) or sl.shape != (d,) or sg.shape != (d,):
        raise ValueError("gate or channelwise branch scale shape mismatch")
    if n != geometry.num_tokens:
        raise ValueError("geometry token count does not match Q")
    if any(t.dtype != torch.int32 or not t.is_contiguous() for t in geometry.tensors):
        raise ValueError("prepared geometry tables must be contiguous int32; use prepare_geometry()")
    every = (q, kl, vl, kg, vg, weight, bias, gate, sl, sg, *geometry.tensors)
    if any(t.device != q.device for t in every):
        raise ValueError("all tensors and prepared geometry must be on the same device")
    if any(not t.is_floating_point() for t in every[:10]):
        raise ValueError("attention inputs must be floating point")
    if not math.isfinite(temperature) or temperature <= 0:
        raise ValueError("temperature must be finite and positive")


def _check_hip(q):
    """No implicit fallback (autograd.py:31-37 of the reference)."""
    if q.device.type != "cuda" or q.dtype not in _lib.DTYPES:
        raise ValueError("hip backend requires HIP-device fp32/fp16/bf16 Q/K/V")


def _rows_ok(t):
    """Unit channel stride and 16-byte aligned rows, as the kernels require."""
    step = 16 // t.element_size()
    s = t.stride()
    return s[-1] == 1 and t.data_ptr() % 16 == 0 and all(x % step == 0 for x in s[:-1])


def _kernel_view(t):
    return t if _rows_ok(t) else t.contiguous()


def brick_tag(geometry):
    """The grid tag (shape, radius, raster_to_packed) when the brick kernels
    apply: a neighbour table known to be a complete grid stencil of radius
    at most 2 per axis (``geometry.grid_tag``); else None."""
    tag = grid_tag(geometry)
    if tag is None or any(r > 2 for r in tag[1]):
        return None
    return tag


def param_f32(t):
    """Contiguous fp32 copy of a small parameter vector (pooling weight, slot
    bias, branch scales) for the kernels.  The copy is kept on the tensor and
    reused while its storage and version counter are unchanged, so an
    inference loop does not launch a conversion per call."""
    if t.dtype == torch.float32 and t.is_contiguous():
        return t.detach()
    key = (t.data_ptr(), t._version, t.device)
    hit = getattr(t, "_p3d_f32", None)
    if hit is not None and hit[0] == key:
        return hit[1]
    v = t.detach().float().contiguous()
    try:
        t._p3d_f32 = (key, v)
    except (AttributeError, RuntimeError):
        pass
    return v


class ForwardPlan:
    """Buffers and ctypes argument blocks of one forward; ``run()`` launches it.

    Splitting construction from launch lets callers time or replay the
    pooling and attention kernels individually.  ``kl_rotated``: kl already
    holds the rotated keys (``p3d_project_pool`` with rotate_kl).  Otherwise
    kl is rotated once into a copy before the attention kernel (``klr``, which
    the backward reuses): the brick kernel would rotate each halo key again
    for every brick and query head that reads it, and the indexed kernel
    gathers it per edge.
    """

    def __init__(self, q, kl, vl, kg, vg, weight, bias, gate, sl, sg, geometry, temperature,
                 rope: RopeSpec, pool_rope: RopeSpec, save_state=False, kl_rotated=False):
        b, h, n, d = q.shape
        g = kl.shape[1]
        dev = q.device
        dt = _lib.DTYPES[q.dtype]
        self.device = dev
        q, kl, vl, kg, vg = (_kernel_view(t) for t in (q, kl, vl, kg, vg))
        f, slots = geometry.blocks.shape
        m = geometry.num_summaries
        mp = -(-m // 32) * 32
        self.sk = torch.empty(b, g, mp, d, dtype=q.dtype, device=dev)
        self.svt = torch.empty(b, g, mp // 32, d, 32, dtype=q.dtype, device=dev)
        # Allocated zeroed, so the first pooling launch needs no clear of its own.
        self.sk_norm_max = torch.zeros(b * g * 64, dtype=torch.float32, device=dev)
        self._keep = [q, kl, vl, kg, vg, geometry, rope, pool_rope]
        w32 = param_f32(weight)
        b32 = param_f32(bias)
        # The attention kernels score against summaries stored pre-multiplied
        # by log2(e)/sqrt(d), so a score is already in the exp2 domain.
        self.key_scale = math.log2(math.e) / math.sqrt(d)
        self.pool_args = _lib.PoolArgs(b, g, n, d, dt, f, slots, geometry.pool_size, m, float(temperature),
                                       self.key_scale, _lib.view(kg), _lib.view(vg), geometry.blocks.data_ptr(),
                                       w32.data_ptr(), b32.data_ptr(), pool_rope.struct(),
                                       self.sk.data_ptr(), self.svt.data_ptr(), self.sk_norm_max.data_ptr(), 1)
        self.y = torch.empty(b, n, h, d, dtype=q.dtype, device=dev).transpose(1, 2)
        sl32, sg32 = param_f32(sl), param_f32(sg)
        if gate.dtype not in _lib.DTYPES:
            gate = gate.float()
        self._keep += [w32, b32, sl32, sg32, gate]
        self.saved = {}
        if save_state:
            self.saved = {"lse_local": torch.empty(b, h, n, dtype=torch.float32, device=dev),
                          "lse_global": torch.empty(b, h, n, dtype=torch.float32, device=dev),
                          "o_local": torch.empty(b, h, n, d, dtype=q.dtype, device=dev),
                          "o_global": torch.empty(b, h, n, d, dtype=q.dtype, device=dev)}
        a = _lib.AttnArgs()
        a.batch, a.heads, a.kv_heads, a.tokens, a.head_dim, a.dtype = b, h, g, n, d, dt
        a.summaries, a.gate_dtype = m, _lib.DTYPES[gate.dtype]
        a.gate = _lib.view3(gate)
        a.local_scale, a.global_scale = sl32.data_ptr(), sg32.data_ptr()
        a.sk, a.svt = self.sk.data_ptr(), self.svt.data_ptr()
        a.sk_norm_max = self.sk_norm_max.data_ptr()
        a.y = _lib.view(self.y)
        a.lse_local = _lib.ptr(self.saved.get("lse_local"))
        a.lse_global = _lib.ptr(self.saved.get("lse_global"))
        a.o_local = _lib.ptr(self.saved.get("o_local"))
        a.o_global = _lib.ptr(self.saved.get("o_global"))
        a.vl = _lib.view(vl)
        a.kl_rotated = 1 if kl_rotated else 0
        self.attn_args = a
        tag = brick_tag(geometry)
        self.grid = tag is not None
        self.pre = []  # (name, args) launched before the attention kernel
        if not rope.identity and not kl_rotated:
            klr = torch.empty(kl.shape, dtype=kl.dtype, device=dev)
            self.pre.append(("p3d_rotate", (_lib.view(kl), _lib.view(klr), b, g, n, d, dt, rope.struct(), 0)))
            kl = klr
            self._keep.append(klr)
            a.kl_rotated = 1
        self.klr = kl  # the keys as the attention kernels read them (rotated unless rope is the identity)
        if self.grid:
            shape, radius, mapping = tag
            a.q, a.kl = _lib.view(q), _lib.view(kl)
            a.rope = rope.struct()
            a.grid[:] = list(shape)
            a.radius[:] = list(radius)
            a.raster_to_packed = _lib.ptr(mapping)
            self._keep.append(mapping)
            self.attn_name = "p3d_attn_fwd_grid"
        else:
            # Arbitrary graph: q rotates on load in both kernels.  The
            # indexed local kernel writes sl * o_L into y, and the rows kernel
            # adds the summary branch in its epilogue.
            a.q, a.kl = _lib.view(q), _lib.view(kl)
            a.rope = rope.struct()
            a.o_local_in = None
            self.pre.append(("p3d_local_fwd_indexed", (a, geometry.neighbors.data_ptr(), geometry.neighbors.shape[1])))
            self.attn_name = "p3d_attn_fwd_rows"

    def pool(self):
        _lib.call("p3d_pool_fwd", self.pool_args, _lib.stream_of(self.device))
        self.pool_args.norms_cleared = 0  # a repeated call must clear the slots again

    def attention(self):
        stream = _lib.stream_of(self.device)
        for name, args in self.pre:
            _lib.call(name, *args, stream)
        _lib.call(self.attn_name, self.attn_args, stream)

    def run(self):
        self.pool()
        self.attention()
        saved = dict(self.saved)
        saved.update({"sk": self.sk, "svt": self.svt})
        return self.y, saved


def forward(q, kl, vl, kg, vg, weight, bias, gate, sl, sg, geometry, temperature,
            rope: RopeSpec, pool_rope: RopeSpec, save_state=False):
    """Launch pooling and attention; returns y [B, H, N, d] (a transposed view of
    a [B, N, H, d] buffer) and, if ``save_state``, the tensors backward needs."""
    return ForwardPlan(q, kl, vl, kg, vg, weight, bias, gate, sl, sg, geometry, temperature, rope, pool_rope,
                       save_state).run()


class _Pack3DHip(torch.autograd.Function):
    """First-order autograd of the core (autograd.py:8-28 of amilworks/Pack3D).

    The forward saves the inputs, the summaries (sk, svt, norm slots), o_L,
    o_G and the two log-sum-exps, and, unless the rotation is the identity,
    kl as the plan rotated it (the backward's rotated keys); nothing of size
    N x M.  The backward refuses a geometry mutated since the forward.
    """

    @staticmethod
    def forward(ctx, q, kl, vl, kg, vg, weight, bias, gate, sl, sg, geometry, temperature, rope, pool_rope):
        plan = ForwardPlan(q, kl, vl, kg, vg, weight, bias, gate, sl, sg, geometry, temperature, rope, pool_rope,
                           save_state=True)
        y, saved = plan.run()
        ctx.save_for_backward(q, kl, vl, kg, vg, weight, bias, gate, sl, sg, saved["sk"], saved["svt"],
                              plan.sk_norm_max, saved["o_local"], saved["o_global"], saved["lse_local"],
                              saved["lse_global"], plan.klr if plan.klr is not kl else None)
        ctx.geometry, ctx.temperature, ctx.rope, ctx.pool_rope = geometry, temperature, rope, pool_rope
        ctx.key_scale = plan.key_scale
        return y

    @staticmethod
    @once_differentiable
    def backward(ctx, dy):
        ctx.geometry.check_unmodified()
        *state, klr = ctx.saved_tensors
        grads = backward(dy, *state, ctx.geometry, ctx.temperature, ctx.rope, ctx.pool_rope, ctx.key_scale,
                         klr=klr)
        return (*grads, None, None, None, None)


def _rotated(x, rope: RopeSpec):
    """x [B, heads, N, d] rotated by ``rope`` into a new contiguous tensor
    (x itself for the identity rotation)."""
    if rope.identity:
        return x
    b, heads, n, d = x.shape
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    _lib.call("p3d_rotate", _lib.view(_kernel_view(x)), _lib.view(out), b, heads, n, d, _lib.DTYPES[x.dtype],
              rope.struct(), 0, _lib.stream_of(x.device))
    return out


def _mix_parts(rows):
    return max(1, min(2048, -(-rows // 256)))


def _splits(n, m, bg):
    """Query splits of the summary dK/dV pass: enough workgroups to fill the
    GPU, each split at least 1024 queries."""
    blocks = -(-m // 128) * bg
    return max(1, min(64, -(-2048 // blocks), -(-n // 1024)))


def backward(dy, q, kl, vl, kg, vg, weight, bias, gate, sl, sg, sk, svt, sk_norm_max, o_local, o_global,
             lse_local, lse_global, geometry, temperature, rope, pool_rope, key_scale, out=None, klr=None):
    """The ten gradients of the core (kernels.py:313-356 of amilworks/Pack3D):
    dq, dkl, dkg with respect to the unrotated inputs (the rotation's backward
    is fused), dvl, dvg, dweight, dbias, dgate, dsl, dsg.  `out` may give
    (dq, dkl, dvl, dkg, dvg) as [B, *, N, d] views (16-byte aligned rows)
    that the kernels write in place, such as column ranges of the
    projections' gradients; they are returned in their place.  `klr`: kl
    already rotated by `rope` (as the forward used it), else it is rotated
    here."""
    b, h, n, d = q.shape
    g = kl.shape[1]
    dev, dt = q.device, _lib.DTYPES[q.dtype]
    f, slots = geometry.blocks.shape
    m = geometry.num_summaries
    mp = -(-m // 32) * 32
    stream = _lib.stream_of(dev)
    q, kl, vl, kg, vg = (_kernel_view(t) for t in (q, kl, vl, kg, vg))
    dy = _kernel_view(dy if dy.dtype == q.dtype else dy.to(q.dtype))
    keep = []
    qr = _rotated(q, rope)
    if klr is None:
        klr = _rotated(kl, rope)
    gate_k = gate if gate.dtype in _lib.DTYPES else gate.float()
    sl32, sg32 = param_f32(sl), param_f32(sg)
    parts = _mix_parts(b * h * n)
    splits = _splits(n, m, b * g)

    def empty(*shape, dtype=q.dtype):
        return torch.empty(*shape, dtype=dtype, device=dev)

    f32 = torch.float32
    bufs = dict(dol=empty(b, h, n, d), dog=empty(b, h, n, d), dl=empty(b, h, n, dtype=f32),
                dg=empty(b, h, n, dtype=f32), dgate=empty(b, h, n, dtype=gate_k.dtype),
                dslp=empty(parts, d, dtype=f32), dsgp=empty(parts, d, dtype=f32),
                sv_rows=empty(b, g, mp, d), skt=empty(b, g, mp // 32, d, 32),
                dql=empty(b, h, n, d, dtype=f32), dqg=empty(b, h, n, d, dtype=f32),
                dkl=empty(b, g, n, d, dtype=f32),
                dskp=empty(splits, b, g, mp, d, dtype=f32), dsvp=empty(splits, b, g, mp, d, dtype=f32))
    a = _lib.BwdArgs()
    a.batch, a.heads, a.kv_heads, a.tokens, a.head_dim, a.dtype = b, h, g, n, d, dt
    a.summaries, a.gate_dtype, a.parts, a.splits = m, _lib.DTYPES[gate_k.dtype], parts, splits
    a.q, a.kl, a.vl, a.gate = _lib.view(qr), _lib.view(klr), _lib.view(vl), _lib.view3(gate_k)
    a.local_scale, a.global_scale = sl32.data_ptr(), sg32.data_ptr()
    a.sk, a.svt, a.key_scale = sk.data_ptr(), svt.data_ptr(), float(key_scale)
    a.o_local, a.o_global = o_local.data_ptr(), o_global.data_ptr()
    a.lse_local, a.lse_global = lse_local.data_ptr(), lse_global.data_ptr()
    a.dy = _lib.view(dy)
    a.dol, a.dog, a.delta_local, a.delta_global = (bufs[k].data_ptr() for k in ("dol", "dog", "dl", "dg"))
    a.dgate, a.dsl_part, a.dsg_part = (bufs[k].data_ptr() for k in ("dgate", "dslp", "dsgp"))
    a.sv_rows, a.skt = bufs["sv_rows"].data_ptr(), bufs["skt"].data_ptr()
    a.dq_local, a.dq_global, a.dk_local = (bufs[k].data_ptr() for k in ("dql", "dqg", "dkl"))
    if out is None:
        out = tuple(empty(b, hh, n, d) for hh in (h, g, g, g, g))
    dq, dkl, dvl, dkg, dvg = out
    a.dv_local = _lib.view(dvl)
    a.dsk_part, a.dsv_part = bufs["dskp"].data_ptr(), bufs["dsvp"].data_ptr()
    keep += [qr, klr, gate_k, sl32, sg32, dy]

    _lib.call("p3d_mix_bwd", a, stream)
    tag = brick_tag(geometry)
    if tag is not None and not (q.dtype == torch.float32 and d == 128):
        # Brick-tiled on MFMA; fp32 planes of head_dim 128 do not fit in LDS.
        shape, radius, mapping = tag
        _lib.call("p3d_local_bwd_grid", a, _lib.i32x3(shape), _lib.i32x3(radius), _lib.ptr(mapping), stream)
    else:
        nb, rev = geometry.neighbors, geometry.reverse_neighbors
        _lib.call("p3d_local_bwd_indexed", a, nb.data_ptr(), nb.shape[1], rev.data_ptr(), rev.shape[1], stream)
    _lib.call("p3d_global_bwd_dq", a, stream)
    if q.dtype != torch.float32 and n >= 64 and n % 8 == 0:
        # Transposed copies of the rotated q and of dO_G: the summary dK/dV
        # pass copies its transposed query stages from them by LDS DMA.
        bufs["q_t"], bufs["dog_t"] = empty(b * h * d * n), empty(b * h * d * n)
        _lib.call("p3d_transpose_rows", _lib.view(qr), bufs["q_t"].data_ptr(), b, h, n, d, dt, stream)
        _lib.call("p3d_transpose_rows", _lib.view(bufs["dog"]), bufs["dog_t"].data_ptr(), b, h, n, d, dt, stream)
        a.q_t, a.dog_t = bufs["q_t"].data_ptr(), bufs["dog_t"].data_ptr()
    _lib.call("p3d_global_bwd_dkv", a, stream)
    _lib.call("p3d_finish_bwd", a, rope.struct(), _lib.view(dq), _lib.view(dkl), stream)

    w32 = param_f32(weight)
    b32 = param_f32(bias)
    pool_args = _lib.PoolArgs(b, g, n, d, dt, f, slots, geometry.pool_size, m, float(temperature), float(key_scale),
                              _lib.view(kg), _lib.view(vg), geometry.blocks.data_ptr(), w32.data_ptr(),
                              b32.data_ptr(), pool_rope.struct(), sk.data_ptr(), svt.data_ptr(),
                              sk_norm_max.data_ptr())
    dwp = empty(b * g * mp, d, dtype=f32)
    dbp = empty(b * g * mp, slots, dtype=f32)
    _lib.call("p3d_pool_bwd", pool_args, bufs["dskp"].data_ptr(), bufs["dsvp"].data_ptr(), splits,
              _lib.view(dkg), _lib.view(dvg), dwp.data_ptr(), dbp.data_ptr(), stream)
    keep += [w32, b32]
    dweight = dwp.sum(0).to(weight.dtype)
    dbias = dbp.sum(0).to(bias.dtype)
    dsl = bufs["dslp"].sum(0).to(sl.dtype)
    dsg = bufs["dsgp"].sum(0).to(sg.dtype)
    dgate = bufs["dgate"] if bufs["dgate"].dtype == gate.dtype else bufs["dgate"].to(gate.dtype)
    return dq, dkl, dvl, dkg, dvg, dweight, dbias, dgate, dsl, dsg


def _run(q, kl, vl, kg, vg, weight, bias, gate, sl, sg, geometry, temperature, rope, pool_rope):
    _validate_inputs(q, kl, vl, kg, vg, weight, bias, gate, sl, sg, geometry, temperature)
    _check_hip(q)
    inputs = (q, kl, vl, kg, vg, weight, bias, gate, sl, sg)
    if torch.is_grad_enabled() and any(t.requires_grad for t in inputs):
        return _Pack3DHip.apply(*inputs, geometry, float(temperature), rope, pool_rope)
    y, _ = forward(*inputs, geometry, float(temperature), rope, pool_rope, save_state=False)
    return y


class _Pack3DProjections(torch.autograd.Function):
    """The core on views of the layer's projections, qp [B, N, H*d] and kvp
    [B, N, 4*G*d] chunked kl | vl | kg | vg (attention.py:64-67), with
    gradients returned for qp and kvp directly: the backward kernels write
    dq, dkl, dvl, dkg and dvg straight into the projections' layout, so
    autograd does not transpose and stack five views."""

    @staticmethod
    def forward(ctx, qp, kvp, weight, bias, gate, sl, sg, heads, kv_heads, geometry, temperature, rope):
        q, kl, vl, kg, vg = _projection_views(qp, kvp, heads, kv_heads)
        plan = ForwardPlan(q, kl, vl, kg, vg, weight, bias, gate, sl, sg, geometry, temperature, rope, rope,
                           save_state=True)
        y, saved = plan.run()
        # plan.klr: kl rotated once by the plan, which the backward reuses
        ctx.save_for_backward(qp, kvp, weight, bias, gate, sl, sg, saved["sk"], saved["svt"], plan.sk_norm_max,
                              saved["o_local"], saved["o_global"], saved["lse_local"], saved["lse_global"],
                              plan.klr if plan.klr is not kl else None)
        ctx.geometry, ctx.temperature, ctx.rope, ctx.key_scale = geometry, temperature, rope, plan.key_scale
        ctx.heads, ctx.kv_heads = heads, kv_heads
        return y

    @staticmethod
    @once_differentiable
    def backward(ctx, dy):
        ctx.geometry.check_unmodified()
        qp, kvp, weight, bias, gate, sl, sg, *state, klr = ctx.saved_tensors
        views = _projection_views(qp, kvp, ctx.heads, ctx.kv_heads)
        dqp, dkvp = torch.empty_like(qp), torch.empty_like(kvp)
        grads = backward(dy, *views, weight, bias, gate, sl, sg, *state, ctx.geometry, ctx.temperature, ctx.rope,
                         ctx.rope, ctx.key_scale, out=_projection_views(dqp, dkvp, ctx.heads, ctx.kv_heads), klr=klr)
        return (dqp, dkvp, *grads[5:], None, None, None, None, None)


def _projection_views(qp, kvp, heads, kv_heads):
    """q [B, H, N, d] and kl, vl, kg, vg [B, G, N, d] as views of qp and kvp."""
    b, n = qp.shape[0], qp.shape[1]
    d = qp.shape[2] // heads
    q = qp.view(b, n, heads, d).transpose(1, 2)
    kv = kvp.view(b, n, 4, kv_heads, d)
    return (q, *(kv[:, :, i].transpose(1, 2) for i in range(4)))


def pack3d_hip_projections(qp, kvp, heads, kv_heads, weight, bias, gate, sl, sg, geometry, rope: RopeSpec, *,
                           temperature=1.0):
    """The core of the layer on its projections qp [B, N, H*d] and kvp
    [B, N, 4*G*d] (kl | vl | kg | vg) with the rotation ``rope``; the same
    values as pack3d_hip_rope on their views.  With autograd active the
    gradients of qp and kvp come back whole (_Pack3DProjections)."""
    views = _projection_views(qp, kvp, heads, kv_heads)
    inputs = (*views, weight, bias, gate, sl, sg)
    if not (torch.is_grad_enabled() and any(t.requires_grad for t in (qp, kvp, weight, bias, gate, sl, sg))):
        return _run(*inputs, geometry, temperature, rope, rope)
    _validate_inputs(*inputs, geometry, temperature)
    _check_hip(qp)
    if any(not (t.stride(-1) == 1 and t.is_contiguous()) for t in (qp, kvp)):
        return _run(*inputs, geometry, temperature, rope, rope)
    return _Pack3DProjections.apply(qp, kvp, weight, bias, gate, sl, sg, heads, kv_heads, geometry,
                                    float(temperature), rope)


def pack3d_hip(q, kl, vl, kg, vg, weight, bias, gate, sl, sg, geometry, *, temperature=1.0):
    """PACK3D core on the GPU with rotated q, kl, kg (the contract of reference.py:8-9).

    Returns ``sl * o_L + gate * sg * o_G`` with shape [B, H, N, d] in q.dtype.
    """
    ident = identity_rope(q.shape[-1], q.device) if q.device.type == "cuda" else None
    return _run(q, kl, vl, kg, vg, weight, bias, gate, sl, sg, geometry, temperature, ident, ident)


def pack3d_hip_rope(q, kl, vl, kg, vg, weight, bias, gate, sl, sg, geometry, rope: RopeSpec, *,
                    temperature=1.0):
    """PACK3D core with unrotated q, kl, kg: the rotation ``rope`` is applied on load."""
    return _run(q, kl, vl, kg, vg, weight, bias, gate, sl, sg, geometry, temperature, rope, rope)
