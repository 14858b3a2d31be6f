"""The layer's linear maps in 16-bit training: p3d_weight_grad against the
fp32 product dy^T x, and the layer's gradients through linear.InputProjections
/ linear.OutputResidual against the same layer on torch's nn.Linear path.

Bars: the kernel accumulates in fp32 over the rows, so against an fp32 GEMM
of the same 16-bit inputs the relative L2 error is that of fp32 summation
order (< 1e-5).  Against torch's autocast path, which rounds each weight
gradient to bf16 before it reaches the fp32 .grad, gradients agree to bf16
rounding (relative L2 < 1e-2).
"""
import math

import pytest
import torch

import pack3d_amd as p3d
from pack3d_amd import _lib, linear
from tests._cases import rel_l2

pytestmark = pytest.mark.gpu


def _reference(dy, x):
    return torch.mm(dy.float().t(), x.float())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,out_f,in_f,splits", [(37, 8, 192, 1), (1000, 200, 32, 3), (4099, 136, 256, 7),
                                                    (70000, 384, 192, 33), (262144, 192, 192, 128),
                                                    (3001, 264, 512, 5), (777, 40, 1024, 2),
                                                    (262144, 512, 512, 52)])
def test_weight_grad_matches_fp32_product(gpu, dtype, rows, out_f, in_f, splits):
    """Ragged row counts (not multiples of the token stage or of the split),
    output widths that leave part of a 256-row workgroup idle, every split
    count from one to the c4 setting, the c4 size itself, and inputs wider
    than 256 columns (column blocks of 256; 512 at 262,144 rows is the
    allen15 preset's to_out)."""
    print(f"weight grad {rows}x{out_f}x{in_f} s{splits} {dtype}", flush=True)
    gen = torch.Generator(device=gpu).manual_seed(rows + out_f)
    dy = torch.randn(rows, out_f, device=gpu, generator=gen).to(dtype)
    x = torch.randn(rows, in_f, device=gpu, generator=gen).to(dtype)
    dw = torch.empty(out_f, in_f, device=gpu)
    work = torch.empty(splits, out_f, in_f, device=gpu)
    _lib.call("p3d_weight_grad", dy.data_ptr(), out_f, x.data_ptr(), in_f, dw.data_ptr(), work.data_ptr(), rows,
              out_f, in_f, splits, _lib.DTYPES[dtype], _lib.stream_of(gpu))
    err = rel_l2(dw, _reference(dy, x))
    print(f"  rel_l2={err:.3g}", flush=True)
    assert err < 1e-5


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,dim,outs", [(37, 192, (192, 768, 8)), (1000, 64, (64, 256, 16)),
                                           (4099, 96, (96, 384, 8)), (5000, 128, (128, 512, 8)),
                                           (3001, 256, (256, 1024, 8)), (262144, 192, (192, 768, 8)),
                                           (2049, 384, (384, 384, 24)), (4100, 512, (512, 512, 16))])
def test_input_grad_matches_fp32_products(gpu, dtype, rows, dim, outs):
    """p3d_input_grad (dq Wq + dkv Wkv + dg Wg as one contraction) against
    the three products in fp32 on the same 16-bit inputs: one rounding of the
    fp32 sum, so every element within half a unit in the last place of the
    16-bit type plus the fp32 summation-order slack.  dq and dkv are column
    ranges of one wider buffer (row strides past the rows, as the layer's
    gradient layout can give); ragged row counts; every supported width and
    the c4 shape."""
    print(f"input grad {rows}x{dim} {outs} {dtype}", flush=True)
    gen = torch.Generator(device=gpu).manual_seed(rows + dim)
    qo, kvo, go = outs
    wide = torch.randn(rows, qo + kvo + 16, device=gpu, generator=gen).to(dtype)
    dq, dkv = wide[:, :qo], wide[:, qo:qo + kvo]
    dg = torch.randn(rows, go, device=gpu, generator=gen).to(dtype)
    ws = [(torch.randn(o, dim, device=gpu, generator=gen) / math.sqrt(dim)).to(dtype) for o in outs]
    got = linear.input_grad([dq, dkv, dg], ws)
    assert got is not None and got.dtype == dtype and got.shape == (rows, dim)
    ref = sum(torch.mm(a.float(), w.float()) for a, w in zip((dq, dkv, dg), ws))
    scale = sum(torch.mm(a.float().abs(), w.float().abs()) for a, w in zip((dq, dkv, dg), ws))
    ulp = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
    excess = ((got.float() - ref).abs() - ulp * ref.abs() - 1e-5 * scale).max().item()
    print(f"  excess={excess:.3g}", flush=True)
    assert excess <= 0


def test_input_grad_declines_unsupported_shapes(gpu):
    """Widths and feature counts the kernel does not take go back to the
    three products (None), and the kernel rejects them before launching."""
    dt = torch.bfloat16
    dys = [torch.zeros(64, o, device=gpu, dtype=dt) for o in (48, 192, 8)]
    ws = [torch.zeros(o, 48, device=gpu, dtype=dt) for o in (48, 192, 8)]
    assert linear.input_grad(dys, ws) is None  # dim 48
    dys = [torch.zeros(64, o, device=gpu, dtype=dt) for o in (64, 256, 4)]
    ws = [torch.zeros(o, 64, device=gpu, dtype=dt) for o in (64, 256, 4)]
    assert linear.input_grad(dys, ws) is None  # 4 gate features
    with pytest.raises(RuntimeError, match="dim must be"):
        _lib.call("p3d_input_grad", 16, 64, 64, 16, 256, 256, 16, 8, 8, 16, 384, 16, 64, 48, _lib.DTYPES[dt], None)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,in_f,outs", [(37, 192, (192, 768, 8)), (4099, 96, (96, 384, 8)),
                                            (262144, 192, (192, 768, 8))])
def test_weight_grads3_match_fp32_products(gpu, dtype, rows, in_f, outs):
    """p3d_weight_grad3 (three dW sharing x from one pass) against the fp32
    products dy^T x of the same 16-bit inputs; two of the dy are column
    ranges of one wider buffer (row strides past the rows, a gap between
    them), the third a separate tensor; ragged and c4 row counts."""
    print(f"weight grads3 {rows}x{in_f} {outs} {dtype}", flush=True)
    gen = torch.Generator(device=gpu).manual_seed(rows + in_f)
    qo, kvo, go = outs
    wide = torch.randn(rows, qo + kvo + 24, device=gpu, generator=gen).to(dtype)
    dys = [wide[:, :qo], wide[:, qo + 8:qo + 8 + kvo], torch.randn(rows, go, device=gpu, generator=gen).to(dtype)]
    x = torch.randn(rows, in_f, device=gpu, generator=gen).to(dtype)
    got = linear.weight_grads3(dys, x)
    assert got is not None
    for dy, dw in zip(dys, got):
        err = rel_l2(dw, _reference(dy, x))
        print(f"  rel_l2={err:.3g}", flush=True)
        assert err < 1e-5


@pytest.mark.parametrize("rows,in_f,outs", [(4099, 512, (512, 512, 16)), (1000, 768, (64, 128, 8))])
def test_weight_grads3_wide_inputs(gpu, rows, in_f, outs):
    """p3d_weight_grad3 over inputs wider than 256 columns (the allen15
    preset's dim 512: to_q 512, to_kv 512, gate 16 outputs) against the fp32
    products, with dy as column slices of one wider buffer."""
    print(f"weight grads3 wide {rows}x{in_f} {outs}", flush=True)
    gen = torch.Generator(device=gpu).manual_seed(rows + in_f)
    qo, kvo, go = outs
    wide = torch.randn(rows, qo + kvo + 24, device=gpu, generator=gen).to(torch.bfloat16)
    dys = [wide[:, :qo], wide[:, qo + 8:qo + 8 + kvo], torch.randn(rows, go, device=gpu, generator=gen).to(torch.bfloat16)]
    x = torch.randn(rows, in_f, device=gpu, generator=gen).to(torch.bfloat16)
    got = linear.weight_grads3(dys, x)
    assert got is not None
    for dy, dw in zip(dys, got):
        err = rel_l2(dw, _reference(dy, x))
        print(f"  rel_l2={err:.3g}", flush=True)
        assert err < 1e-5


def test_weight_grad_strided_rows_and_determinism(gpu):
    """Row strides wider than the rows (column slices of wider tensors, as the
    layer's projections are) and bit-identical repeats."""
    print("weight grad strided", flush=True)
    gen = torch.Generator(device=gpu).manual_seed(3)
    wide_dy = torch.randn(5000, 400, device=gpu, generator=gen).to(torch.bfloat16)
    wide_x = torch.randn(5000, 264, device=gpu, generator=gen).to(torch.bfloat16)
    dy, x = wide_dy[:, 16:208], wide_x[:, 8:200]
    a = linear.weight_grad(dy, x)
    b = linear.weight_grad(dy, x)
    assert torch.equal(a, b)
    assert rel_l2(a, _reference(dy, x)) < 1e-5


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_layer_training_gradients_match_torch_linear(gpu, dtype):
    """Forward and every gradient of the layer under autocast with the HIP
    weight gradients, against the same layer with its linear maps on
    torch's nn.Linear autograd; the kernel path must actually run."""
    print(f"layer training linear {dtype}", flush=True)
    torch.manual_seed(0)
    shape = (8, 16, 12)
    n = math.prod(shape)
    layer = p3d.PACK3DAttention(192, heads=4, kv_heads=4, head_dim=48, block_volume=64).to(gpu)
    lay = p3d.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout="raster_block", device=gpu)
    x = torch.randn(1, n, 192, generator=torch.Generator().manual_seed(1)).to(gpu)
    dy = torch.randn(1, n, 192, generator=torch.Generator().manual_seed(2)).to(gpu)

    def run(hip):
        layer.zero_grad(set_to_none=True)
        xg = x.clone().requires_grad_()
        if not hip:
            layer._hip_linear = lambda _x: False
        try:
            with torch.autocast("cuda", dtype=dtype):
                y = layer(xg, lay)
            y.backward(dy.to(y.dtype))
        finally:
            layer.__dict__.pop("_hip_linear", None)
        return y.detach().float(), xg.grad.detach().clone(), {k: p.grad.detach().clone()
                                                              for k, p in layer.named_parameters()}

    calls = []
    real = _lib.call

    def counting(name, *args):
        calls.append(name)
        return real(name, *args)

    linear._lib.call = counting
    try:
        y_h, dx_h, g_h = run(True)
    finally:
        linear._lib.call = real
    # to_out's weight gradient alone; to_q / to_kv / gate share one pass over
    # the tokens, and their input gradients one contraction.
    assert calls.count("p3d_weight_grad") == 1 and calls.count("p3d_weight_grad3") == 1, calls
    assert calls.count("p3d_input_grad") == 1 and calls.count("p3d_project_linear") == 1, calls
    y_t, dx_t, g_t = run(False)
    assert rel_l2(y_h, y_t) < 1e-2
    assert rel_l2(dx_h, dx_t) < 1e-2
    for k in g_t:
        err = rel_l2(g_h[k], g_t[k])
        print(f"  {k}: rel_l2={err:.3g}", flush=True)
        assert err < 1e-2, (k, err)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dim,q_out,kv_out,g_out,rows", [(192, 192, 768, 8, 1003), (64, 64, 128, 4, 77),
                                                         (96, 48, 64, 6, 300), (256, 128, 512, 4, 129),
                                                         (512, 256, 256, 2, 65), (128, 32, 96, 16, 2048)])
def test_project_linear_matches_fp32_products(gpu, dtype, dim, q_out, kv_out, g_out, rows):
    """p3d_project_linear (the training layer's three input projections in one
    pass) against the products of the same 16-bit operands in fp32, rounded
    once to the 16-bit type (what torch.mm / torch.addmm compute up to the
    order of the fp32 sums): every value within one rounding step of the
    output.  Ragged row counts; blocks of 32 outputs that straddle q / kv and
    kv / gate (q_out 48, g_out 6); a gate bias in fp32 that the layer rounds
    to the compute type first, as torch.addmm(bg.to(dt), ...) does."""
    print(f"project linear {dim} {q_out}/{kv_out}/{g_out} rows={rows} {dtype}", flush=True)
    gen = torch.Generator(device=gpu).manual_seed(dim + rows)
    x = (torch.randn(rows, dim, device=gpu, generator=gen) * 1.5).to(dtype)
    ws = [(torch.randn(o, dim, device=gpu, generator=gen) / dim ** 0.5).to(dtype) for o in (q_out, kv_out, g_out)]
    bg = torch.randn(g_out, device=gpu, generator=gen)
    got = linear.project_linear(x, ws, bg)
    assert got is not None
    bias = bg.to(dtype).float()
    exp = [x.float() @ ws[0].float().t(), x.float() @ ws[1].float().t(), x.float() @ ws[2].float().t() + bias]
    tol = {torch.bfloat16: 2 ** -8, torch.float16: 2 ** -11}[dtype]
    for name, g_, e_ in zip(("q", "kv", "gate"), got, exp):
        assert g_.shape == e_.shape and g_.dtype == dtype, name
        g32 = g_.float()
        bound = tol * e_.abs() * 1.01 + 1e-6
        assert ((g32 - e_).abs() <= bound).all(), (name, float((g32 - e_).abs().max()))
        # almost every value is the correctly rounded fp32 product
        assert float((g32 == e_.to(dtype).float()).float().mean()) > 0.98, name


def test_project_linear_declines_unsupported_shapes():
    """Shapes the kernel does not take go back to the torch products (None)
    before anything is launched: a width outside its list, q_out not a
    multiple of 16, an odd gate width, fp32."""
    x = torch.zeros(4, 80, dtype=torch.bfloat16)
    ws = [torch.zeros(o, 80, dtype=torch.bfloat16) for o in (32, 64, 2)]
    assert linear.project_linear(x, ws, torch.zeros(2)) is None
    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    ws = [torch.zeros(o, 64, dtype=torch.bfloat16) for o in (24, 64, 2)]
    assert linear.project_linear(x, ws, torch.zeros(2)) is None
    ws = [torch.zeros(o, 64, dtype=torch.bfloat16) for o in (32, 64, 3)]
    assert linear.project_linear(x, ws, torch.zeros(3)) is None
    x32 = torch.zeros(4, 64)
    ws32 = [torch.zeros(o, 64) for o in (32, 64, 2)]
    assert linear.project_linear(x32, ws32, torch.zeros(2)) is None


@pytest.mark.parametrize("x_dtype,y_dtype", [(torch.float32, torch.bfloat16), (torch.float32, torch.float16),
                                              (torch.bfloat16, torch.bfloat16), (torch.float32, torch.float32)])
@pytest.mark.parametrize("rows,dim", [(1, 192), (1003, 192), (517, 64), (300, 512), (777, 384), (4099, 512),
                                      (97, 272)])
@pytest.mark.parametrize("residual", [False, True, "pass"])
def test_layer_norm_train_forward_backward_match_torch(gpu, x_dtype, y_dtype, rows, dim, residual):
    """LayerNormTrain against torch.layer_norm in fp64 on the same inputs: the
    output to one rounding of the output type, dx to fp32 accuracy, the
    affine gradients summed over the rows.  With the residual copy: the copy
    is x cast to the output type (bit-exact), and its gradient is added to
    dx.  With the pass-through: x itself, its gradient (in x's type) added
    to dx."""
    print(f"layer norm train {rows}x{dim} {x_dtype}->{y_dtype} residual={residual}", flush=True)
    gen = torch.Generator(device=gpu).manual_seed(rows + dim)
    x = (torch.randn(rows, dim, device=gpu, generator=gen) * 2 + 0.5).to(x_dtype)
    w = torch.randn(dim, device=gpu, generator=gen)
    b = torch.randn(dim, device=gpu, generator=gen)
    dy = torch.randn(rows, dim, device=gpu, generator=gen).to(y_dtype)
    dres = torch.randn(rows, dim, device=gpu, generator=gen).to(x_dtype if residual == "pass" else y_dtype)
    xg, wg, bg = (t.clone().requires_grad_() for t in (x, w, b))
    if residual == "pass":
        y, xr = linear.LayerNormTrain.apply(xg, wg, bg, 1e-5, y_dtype, "pass")
        assert xr.dtype == x_dtype and torch.equal(xr, x)
        torch.autograd.backward([y, xr], [dy, dres])
    elif residual:
        y, xc = linear.LayerNormTrain.apply(xg, wg, bg, 1e-5, y_dtype, True)
        assert xc.dtype == y_dtype and torch.equal(xc, x.to(y_dtype))
        torch.autograd.backward([y, xc], [dy, dres])
    else:
        y = linear.LayerNormTrain.apply(xg, wg, bg, 1e-5, y_dtype)
        y.backward(dy)
    xd, wd, bd = (t.detach().double().requires_grad_() for t in (x, w, b))
    e = torch.nn.functional.layer_norm(xd, (dim,), wd, bd, 1e-5)
    e.backward(dy.double())
    if residual:
        xd.grad += dres.double()
    ulp = {torch.bfloat16: 2 ** -8, torch.float16: 2 ** -10, torch.float32: 2 ** -18}[y_dtype]
    assert y.dtype == y_dtype
    # One rounding of the output type, plus fp32 arithmetic on terms of order
    # one (the bias): an absolute floor of ulp.
    excess = float(((y.double() - e.detach()).abs() - ulp * (e.detach().abs() + 1.0)).max())
    assert excess <= 0, excess
    assert xg.grad.dtype == x_dtype
    tol = 1e-5 if x_dtype == torch.float32 else 1e-2
    assert rel_l2(xg.grad, xd.grad) < tol, rel_l2(xg.grad, xd.grad)
    assert rel_l2(wg.grad, wd.grad) < 1e-5 and rel_l2(bg.grad, bd.grad) < 1e-5


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,dim,k", [(777, 192, 192), (300, 64, 128), (33, 512, 96)])
def test_output_residual_wide_matches_torch(gpu, dt, rows, dim, k):
    """OutputResidualWide (p3d_out_residual with an fp32 residual) against
    x + (y Wo^T in dt) as torch computes it under autocast: the product
    rounded to dt (the kernel's fp32 sum may round the other way, one unit
    of dt at the product), added to the unrounded fp32 x; and its
    gradients: dx = dout, dy and dWo against torch's in fp32."""
    print(f"output residual wide {rows}x{dim} k{k} {dt}", flush=True)
    gen = torch.Generator(device=gpu).manual_seed(rows + dim + k)
    x = torch.randn(rows, dim, device=gpu, generator=gen) * 4
    y = torch.randn(rows, k, device=gpu, generator=gen).to(dt)
    w = torch.randn(dim, k, device=gpu, generator=gen) / math.sqrt(k)
    xg, yg, wg = (t.clone().requires_grad_() for t in (x, y, w))
    out = linear.OutputResidualWide.apply(xg, yg, wg, dt)
    assert out.dtype == torch.float32
    prod = torch.mm(y, w.to(dt).t())
    step = {torch.bfloat16: 2 ** -8, torch.float16: 2 ** -11}[dt]
    err = (out.detach() - (x + prod.float())).abs()
    assert (err <= 2 * step * prod.float().abs() + 1e-6).all(), float(err.max())
    dout = torch.randn(rows, dim, device=gpu, generator=gen)
    out.backward(dout)
    assert torch.equal(xg.grad, dout)
    d16 = dout.to(dt)
    assert rel_l2(yg.grad.float(), (d16.float() @ w.to(dt).float())) < 1e-2
    assert rel_l2(wg.grad, d16.float().t() @ y.float()) < 1e-2


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_copy_rows_into_projection_layout(gpu, dtype):
    """p3d_copy_rows: dense [B, G, N, d] into the strided kv-chunk views of a
    [B, N, 4, G, d] buffer, bit-exact, other chunks untouched."""
    print(f"copy rows {dtype}", flush=True)
    b, g, n, d = 2, 3, 1001, 48
    src = torch.randn(b, g, n, d, device=gpu).to(dtype)
    dst = torch.full((b, n, 4, g, d), 7.0, device=gpu, dtype=dtype)
    view = dst[:, :, 2].transpose(1, 2)
    _lib.call("p3d_copy_rows", _lib.view(src), _lib.view(view), b, g, n, d, _lib.DTYPES[dtype], _lib.stream_of(gpu))
    assert torch.equal(view, src)
    others = dst[:, :, [0, 1, 3]]
    assert torch.equal(others, torch.full_like(others, 7.0))


@pytest.mark.parametrize("amp_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("grad", [True, False])
def test_layer_autocast_keeps_the_wide_residual(gpu, grad, amp_dtype):
    """Under autocast with an fp32 input the reference returns
    ``residual + to_out(...)`` in fp32 with the residual unrounded
    (attention.py:89).  Inputs of scale 4 make a bf16-rounded residual miss
    the bound by a factor of ~3 while the bf16 attention branch stays inside."""
    import oracle.pack3d_oracle as ref
    from tests._cases import max_abs
    print(f"layer autocast residual grad={grad} {amp_dtype}", flush=True)
    torch.manual_seed(0)
    shape = (8, 16, 12)
    n = math.prod(shape)
    oracle = ref.PACK3DAttention(192, heads=4, kv_heads=4, head_dim=48, block_volume=64)
    layer = p3d.PACK3DAttention(192, heads=4, kv_heads=4, head_dim=48, block_volume=64)
    layer.load_state_dict(oracle.state_dict())
    layer = layer.to(gpu)
    lay_h = p3d.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout="raster_block", device=gpu)
    lay_r = ref.build_layout(shape, (4, 4, 4), radius=2, pool_size=1, layout="raster_block")
    x = torch.randn(1, n, 192, generator=torch.Generator().manual_seed(1)) * 4
    xg = x.to(gpu).requires_grad_(grad)
    calls = []
    real = _lib.call

    def counting(name, *args):
        calls.append(name)
        return real(name, *args)

    linear._lib.call = counting
    try:
        with torch.set_grad_enabled(grad), torch.autocast("cuda", dtype=amp_dtype):
            y = layer(xg, lay_h)
    finally:
        linear._lib.call = real
    # The fp32 residual goes through the output product's own kernel, and
    # the projections through the linear-mode projection kernel, with and
    # without autograd.
    assert "p3d_out_residual" in calls and "p3d_project_linear" in calls, calls
    assert "p3d_layer_norm_train" in calls, calls
    with torch.no_grad():
        exp = oracle(x, lay_r)
    assert y.dtype == torch.float32
    m = max_abs(y.detach(), exp)
    print(f"  max_abs={m:.3g}", flush=True)
    assert m < 1e-2
    if grad:
        y.backward(torch.ones_like(y))
        assert xg.grad.dtype == torch.float32 and torch.isfinite(xg.grad).all()
