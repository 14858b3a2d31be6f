"""Shared input generators for the parity tests (not collected by pytest)."""
import torch

from oracle.pack3d_oracle import prepare_geometry as oracle_prepare


def make_case(n=37, d=16, b=2, h=4, g=2, volume=4, pool=3, dtype=torch.float32, seed=18):
    """Ragged asymmetric graph with an all-masked row and a padded last block.

    The generator of tests/test_triton.py:27-49 of the reference: edges
    {i, i+1 mod n, max(i-2, 0)}, row 0 empty, blocks = arange padded with -1,
    inputs ~ N(0, 0.5^2), pool weight/bias ~ N(0, 0.2^2), sigmoid gate,
    scales 1 + N and 0.25 + N.  Returns CPU inputs and the raw tables.
    """
    gen = torch.Generator().manual_seed(seed)
    nb = torch.full((n, 5), -1, dtype=torch.int32)
    for i in range(n):
        edges = sorted({i, (i + 1) % n, max(i - 2, 0)})
        nb[i, :len(edges)] = torch.tensor(edges)
    nb[0] = -1
    blocks = torch.full(((n + volume - 1) // volume, volume), -1, dtype=torch.int32)
    blocks.view(-1)[:n] = torch.arange(n)
    shapes = [(b, h, n, d)] + [(b, g, n, d)] * 4 + [(d,), (volume,), (b, h, n), (d,), (d,)]
    inputs = []
    for index, shape in enumerate(shapes):
        t = torch.randn(shape, generator=gen) * (0.2 if index in (5, 6) else 0.5)
        if index == 7:
            t = t.sigmoid()
        if index == 8:
            t = t + 1
        if index == 9:
            t = t + 0.25
        inputs.append(t.to(dtype))
    return inputs, nb, blocks, pool


def oracle_geometry(nb, blocks, pool):
    return oracle_prepare(nb, blocks, pool)


def random_core_inputs(b, h, g, n, d, volume, dtype, seed, scale=0.5, device="cpu"):
    """Unit-ish random core inputs for a layout with ``volume`` slots."""
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(b, h, n, d, generator=gen) * scale
    kl, vl, kg, vg = (torch.randn(b, g, n, d, generator=gen) * scale for _ in range(4))
    w = torch.randn(d, generator=gen) * 0.2
    bias = torch.randn(volume, generator=gen) * 0.2
    gate = torch.rand(b, h, n, generator=gen)
    sl = 1 + 0.1 * torch.randn(d, generator=gen)
    sg = 0.25 + 0.1 * torch.randn(d, generator=gen)
    out = [q, kl, vl, kg, vg, w, bias, gate, sl, sg]
    return [t.to(dtype=dtype, device=device) for t in out]


def rel_l2(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-12))


def max_abs(a, b):
    return float((a.detach().double().cpu() - b.detach().double().cpu()).abs().max())


def oracle_layer_grads(oracle, x, layout, dy, chunk=2048):
    """The oracle layer's output and gradients (input and every parameter,
    by name) for the upstream gradient ``dy``, in fp32, without an autograd
    graph over more than one chunk of query rows of the core, so that it runs
    at 262,144 tokens: the projections (LayerNorm, to_q, to_kv, RoPE, gate)
    and to_out are differentiated by autograd over the whole volume, the core
    by ``pack3d_reference_grads`` (chunked).  The same values as autograd of
    ``oracle(x, layout)`` up to summation order, which
    tests/test_oracle_layer.py checks on a small volume."""
    from oracle.pack3d_oracle import pack3d_reference, pack3d_reference_grads

    work = torch.float64 if x.dtype == torch.float64 else torch.float32
    x = x.detach().to(work).clone().requires_grad_()
    b, n = x.shape[0], x.shape[1]
    with torch.enable_grad():
        q, kl, vl, kg, vg, gate = oracle.project(x, layout)
        core_in = [t.detach() for t in (q, kl, vl, kg, vg)]
        params = [oracle.pool_weight, oracle.slot_bias, gate.detach(), oracle.local_scale, oracle.global_scale]
        params = [t.detach() for t in params]
        core = pack3d_reference(*core_in, *params, layout.geometry, temperature=oracle.temperature, chunk=chunk)
        core_leaf = core.detach().requires_grad_()
        y = x + oracle.to_out(core_leaf.transpose(1, 2).reshape(b, n, -1))
        y.backward(dy.to(work))
        grads = pack3d_reference_grads(*core_in, *params, layout.geometry, core_leaf.grad,
                                       temperature=oracle.temperature, chunk=chunk)
        torch.autograd.backward([q, kl, vl, kg, vg, gate], [grads[0], grads[1], grads[2], grads[3], grads[4],
                                                             grads[7]])
    named = {name: p.grad for name, p in oracle.named_parameters()}
    named["pool_weight"], named["slot_bias"] = grads[5], grads[6]
    named["local_scale"], named["global_scale"] = grads[8], grads[9]
    return y.detach(), x.grad, named
