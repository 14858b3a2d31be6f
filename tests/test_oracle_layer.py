"""Closed-form pins of the oracle's PACK3DAttention composition (CPU, fp64).

The layer (``src/pack3d/attention.py:63-89`` of amilworks/Pack3D) wires
LayerNorm, to_q, to_kv chunked kl | vl | kg | vg, the rotation of q, kl and
kg, the gate ``softmax(...)[..., 1]``, the head flattening before to_out and
the outer residual.  Each test below zeroes all but one part of the
projections so that the layer reduces to a formula that needs no softmax
over data-dependent scores, or only one whose scores are a cosine of a
coordinate difference:

* only kl or only kg nonzero        -> y == x exactly;
* only vl nonzero (kl = 0)          -> o_L is the mean of vl over the
                                        coordinate neighbourhood;
* only vg nonzero (kg = 0, b = 0)   -> o_G is the mean of vg over all tokens,
                                        scaled by the gate, which is the
                                        logistic function of the gate-bias
                                        difference when the gate weight is 0;
* one rotary pair on a 1-D row      -> local and global scores are
                                        a*b*cos(x_j - x_i)/sqrt(d) sums.

LayerNorm is evaluated from its definition (biased variance, eps).  The
last test plants each plausible composition slip in a subclass of the
oracle layer and requires that at least one of these pins fails for it.
"""
import math

import pytest
import torch

from oracle.pack3d_oracle import PACK3DAttention, axial_rope, build_layout, pack3d_reference

F64 = torch.float64


def layer_norm_def(x, w, b, eps):
    """LayerNorm from its definition: (x - mean) / sqrt(biased var + eps) * w + b."""
    mu = x.mean(-1, keepdim=True)
    var = ((x - mu) ** 2).mean(-1, keepdim=True)
    return (x - mu) / torch.sqrt(var + eps) * w + b


def neighbour_sets(coords, radius):
    """Rows j with |coord_j - coord_i| <= radius per axis, by brute force over coordinates."""
    c = coords.tolist()
    out = []
    for ci in c:
        out.append([j for j, cj in enumerate(c) if all(abs(cj[a] - ci[a]) <= radius[a] for a in range(3))])
    return out


def flatten_heads(o):
    """[B, H, N, d] -> [B, N, H*d] with head-major channels."""
    b, h, n, d = o.shape
    return torch.stack([o[:, i] for i in range(h)], 2).reshape(b, n, h * d)


def new_layer(cls, dim, heads, kv_heads, head_dim, block_volume, seed):
    torch.manual_seed(seed)
    layer = cls(dim, heads=heads, kv_heads=kv_heads, head_dim=head_dim, block_volume=block_volume).double()
    with torch.no_grad():
        layer.norm.weight.copy_(1 + 0.3 * torch.randn(dim, dtype=F64))
        layer.norm.bias.copy_(0.2 * torch.randn(dim, dtype=F64))
        layer.local_scale.copy_(1 + 0.3 * torch.randn(head_dim, dtype=F64))
        layer.global_scale.copy_(0.25 + 0.3 * torch.randn(head_dim, dtype=F64))
    return layer


def keep_chunks(layer, chunks):
    """Zero every to_kv output chunk (kl=0, vl=1, kg=2, vg=3) not in ``chunks``."""
    width = layer.kv_heads * layer.head_dim
    with torch.no_grad():
        for c in range(4):
            if c not in chunks:
                layer.to_kv.weight[c * width:(c + 1) * width] = 0


# ---- the pins: each returns the max-abs error of the layer against its closed form ----


def pin_identity(cls, chunk):
    """Only the kl (0) or kg (2) chunk nonzero: o_L = P @ 0 and o_G = P @ pool(0), so y == x."""
    layout = build_layout((2, 4, 4), (1, 2, 2), radius=1, pool_size=2)
    layer = new_layer(cls, 32, 4, 2, 16, 4, seed=1)
    keep_chunks(layer, (chunk,))
    x = torch.randn(2, 32, 32, dtype=F64, generator=torch.Generator().manual_seed(2))
    with torch.no_grad():
        return float((layer(x, layout) - x).abs().max())


def pin_local_value_mean(cls):
    """Only vl nonzero: kl = 0 makes every local score 0, so o_L(i) is the mean
    of vl over i's coordinate neighbourhood; vg = 0 makes o_G = 0.  Four query
    heads on two kv heads (query head h reads kv head h // 2)."""
    layout = build_layout((2, 4, 4), (1, 2, 2), radius=1, pool_size=2)
    layer = new_layer(cls, 32, 4, 2, 16, 4, seed=3)
    keep_chunks(layer, (1,))
    x = torch.randn(2, 32, 32, dtype=F64, generator=torch.Generator().manual_seed(4))
    with torch.no_grad():
        y = layer(x, layout)
        xn = layer_norm_def(x, layer.norm.weight, layer.norm.bias, layer.norm.eps)
        w = layer.to_kv.weight[32:64]                      # vl rows: [G*d, 2*G*d)
        vl = (xn @ w.t()).view(2, 32, 2, 16)               # [B, N, G, d]
        sets = neighbour_sets(layout.coords, (1, 1, 1))
        mean = torch.stack([vl[:, s].mean(1) for s in sets], 1)      # [B, N, G, d]
        o = torch.stack([mean[:, :, h // 2] for h in range(4)], 1)  # [B, H, N, d]
        expect = x + flatten_heads(layer.local_scale * o) @ layer.to_out.weight.t()
        return float((y - expect).abs().max())


def pin_global_value_mean(cls, gap):
    """Only vg nonzero (kl may be anything): kg = 0 and slot bias 0 make the
    slot softmax uniform and every summary score 0, so o_G is the mean of vg
    over all tokens (full fine blocks, equal coarse groups).  Gate weight 0 and
    biases (a, a + gap_h) per head make gate_h = 1 / (1 + exp(-gap_h))."""
    layout = build_layout((2, 4, 4), (1, 2, 2), radius=1, pool_size=2)
    layer = new_layer(cls, 32, 4, 2, 16, 4, seed=5)
    keep_chunks(layer, (0, 3))
    gaps = torch.tensor([gap, -gap, 0.5 * gap, 1.3], dtype=F64)
    with torch.no_grad():
        layer.slot_bias.zero_()
        layer.gate.weight.zero_()
        base = torch.randn(4, dtype=F64)
        layer.gate.bias.copy_(torch.stack((base, base + gaps), -1).reshape(-1))
        x = torch.randn(2, 32, 32, dtype=F64, generator=torch.Generator().manual_seed(6))
        y = layer(x, layout)
        xn = layer_norm_def(x, layer.norm.weight, layer.norm.bias, layer.norm.eps)
        vg = (xn @ layer.to_kv.weight[96:128].t()).view(2, 32, 2, 16)   # vg rows: [3*G*d, 4*G*d)
        mean = vg.mean(1)                                                # [B, G, d]
        gate = torch.tensor([1 / (1 + math.exp(-float(t))) for t in gaps], dtype=F64)
        o = torch.stack([gate[h] * mean[:, h // 2, None, :].expand(2, 32, 16) for h in range(4)], 1)
        expect = x + flatten_heads(layer.global_scale * o) @ layer.to_out.weight.t()
        return float((y - expect).abs().max())


def _one_pair_layer(cls, a, b, chunk, seed):
    """A 1 x 1 x 8 row, head_dim 16 (pairs (3, 3, 2): x-axis pair 0 is channels
    12, 13 at frequency 1), two query heads on one kv head.  LayerNorm weight 0
    and bias 1 on channel 8 make xn[8] = 1 for every token, so query head 0 is
    a e_12, query head 1 is 0, and the kept key chunk is b e_12 before
    rotation; the value chunks read only channels 0-7, which vary."""
    layer = new_layer(cls, 16, 2, 1, 16, 2, seed=seed)
    with torch.no_grad():
        layer.norm.weight[8:] = 0
        layer.norm.bias[8:] = 0
        layer.norm.bias[8] = 1
        layer.norm.weight[:8] = 1 + 0.3 * torch.randn(8, dtype=F64)
        layer.norm.bias[:8] = 0.2 * torch.randn(8, dtype=F64)
        layer.to_q.weight.zero_()
        layer.to_q.weight[12, 8] = a
        value_chunk = chunk + 1
        for c in range(4):
            rows = layer.to_kv.weight[16 * c:16 * (c + 1)]
            if c == chunk:
                rows.zero_()
                rows[12, 8] = b
            elif c == value_chunk:
                rows[:, 8:] = 0
            else:
                rows.zero_()
        layer.gate.weight.zero_()
        layer.gate.bias.zero_()          # gate = 1/2
        layer.pool_weight.zero_()
        layer.slot_bias.zero_()
    return layer


def pin_local_rotation(cls):
    """Rotation of q and kl: head 0 scores s_ij = a b cos(x_j - x_i) / 4 over
    |x_j - x_i| <= 1; head 1 (q = 0) weighs the neighbours uniformly."""
    a, b = 2.0, 1.5
    layout = build_layout((1, 1, 8), (1, 1, 2), radius=(0, 0, 1), pool_size=1, layout="raster_block")
    layer = _one_pair_layer(cls, a, b, 0, seed=7)
    x = torch.randn(1, 8, 16, dtype=F64, generator=torch.Generator().manual_seed(8))
    with torch.no_grad():
        y = layer(x, layout)
        xn = layer_norm_def(x, layer.norm.weight, layer.norm.bias, layer.norm.eps)
        vl = xn[0] @ layer.to_kv.weight[16:32].t()         # [N, d]
        xs = layout.coords[:, 2].tolist()
        rows = []
        for i in range(8):
            js = [j for j in range(8) if abs(xs[j] - xs[i]) <= 1]
            wts = torch.tensor([math.exp(a * b * math.cos(xs[j] - xs[i]) / 4) for j in js], dtype=F64)
            rows.append(((wts[:, None] * vl[js]).sum(0) / wts.sum(), vl[js].mean(0)))
        o = torch.stack([torch.stack([r[h] for r in rows]) for h in range(2)])[None]
        expect = x + flatten_heads(layer.local_scale * o) @ layer.to_out.weight.t()
        return float((y - expect).abs().max())


def pin_global_rotation(cls):
    """Rotation of q and kg: summary f pools the rotated keys of its two tokens
    uniformly (w = 0, b = 0), so head 0 scores s_if = a b (cos(x_f0 - x_i) +
    cos(x_f1 - x_i)) / 8; o_G is softmax_f(s) times the block means of vg
    (uniform for head 1), and the gate is 1/2."""
    a, b = 2.0, 1.5
    layout = build_layout((1, 1, 8), (1, 1, 2), radius=(0, 0, 1), pool_size=1, layout="raster_block")
    layer = _one_pair_layer(cls, a, b, 2, seed=9)
    x = torch.randn(1, 8, 16, dtype=F64, generator=torch.Generator().manual_seed(10))
    with torch.no_grad():
        y = layer(x, layout)
        xn = layer_norm_def(x, layer.norm.weight, layer.norm.bias, layer.norm.eps)
        vg = xn[0] @ layer.to_kv.weight[48:64].t()
        xs = layout.coords[:, 2].tolist()
        blocks = [[2 * f, 2 * f + 1] for f in range(4)]
        sv = torch.stack([vg[bl].mean(0) for bl in blocks])
        rows = []
        for i in range(8):
            s = [a * b * sum(math.cos(xs[t] - xs[i]) for t in bl) / 8 for bl in blocks]
            wts = torch.tensor([math.exp(v) for v in s], dtype=F64)
            rows.append(((wts[:, None] * sv).sum(0) / wts.sum(), sv.mean(0)))
        o = 0.5 * torch.stack([torch.stack([r[h] for r in rows]) for h in range(2)])[None]
        expect = x + flatten_heads(layer.global_scale * o) @ layer.to_out.weight.t()
        return float((y - expect).abs().max())


def all_pins(cls):
    errs = {"identity_kl": pin_identity(cls, 0), "identity_kg": pin_identity(cls, 2),
            "local_mean": pin_local_value_mean(cls), "local_rotation": pin_local_rotation(cls),
            "global_rotation": pin_global_rotation(cls)}
    for gap in (30.0, -30.0, 0.7):
        errs[f"global_mean_gap{gap}"] = pin_global_value_mean(cls, gap)
    return errs


def test_identity_when_only_kl_or_kg_is_nonzero():
    assert pin_identity(PACK3DAttention, 0) == 0.0
    assert pin_identity(PACK3DAttention, 2) == 0.0


def test_local_branch_is_neighbour_mean_of_vl():
    assert pin_local_value_mean(PACK3DAttention) < 1e-12


@pytest.mark.parametrize("gap", [30.0, -30.0, 0.7])
def test_global_branch_is_gated_token_mean_of_vg(gap):
    assert pin_global_value_mean(PACK3DAttention, gap) < 1e-12


def test_q_and_local_keys_are_rotated():
    assert pin_local_rotation(PACK3DAttention) < 1e-12


def test_q_and_global_keys_are_rotated_before_pooling():
    assert pin_global_rotation(PACK3DAttention) < 1e-12


# ---- planted mistakes: every one must fail at least one pin ----


class _Mutant(PACK3DAttention):
    """The oracle layer with one composition slip planted (``slip``)."""

    slip = None

    def project(self, x, layout):
        b, n = x.shape[0], x.shape[1]
        xn = x if self.slip == "no_norm" else self.norm(x)
        qf = self.to_q(xn)
        if self.slip == "q_channel_major":
            q = qf.reshape(b, n, self.head_dim, self.heads).permute(0, 3, 1, 2)
        else:
            q = qf.reshape(b, n, self.heads, self.head_dim).transpose(1, 2)
        chunks = list(self.to_kv(xn).chunk(4, -1))
        order = {"kl_kg": (2, 1, 0, 3), "vl_vg": (0, 3, 2, 1), "kl_vl": (1, 0, 2, 3),
                 "kg_vg": (0, 1, 3, 2)}.get(self.slip, (0, 1, 2, 3))
        kl, vl, kg, vg = (chunks[i].reshape(b, n, self.kv_heads, self.head_dim).transpose(1, 2) for i in order)
        coords = layout.coords
        rot = {"q": q, "kl": kl, "kg": kg}
        for name in ("q", "kl", "kg"):
            if self.slip != f"no_rope_{name}":
                rot[name] = axial_rope(rot[name], coords)
        q, kl, kg = rot["q"], rot["kl"], rot["kg"]
        if self.slip == "rope_vl":
            vl = axial_rope(vl, coords)
        index = 0 if self.slip == "gate_index0" else 1
        gate = self.gate(xn).reshape(b, n, self.heads, 2).softmax(-1)[..., index].transpose(1, 2)
        return q, kl, vl, kg, vg, gate

    def forward(self, x, layout):
        b, n = x.shape[0], x.shape[1]
        q, kl, vl, kg, vg, gate = self.project(x, layout)
        out = pack3d_reference(q, kl, vl, kg, vg, self.pool_weight, self.slot_bias, gate, self.local_scale,
                               self.global_scale, layout.geometry, temperature=self.temperature)
        flat = out.reshape(b, n, -1) if self.slip == "flat_no_transpose" else out.transpose(1, 2).reshape(b, n, -1)
        res = self.to_out(flat)
        return res if self.slip == "no_residual" else x + res


SLIPS = ["none", "no_norm", "q_channel_major", "kl_kg", "vl_vg", "kl_vl", "kg_vg", "no_rope_q", "no_rope_kl",
         "no_rope_kg", "rope_vl", "gate_index0", "flat_no_transpose", "no_residual"]


@pytest.mark.parametrize("slip", SLIPS)
def test_planted_slip_fails_a_pin(slip):
    cls = type(f"Mutant_{slip}", (_Mutant,), {"slip": slip})
    errs = all_pins(cls)
    worst = max(errs.values())
    if slip == "none":
        # The mutant scaffold without a slip is the oracle's composition.
        assert worst < 1e-12, errs
    else:
        assert worst > 1e-6, f"slip {slip} passes every pin: {errs}"


def test_chunked_layer_gradients_equal_autograd():
    """tests/_cases.oracle_layer_grads (projections by autograd, the core by
    the chunked pack3d_reference_grads) gives the same input and parameter
    gradients as autograd of the whole oracle layer, in fp64, with chunks
    smaller than the volume and random pooling parameters."""
    from tests._cases import oracle_layer_grads

    torch.manual_seed(4)
    layer = PACK3DAttention(32, heads=4, kv_heads=2, head_dim=16, block_volume=8).double()
    with torch.no_grad():
        for p in layer.parameters():
            p.add_(0.1 * torch.randn_like(p))
    layout = build_layout((4, 4, 6), (2, 2, 2), radius=1, pool_size=2, layout="native_block_morton")
    gen = torch.Generator().manual_seed(5)
    x = torch.randn(2, 96, 32, generator=gen, dtype=F64)
    dy = torch.randn(2, 96, 32, generator=gen, dtype=F64)
    y, dx, named = oracle_layer_grads(layer, x, layout, dy, chunk=40)
    xr = x.clone().requires_grad_()
    layer.zero_grad(set_to_none=True)
    yr = layer(xr, layout)
    yr.backward(dy)
    torch.testing.assert_close(y, yr.detach(), atol=1e-12, rtol=1e-12)
    torch.testing.assert_close(dx, xr.grad, atol=1e-11, rtol=1e-11)
    for name, p in layer.named_parameters():
        torch.testing.assert_close(named[name], p.grad, atol=1e-11, rtol=1e-11, msg=name)
