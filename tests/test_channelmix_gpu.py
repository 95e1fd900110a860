"""GPU parity of the fused channel-mix kernels (shift + static lerps, relu^2, sigmoid gate)
and of the RWKV6ChannelMix module built on them, against the numpy oracle on identical
bf16 inputs.

Tolerance: max|gpu - oracle| / max|oracle| <= 1e-2 and relative L2 <= 1e-2 for the
elementwise kernels (their only rounding is the bf16 store; fp32 inside); the module
goes through bf16 hipBLASLt GEMMs and uses 2e-2.  The reference's elementwise metric is
reported for every tensor (tests/parity.py).
"""
import numpy as np
import pytest
import torch

import parity
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _n(t):
    return t.detach().float().cpu().numpy()


def _check(name, got, ref, tol=1e-2):
    parity.check(name, got, ref, tol_max=tol, tol_l2=tol,
                 elem_mean=parity.ELEM_MEAN if tol <= 1e-2 else parity.ELEM_MEAN_LORA)


def _bf(t):
    return t.to(torch.bfloat16)


# T = 1; T crossing the 8-token sub-segments and the 64-token blocks of the backward;
# C = 8 (one vector); C = 264 (a partial 256-channel block)
@pytest.mark.parametrize("shape", [(1, 1, 8), (9, 3, 64), (70, 2, 264), (130, 2, 512)])
@pytest.mark.parametrize("pdt", [torch.float32, torch.bfloat16])
def test_cmix_lerp_forward_backward(pkg, shape, pdt):
    T, B, C = shape
    g = torch.Generator().manual_seed(T * 7 + C)
    x = _bf(torch.randn(T, B, C, generator=g))
    mix = torch.rand(2, C, generator=g).to(pdt)
    d_mixed = _bf(torch.randn(2, T, B, C, generator=g))
    xd = x.to(DEV).requires_grad_(True)
    md = mix.to(DEV).requires_grad_(True)
    mixes = pkg.channelmix.cmix_lerp(xd, md)
    sum((m.float() * d.float()).sum() for m, d in zip(mixes, d_mixed.to(DEV))).backward()
    torch.cuda.synchronize()
    mixed = torch.stack(mixes)
    assert mixed.shape == (2, T, B, C) and md.grad.dtype == pdt
    _check("mixed", _n(mixed), orc.cmix_lerp_fwd(_n(x), _n(mix)))
    dx, d_mix = orc.cmix_lerp_bwd(_n(x), _n(mix), _n(d_mixed))
    _check("dx", _n(xd.grad), dx)
    _check("d_mix", _n(md.grad), d_mix)


@pytest.mark.parametrize("n", [8, 24, 4096 * 3 + 8])
def test_relu_sq_and_sigmoid_gate(pkg, n):
    g = torch.Generator().manual_seed(n)
    up, out, gp, dh, dy = (_bf(2 * torch.randn(n, generator=g)) for _ in range(5))
    upd = up.to(DEV).requires_grad_(True)
    h = pkg.channelmix.relu_sq(upd)
    h.backward(dh.to(DEV))
    od, gd = out.to(DEV).requires_grad_(True), gp.to(DEV).requires_grad_(True)
    y = pkg.channelmix.sigmoid_gate(od, gd)
    y.backward(dy.to(DEV))
    torch.cuda.synchronize()
    _check("h", _n(h), orc.relu_sq_fwd(_n(up)))
    _check("d_up", _n(upd.grad), orc.relu_sq_bwd(_n(up), _n(dh)))
    _check("y", _n(y), orc.sigmoid_gate_fwd(_n(out), _n(gp)))
    d_out, d_gp = orc.sigmoid_gate_bwd(_n(out), _n(gp), _n(dy))
    _check("d_out", _n(od.grad), d_out)
    _check("d_gate_pre", _n(gd.grad), d_gp)
    # relu^2 rounds once from fp32, as torch.square(torch.relu(.)) on bf16 does: bit-identical
    ref = torch.square(torch.relu(up.to(DEV)))
    assert torch.equal(h, ref)


def test_cmix_lerp_backward_deterministic(pkg):
    T, B, C = 300, 2, 512
    g = torch.Generator().manual_seed(5)
    x = _bf(torch.randn(T, B, C, generator=g)).to(DEV)
    mix = torch.rand(2, C, generator=g).to(DEV)
    dm = _bf(torch.randn(2, T, B, C, generator=g)).to(DEV)
    res = []
    for _ in range(2):
        xd, md = x.clone().requires_grad_(True), mix.clone().requires_grad_(True)
        up, gate = pkg.channelmix.cmix_lerp(xd, md)
        torch.autograd.backward([up, gate], [dm[0], dm[1]])
        res.append((xd.grad.clone(), md.grad.clone()))
    assert torch.equal(res[0][0], res[1][0]) and torch.equal(res[0][1], res[1][1])


@pytest.mark.parametrize("T,B,C,F", [(70, 2, 128, 448)])
def test_channel_mix_module(pkg, T, B, C, F):
    M = pkg.modules
    cfg = M.TransformerConfig(hidden_size=C, num_attention_heads=C // 64, ffn_hidden_size=F,
                              num_layers=2, params_dtype=torch.bfloat16)
    torch.manual_seed(0)
    mod = M.RWKV6ChannelMix(cfg, layer_number=1, device=DEV)
    with torch.no_grad():
        for p in (mod.linear_up.weight, mod.linear_gate.weight, mod.linear_down.weight):
            p.normal_(0.0, 0.5 / p.shape[1] ** 0.5)
    g = torch.Generator().manual_seed(1)
    x = _bf(torch.randn(T, B, C, generator=g))
    dy = _bf(torch.randn(T, B, C, generator=g))
    xd = x.to(DEV).requires_grad_(True)
    y, bias = mod(xd)
    assert bias is None and y.shape == (T, B, C)
    y.backward(dy.to(DEV))
    torch.cuda.synchronize()
    wu, wg, wd = (_n(p) for p in (mod.linear_up.weight, mod.linear_gate.weight, mod.linear_down.weight))
    mix = _n(mod.mix_coeffs)
    _check("y", _n(y), orc.channel_mix_fwd(_n(x), mix, wu, wg, wd), 2e-2)
    ref = orc.channel_mix_bwd(_n(x), mix, wu, wg, wd, _n(dy))
    got = (xd.grad, mod.mix_coeffs.grad, mod.linear_up.weight.grad, mod.linear_gate.weight.grad,
           mod.linear_down.weight.grad)
    for name, a, r in zip(("dx", "d_mix", "d_w_up", "d_w_gate", "d_w_down"), got, ref):
        _check(name, _n(a), r, 2e-2)


def test_cmix_lerp_one_output_used(pkg):
    """A loss on mixed_up alone leaves the gate gradient None: it counts as zero."""
    T, B, C = 40, 2, 64
    g = torch.Generator().manual_seed(9)
    x = _bf(torch.randn(T, B, C, generator=g))
    mix = torch.rand(2, C, generator=g)
    d_up = _bf(torch.randn(T, B, C, generator=g))
    xd, md = x.to(DEV).requires_grad_(True), mix.to(DEV).requires_grad_(True)
    up, _ = pkg.channelmix.cmix_lerp(xd, md)
    up.backward(d_up.to(DEV))
    torch.cuda.synchronize()
    dx, d_mix = orc.cmix_lerp_bwd(_n(x), _n(mix), np.stack([_n(d_up), np.zeros((T, B, C))]))
    _check("dx", _n(xd.grad), dx)
    _check("d_mix", _n(md.grad[0]), d_mix[0])
    assert torch.all(md.grad[1] == 0)
