"""GPU parity of the fused time-mix kernels (token shift / lerp, the LoRA bottlenecks fused
with the ddlerp or bias, GroupNorm*gate) against the numpy oracle on identical bf16 inputs.

Tolerance: max|gpu - oracle| / max|oracle| <= 1e-2 and relative L2 <= 1e-2 for the
elementwise kernels (their only rounding is the bf16 store); the LoRA weight
gradients and the decay bottleneck's input gradient go through bf16 hipBLASLt GEMMs and
use 2e-2.  The reference's elementwise metric is reported for every tensor (tests/parity.py).
"""
import ctypes

import numpy as np
import pytest
import torch

import parity
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _n(t):
    return t.detach().float().cpu().numpy()


def _check(name, got, ref, tol=1e-2, elem_mean=parity.ELEM_MEAN):
    parity.check(name, got, ref, tol_max=tol, tol_l2=tol, elem_mean=elem_mean)


def _check_lora(name, got, ref, tol=1e-2):
    """Tensors of the LoRA paths: an hipBLASLt GEMM with bf16 operands sits on the way."""
    parity.check(name, got, ref, tol_max=tol, tol_l2=tol, elem_mean=parity.ELEM_MEAN_LORA)


def _bf(t):
    return t.to(torch.bfloat16)


@pytest.mark.parametrize("shape", [(1, 1, 8), (7, 3, 64), (130, 2, 512)])
@pytest.mark.parametrize("pdt", [torch.float32, torch.bfloat16])
def test_shift_lerp(pkg, shape, pdt):
    T, B, C = shape
    g = torch.Generator().manual_seed(T + C)
    x = _bf(torch.randn(T, B, C, generator=g))
    maa = torch.rand(C, generator=g).to(pdt)
    xxx = pkg.timemix.shift_lerp(x.to(DEV), maa.to(DEV))
    torch.cuda.synchronize()
    _check("xxx", _n(xxx), orc.shift_lerp_fwd(_n(x), _n(maa)))


@pytest.mark.parametrize("E,R", [(5, 32), (5, 64), (1, 64), (1, 96)])
def test_bottleneck_module(pkg, E, R):
    """RWKV6Bottleneck.forward (:177-195) on its own, both expansions: [T,B,C] -> [T,B,E,C]
    through the HIP up-projection + bias, forward and every gradient, against the oracle."""
    M = pkg.modules
    T, B, C = 67, 2, 192
    cfg = M.TransformerConfig(hidden_size=C, num_attention_heads=3, params_dtype=torch.float32)
    bn = M.RWKV6Bottleneck(cfg, R, E, E == 1, device=DEV)
    g = torch.Generator().manual_seed(E * 100 + R)
    with torch.no_grad():      # GEMM operands are bf16: keep the weights bf16-representable
        bn.weight_down.copy_(_bf(torch.empty(C, E, R).uniform_(-0.1, 0.1, generator=g)).float())
        bn.weight_up.copy_(_bf(torch.empty(E, R, C).uniform_(-0.3, 0.3, generator=g)).float())
        bn.bias.uniform_(-1, 1)
    x = _bf(torch.randn(T, B, C, generator=g))
    dy = _bf(torch.randn(T, B, E, C, generator=g))
    xg = x.to(DEV).requires_grad_(True)
    out = bn(xg)
    assert out.shape == (T, B, E, C)
    (out.float() * dy.to(DEV).float()).sum().backward()
    torch.cuda.synchronize()
    xn, wdn, wun, bnn = (_n(t) for t in (x, bn.weight_down, bn.weight_up, bn.bias))
    _check_lora("out", _n(out), orc.bottleneck_fwd(xn, wdn, wun, bnn))
    dx, d_wd, d_wu, d_b = orc.bottleneck_bwd(xn, wdn, wun, _n(dy))
    _check_lora("dx", _n(xg.grad), dx, 2e-2)
    _check_lora("d_w_down", _n(bn.weight_down.grad), d_wd, 2e-2)
    _check_lora("d_w_up", _n(bn.weight_up.grad), d_wu, 2e-2)
    _check_lora("d_bias", _n(bn.bias.grad), d_b)


@pytest.mark.parametrize("pdt", [torch.float32, torch.bfloat16])
def test_group_norm_module(pkg, pdt):
    """GroupNorm.forward (:90-97) on its own over [N, C] (groups of 64), on the HIP kernel
    without the gate: forward and gradients against torch.nn.functional.group_norm in fp64,
    the routine the reference calls."""
    M = pkg.modules
    N, H = 300, 4
    C = 64 * H
    cfg = M.TransformerConfig(hidden_size=C, num_attention_heads=H, params_dtype=pdt)
    gn = M.GroupNorm(cfg, H, C, device=DEV)
    g = torch.Generator().manual_seed(7)
    with torch.no_grad():
        gn.weight.copy_((1 + 0.3 * torch.randn(C, generator=g)).to(pdt))
        gn.bias.copy_((0.2 * torch.randn(C, generator=g)).to(pdt))
    x = _bf(torch.randn(N, C, generator=g) * 2 + 0.5)
    dy = _bf(torch.randn(N, C, generator=g))
    xg = x.to(DEV).requires_grad_(True)
    y = gn(xg)
    (y.float() * dy.to(DEV).float()).sum().backward()
    torch.cuda.synchronize()
    xr = x.double().requires_grad_(True)
    wr = gn.weight.detach().double().cpu().requires_grad_(True)
    br = gn.bias.detach().double().cpu().requires_grad_(True)
    yr = torch.nn.functional.group_norm(xr, H, wr, br, eps=cfg.layernorm_epsilon)
    (yr * dy.double()).sum().backward()
    _check("y", _n(y), yr.detach().numpy())
    _check("dx", _n(xg.grad), xr.grad.numpy())
    _check("dgamma", _n(gn.weight.grad), wr.grad.numpy())
    _check("dbeta", _n(gn.bias.grad), br.grad.numpy())
    with pytest.raises(NotImplementedError):
        M.GroupNorm(cfg, 2 * H, C, device=DEV)(xg)          # 32-channel groups: no kernel


# N = T*B = 10 (a partial 64-token tile), 210 and 520 (several tiles, C > 64); rank 32 (the
# reference's token-shift bottleneck) and 64 (the other rank the kernels take for five mixes,
# compiled with its own step count)
@pytest.mark.parametrize("T,B,C,pdt,R", [(5, 2, 64, torch.float32, 32), (70, 3, 256, torch.float32, 32),
                                         (130, 4, 192, torch.bfloat16, 32),
                                         (70, 3, 256, torch.float32, 64)])
def test_token_shift_mix_forward_backward(pkg, T, B, C, pdt, R):
    g = torch.Generator().manual_seed(C)
    x = _bf(torch.randn(T, B, C, generator=g))
    maa = torch.rand(C, generator=g).to(pdt)
    wd = torch.empty(C, 5, R).uniform_(-0.1, 0.1, generator=g)
    wu = torch.empty(5, R, C).uniform_(-0.1, 0.1, generator=g)
    bias = torch.empty(5, C).uniform_(-1, 1, generator=g).to(pdt)
    dmix = _bf(torch.randn(5, T, B, C, generator=g))
    # the GEMMs run in bf16: give the oracle the same bf16-rounded weights
    wd_b, wu_b = _bf(wd), _bf(wu)
    leaves = [t.to(DEV).requires_grad_(True) for t in (x, maa, wd_b, wu_b, bias)]
    mixes = pkg.timemix.token_shift_mix(*leaves)
    assert len(mixes) == 5 and all(t.is_contiguous() for t in mixes)
    sum((m.float() * d.float()).sum() for m, d in zip(mixes, dmix.to(DEV))).backward()
    mixed = torch.stack(mixes)
    torch.cuda.synchronize()
    xn, maan, wdn, wun, bn = (_n(t) for t in (x, maa, wd_b, wu_b, bias))
    xxx = orc.shift_lerp_fwd(xn, maan)
    m = orc.bottleneck_fwd(xxx, wdn, wun, np.zeros_like(bn))           # [T,B,5,C] without bias
    ref_mixed = orc.ddlerp_fwd(xn, m, bn)
    _check_lora("mixed", _n(mixed), ref_mixed)
    dmn = _n(dmix)
    _, d_m, _, _ = orc.mix_bwd(xn, maan, m, bn, dmn, np.zeros_like(xn))
    d_xxx, d_wd, d_wu, _ = orc.bottleneck_bwd(xxx, wdn, wun, d_m)
    dx, _, d_bias, d_maa = orc.mix_bwd(xn, maan, m, bn, dmn, d_xxx)
    _check_lora("dx", _n(leaves[0].grad), dx)
    _check_lora("d_maa", _n(leaves[1].grad), d_maa)
    _check_lora("d_w_down", _n(leaves[2].grad), d_wd, 2e-2)
    _check_lora("d_w_up", _n(leaves[3].grad), d_wu, 2e-2)
    _check_lora("d_bias", _n(leaves[4].grad), d_bias)


@pytest.mark.parametrize("T,B,C,R", [(5, 2, 64, 64), (70, 3, 256, 64), (33, 2, 128, 32)])
def test_decay_lora_forward_backward(pkg, T, B, C, R):
    """The decay bottleneck (E = 1): tanh(x W_down) W_up + bias with the fused up-projection."""
    g = torch.Generator().manual_seed(T + R)
    x = _bf(torch.randn(T, B, C, generator=g))
    wd = _bf(torch.empty(C, 1, R).uniform_(-0.1, 0.1, generator=g))
    wu = _bf(torch.empty(1, R, C).uniform_(-0.3, 0.3, generator=g))
    bias = torch.empty(1, C).uniform_(-6, -1, generator=g)
    dy = _bf(torch.randn(T, B, C, generator=g))
    leaves = [t.to(DEV).requires_grad_(True) for t in (x, wd, wu, bias)]
    out = pkg.timemix.decay_lora(*leaves)
    (out.float() * dy.to(DEV).float()).sum().backward()
    torch.cuda.synchronize()
    xn, wdn, wun, bn = (_n(t) for t in (x, wd, wu, bias))
    _check_lora("decay", _n(out), orc.bottleneck_fwd(xn, wdn, wun, bn)[:, :, 0])
    dx, d_wd, d_wu, d_b = orc.bottleneck_bwd(xn, wdn, wun, _n(dy)[:, :, None])
    _check_lora("dx", _n(leaves[0].grad), dx, 2e-2)
    _check_lora("d_w_down", _n(leaves[1].grad), d_wd, 2e-2)
    _check_lora("d_w_up", _n(leaves[2].grad), d_wu, 2e-2)
    _check_lora("d_bias", _n(leaves[3].grad), d_b)


@pytest.mark.parametrize("head_first", [True, False])
@pytest.mark.parametrize("pdt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("T,B,H", [(1, 1, 1), (70, 3, 4), (129, 2, 8)])
def test_group_norm_gate(pkg, head_first, pdt, T, B, H):
    K, eps = 64, 1e-5
    C = H * K
    g = torch.Generator().manual_seed(T * 10 + H)
    o_hf = _bf(torch.randn(B, H, T, K, generator=g) * 2 + 0.5)
    gp = _bf(torch.randn(T, B, C, generator=g))
    gamma = (1 + 0.3 * torch.randn(C, generator=g)).to(pdt)
    beta = (0.2 * torch.randn(C, generator=g)).to(pdt)
    dy = _bf(torch.randn(T, B, C, generator=g))
    o_tb = o_hf.permute(2, 0, 1, 3).reshape(T, B, C).contiguous()
    o_in = o_hf if head_first else o_tb
    leaves = [t.to(DEV).requires_grad_(True) for t in (o_in, gp, gamma, beta)]
    y = pkg.timemix.group_norm_gate(leaves[0], leaves[1], leaves[2], leaves[3], eps, head_first=head_first)
    (y.float() * dy.to(DEV).float()).sum().backward()
    torch.cuda.synchronize()
    on = _n(o_tb).reshape(T * B, C)
    y_ref, _, _ = orc.gn_gate_fwd(on, _n(gp).reshape(T * B, C), H, _n(gamma), _n(beta), eps)
    _check("y", _n(y).reshape(T * B, C), y_ref)
    do, dz, dgam, dbet = orc.gn_gate_bwd(on, _n(gp).reshape(T * B, C), H, _n(gamma), _n(beta), eps,
                                         _n(dy).reshape(T * B, C))
    d_o = _n(leaves[0].grad)
    if head_first:
        d_o = np.transpose(d_o, (2, 0, 1, 3))
    _check("d_o", d_o.reshape(T * B, C), do)
    _check("d_g", _n(leaves[1].grad).reshape(T * B, C), dz)
    _check("dgamma", _n(leaves[2].grad), dgam)
    _check("dbeta", _n(leaves[3].grad), dbet)


def test_mix_and_gn_deterministic(pkg):
    T, B, C, H = 200, 3, 256, 4
    g = torch.Generator().manual_seed(1)
    x = _bf(torch.randn(T, B, C, generator=g)).to(DEV)
    params = [torch.rand(C, generator=g), torch.empty(C, 5, 32).uniform_(-0.1, 0.1, generator=g),
              torch.empty(5, 32, C).uniform_(-0.1, 0.1, generator=g), torch.randn(5, C, generator=g)]
    o = _bf(torch.randn(B, H, T, 64, generator=g)).to(DEV)
    gp = _bf(torch.randn(T, B, C, generator=g)).to(DEV)

    def run():
        ps = [p.to(DEV).requires_grad_(True) for p in params]
        xi = x.clone().requires_grad_(True)
        mixed = torch.stack(pkg.timemix.token_shift_mix(xi, *ps))
        gam = torch.ones(C, device=DEV, requires_grad=True)
        bet = torch.zeros(C, device=DEV, requires_grad=True)
        y = pkg.timemix.group_norm_gate(o, gp, gam, bet, 1e-5)
        (mixed.float().sum() + y.float().square().sum()).backward()
        return [mixed, y, xi.grad, gam.grad, bet.grad] + [p.grad for p in ps]

    a, b = run(), run()
    for ta, tb in zip(a, b):
        assert torch.equal(ta, tb)


@pytest.mark.parametrize("layout", ["e_n_r", "n_e_r"])
@pytest.mark.parametrize("N,E,R", [(1, 1, 8), (333, 5, 32), (4096, 1, 64)])
def test_lora_tanh_bwd(pkg, layout, N, E, R):
    """d_pre = d_neck * (1 - neck^2) in the down-projection's [N, E*R] layout, from d_neck laid
    out [E,N,R] (the batched GEMM) or [N,E,R]; against fp64 on the same bf16 inputs."""
    g = torch.Generator().manual_seed(N + E + R)
    neck = _bf(torch.tanh(torch.randn(N, E * R, generator=g)))
    d_ner = _bf(torch.randn(N, E, R, generator=g))
    ref = (d_ner.double() * (1.0 - neck.double().view(N, E, R) ** 2)).reshape(N, E * R)
    if layout == "e_n_r":
        d_in, sE, sN = d_ner.permute(1, 0, 2).contiguous(), N * R, R
    else:
        d_in, sE, sN = d_ner.contiguous(), R, E * R
    got = pkg.timemix.tanh_bwd(d_in.to(DEV), sE, sN, neck.to(DEV), N, E, R)
    torch.cuda.synchronize()
    _check("d_pre", _n(got), ref.numpy())


# (16384, 4096): 1024 blocks, the launch that issues one row at a time; the others eight
@pytest.mark.parametrize("N,M", [(1, 8), (255, 360), (257, 64), (16384, 2048), (16384, 4096)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_col_sum(pkg, N, M, dtype):
    """Column sums of a bf16 [N, M] (a bottleneck's bias gradient over the tokens), ragged N
    and M, both parameter dtypes; bit-identical on a rerun (fixed reduction order)."""
    g = torch.Generator().manual_seed(N + M)
    x = _bf(torch.randn(N, M, generator=g))
    ref = x.double().sum(0).numpy()
    got = pkg.timemix.col_sum(x.to(DEV), dtype)
    again = pkg.timemix.col_sum(x.to(DEV), dtype)
    torch.cuda.synchronize()
    assert got.dtype == dtype and torch.equal(got, again)
    # fp32 sums of N terms of magnitude ~1: error ~ N * 2^-24 * sqrt(N)-scale, well inside the bar
    _check("col_sum", _n(got), ref)


@pytest.mark.parametrize("S,n", [(1, 8), (2, 1000 * 8), (4, 2048 * 2048), (7, 2048 * 160), (64, 24)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_sum_partials(pkg, S, n, dtype):
    """rwkv6_sum_partials against a left-to-right fp32 sum on the host: bit-identical in fp32
    (same additions in the same order), and the bf16 output is that fp32 sum rounded to nearest
    even (torch's own fp32 -> bf16 conversion)."""
    g = torch.Generator().manual_seed(S * 1000 + n)
    part = torch.randn(S, n, generator=g)
    acc = part[0].clone()
    for j in range(1, S):
        acc = acc + part[j]                       # fp32, left to right
    got = pkg.timemix.sum_partials(part.to(DEV), dtype)
    torch.cuda.synchronize()
    assert got.dtype == dtype and got.shape == (n,)
    assert torch.equal(got.cpu(), acc.to(dtype))


def test_sum_partials_rejects_bad_arguments(pkg):
    L = pkg._lib.load()
    x = torch.zeros(2, 16, device=DEV)
    o = torch.empty(16, device=DEV)
    p = lambda t: t.data_ptr()
    s = torch.cuda.current_stream().cuda_stream
    assert L.rwkv6_sum_partials(p(x), 0, 16, 0, p(o), s) == pkg._lib.RWKV6_ERR_INVALID_ARG
    assert L.rwkv6_sum_partials(p(x), 2, 12, 0, p(o), s) == pkg._lib.RWKV6_ERR_UNSUPPORTED
    assert L.rwkv6_sum_partials(p(x), 2, 16, 5, p(o), s) == pkg._lib.RWKV6_ERR_INVALID_ARG
    assert L.rwkv6_sum_partials(p(x), 2, 16, 0, p(x), s) == pkg._lib.RWKV6_ERR_INVALID_ARG   # aliasing


def test_empty_inputs_zero_parameter_gradients(pkg):
    """No tokens: every backward that reduces a parameter gradient over the tokens writes zeros
    (the fixed-order partial sum over zero blocks), and the column sum of an empty matrix is
    zero.  Outputs start as NaN; the token tensors are never read."""
    L = pkg._lib.load()
    E = pkg._lib
    C, H, K = 128, 2, 64
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    sp = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    act = torch.zeros(64, C, dtype=torch.bfloat16, device=DEV)      # stand-in token tensors
    par = torch.zeros(5, C, device=DEV)
    nan = lambda n, dt=torch.float32: torch.full((n,), float("nan"), dtype=dt, device=DEV)
    ws = lambda nbytes: torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=DEV)

    out = nan(C)
    assert L.rwkv6_col_sum(P(act), 0, C, E.RWKV6_F32, P(out), P(ws(L.rwkv6_col_sum_workspace_bytes(0, C))),
                           sp) == E.RWKV6_OK
    d_maa = nan(C)                                                   # fp32, as maa
    assert L.rwkv6_shift_lerp_bwd(P(act), P(par), E.RWKV6_F32, P(act), P(act), P(act), P(act), P(d_maa),
                                  P(ws(L.rwkv6_shift_lerp_bwd_workspace_bytes(0, 2, C))), 0, 2, C,
                                  sp) == E.RWKV6_OK
    d_mix = nan(2 * C)
    dm2 = (ctypes.c_void_p * 2)(act.data_ptr(), act.data_ptr())
    assert L.rwkv6_cmix_lerp_bwd(P(act), P(par), E.RWKV6_F32, ctypes.cast(dm2, ctypes.c_void_p), P(act),
                                 P(d_mix), P(ws(L.rwkv6_cmix_lerp_bwd_workspace_bytes(0, 2, C))), 0, 2, C,
                                 sp) == E.RWKV6_OK
    dgamma, dbeta = nan(H * K), nan(H * K)
    stats = torch.zeros(64, device=DEV)
    assert L.rwkv6_gn_gate_bwd(P(act), 1, P(act), P(par), P(par), E.RWKV6_F32, P(stats), P(stats), P(act),
                               P(act), P(act), P(dgamma), P(dbeta),
                               P(ws(L.rwkv6_gn_gate_bwd_workspace_bytes(0, 2, H, K))), 0, 2, H, K,
                               sp) == E.RWKV6_OK
    d_bias = nan(5 * C)
    dm5 = (ctypes.c_void_p * 5)(*[act.data_ptr()] * 5)
    assert L.rwkv6_ddlerp_lora_bwd(P(act), P(act), P(act), P(par), E.RWKV6_F32,
                                   ctypes.cast(dm5, ctypes.c_void_p), P(act), P(act), P(act), P(d_bias),
                                   P(ws(L.rwkv6_ddlerp_lora_bwd_workspace_bytes(0, 2, C))), 0, 2, C, 32,
                                   sp) == E.RWKV6_OK
    torch.cuda.synchronize()
    for name, t in (("col_sum", out), ("d_maa", d_maa), ("d_mix", d_mix), ("dgamma", dgamma),
                    ("dbeta", dbeta), ("d_bias", d_bias)):
        assert torch.equal(t, torch.zeros_like(t)), name
