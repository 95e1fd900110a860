"""End-to-end drop-in check of RWKV6TimeMix on the GPU against a CPU restatement of
the reference's forward (rwkv6_layer_specs.py:431-468) in torch fp32, with the WKV
of :339 provided by the CPU oracle through a small autograd wrapper.

Block-level tolerance: relative L2 <= 3e-2 and max|err|/max|ref| <= 5e-2 — the GPU
path keeps activations in bf16 between the GEMMs (as bf16 training does); every
kernel on it is pinned separately at 1e-2.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as orc

pytestmark = pytest.mark.gpu


class _OracleWKV(torch.autograd.Function):
    @staticmethod
    def forward(ctx, r, k, v, w, u):
        n = lambda t: t.detach().float().numpy()
        o, _ = orc.wkv6_fwd(n(r), n(k), n(v), n(w), n(u), None, 1.0)
        ctx.save_for_backward(r, k, v, w, u)
        return torch.from_numpy(o)

    @staticmethod
    def backward(ctx, do):
        n = lambda t: t.detach().float().numpy()
        r, k, v, w, u = ctx.saved_tensors
        g = orc.wkv6_bwd(n(r), n(k), n(v), n(w), n(u), n(do), None, None, 1.0)
        return tuple(torch.from_numpy(g[x]) for x in ("dr", "dk", "dv", "dw", "du"))


def reference_timemix(p, x, H, eps):
    """rwkv6_layer_specs.py:440-466 on CPU in fp32 (TP=1, no sequence parallel)."""
    shifted = torch.cat([torch.zeros_like(x.select(0, 0)).unsqueeze(0), x.narrow(0, 0, x.size(0) - 1)], 0)
    delta = shifted - x
    mixed_input = x + delta * p["mix_coeff_input"]
    def bottleneck(z, pre):
        neck = torch.einsum("tbd,der->tber", z, p[pre + ".weight_down"]).tanh()
        return torch.einsum("tber,erd->tbed", neck, p[pre + ".weight_up"]) + p[pre + ".bias"]
    mix = bottleneck(mixed_input, "bottleneck_token_shift")
    ddm = x.unsqueeze(-2) + delta.unsqueeze(-2) * mix
    m_w, m_k, m_v, m_r, m_g = ddm.unbind(-2)
    decay = bottleneck(m_w, "bottleneck_decay").squeeze(-2)
    key = m_k @ p["linear_key.weight"].t()
    value = m_v @ p["linear_value.weight"].t()
    rec = m_r @ p["linear_receptance.weight"].t()
    gate = F.silu(m_g @ p["linear_gate.weight"].t())
    T, B, C = x.shape
    hf = lambda t: t.reshape(T, B, H, C // H).permute(1, 2, 0, 3).contiguous()
    o = _OracleWKV.apply(hf(rec), hf(key), hf(value), hf(decay).exp().neg(),
                         p["core_attention.time_first"].reshape(H, -1))
    o = o.permute(2, 0, 1, 3).reshape(T * B, C)
    y = F.group_norm(o, H, p["group_norm.weight"], p["group_norm.bias"], eps=eps).reshape(T, B, C)
    return (y * gate) @ p["linear_proj.weight"].t()


def _err(a, b):
    a, b = a.double(), b.double()
    return ((a - b).abs().max() / b.abs().max()).item(), ((a - b).norm() / b.norm()).item()


@pytest.mark.parametrize("params_dtype", [torch.float32, torch.bfloat16])
def test_timemix_module_matches_reference_forward(pkg, params_dtype):
    M = pkg.modules
    cfg = M.TransformerConfig(hidden_size=256, num_attention_heads=4, ffn_hidden_size=896,
                              num_layers=2, params_dtype=params_dtype)
    torch.manual_seed(0)
    mod = M.RWKV6TimeMix(cfg, layer_number=1, device="cuda:0")
    with torch.no_grad():   # make the data-dependent paths matter
        for bn in (mod.bottleneck_token_shift, mod.bottleneck_decay):
            bn.weight_down.uniform_(-0.1, 0.1)
            bn.weight_up.uniform_(-0.1, 0.1)
        mod.group_norm.weight.normal_(1.0, 0.2)
        mod.group_norm.bias.normal_(0.0, 0.2)
    T, B, C = 100, 2, 256
    g = torch.Generator().manual_seed(1)
    x = torch.randn(T, B, C, generator=g).to(torch.bfloat16)
    dy = torch.randn(T, B, C, generator=g).to(torch.bfloat16)
    xg = x.to("cuda:0").requires_grad_(True)
    out, bias = mod(xg, None)
    assert bias is None and out.shape == (T, B, C)
    (out.float() * dy.to("cuda:0").float()).sum().backward()
    torch.cuda.synchronize()

    p = {n: t.detach().float().cpu().requires_grad_(True) for n, t in mod.named_parameters()}
    xc = x.float().requires_grad_(True)
    ref = reference_timemix(p, xc, cfg.num_attention_heads, cfg.layernorm_epsilon)
    (ref * dy.float()).sum().backward()

    e = _err(out.float().cpu(), ref.detach())
    print("out", e)
    assert e[0] < 5e-2 and e[1] < 3e-2
    e = _err(xg.grad.float().cpu(), xc.grad)
    print("dx", e)
    assert e[0] < 5e-2 and e[1] < 3e-2
    for name, prm in mod.named_parameters():
        e = _err(prm.grad.float().cpu(), p[name].grad)
        print(name, e)
        assert e[1] < 3e-2 and e[0] < 5e-2, name


def test_state_dict_contract(pkg):
    """Parameter names and shapes of the reference's TimeMix/ChannelMix (TP = 1)."""
    M = pkg.modules
    cfg = M.TransformerConfig(hidden_size=128, num_attention_heads=2, ffn_hidden_size=448, num_layers=1)
    tm = M.RWKV6TimeMix(cfg, 1, device="cuda:0")
    shapes = {n: tuple(t.shape) for n, t in tm.state_dict().items()}
    C = 128
    assert shapes == {
        "bottleneck_token_shift.weight_down": (C, 5, 32), "bottleneck_token_shift.weight_up": (5, 32, C),
        "bottleneck_token_shift.bias": (5, C), "bottleneck_decay.weight_down": (C, 1, 64),
        "bottleneck_decay.weight_up": (1, 64, C), "bottleneck_decay.bias": (1, C),
        "mix_coeff_input": (C,), "linear_receptance.weight": (C, C), "linear_key.weight": (C, C),
        "linear_value.weight": (C, C), "linear_gate.weight": (C, C),
        "core_attention.time_first": (C,), "group_norm.weight": (C,), "group_norm.bias": (C,),
        "linear_proj.weight": (C, C)}
    cm = M.RWKV6ChannelMix(cfg, 1, device="cuda:0")
    assert {n: tuple(t.shape) for n, t in cm.state_dict().items()} == {
        "mix_coeffs": (2, C), "linear_up.weight": (448, C), "linear_gate.weight": (C, C),
        "linear_down.weight": (C, 448)}
