"""Full-width RWKV-6 layers on the GPU at the widths of BASELINE configs 3 (1.6B shape:
C=2048, 32 heads, ffn 7168, B=4 x T=4096) and 4 (7B shape: C=4096, 64 heads, ffn 14336,
B=2 x T=8192).

* Parity: one RWKV6Layer (LN -> time mix -> residual -> LN -> channel mix -> residual,
  rwkv6_layer_specs.py:431-468, :512-536, :539-550) at the full width and a short ragged
  T = 130, B = 2, forward and every gradient, against oracle/lm.py in fp64 on the same
  (bf16) weights.  The residual carries x through unchanged, so the block's own output
  y - x and the input gradient's non-identity part dx - dy are compared.  Bars for a block
  that keeps bf16 activations between hipBLASLt GEMMs (as bf16 training does; every kernel
  on it is pinned separately at 1e-2): parity.BLOCK_BARS (max_rel 1e-1, l2_rel 3e-2,
  reference-metric mean 3e-1), and a relative L2 error at most 1.5x that of the same layer
  restated in bf16 storage (lm.bf16_storage(): the reference as it runs in bf16) plus 2e-3.
* Full shape: the same layer over the config's whole T x B: finite, bit-identical on a
  second run, and a gradient for every parameter.
"""
import pytest
import torch

import parity
from oracle import lm

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

# name: (C, H, F, B, T)
WIDTHS = {"config3": (2048, 32, 7168, 4, 4096), "config4": (4096, 64, 14336, 2, 8192)}
BARS = parity.BLOCK_BARS


def _layer(pkg, C, H, F):
    M = pkg.modules
    cfg = M.TransformerConfig(hidden_size=C, num_attention_heads=H, ffn_hidden_size=F,
                              num_layers=4, params_dtype=torch.bfloat16)
    torch.manual_seed(0)
    layer = M.RWKV6Layer(cfg, layer_number=2, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(1)
    with torch.no_grad():          # make the data-dependent paths matter
        tm = layer.self_attention
        for bn in (tm.bottleneck_token_shift, tm.bottleneck_decay):
            bn.weight_down.uniform_(-0.1, 0.1, generator=g)
            bn.weight_up.uniform_(-0.1, 0.1, generator=g)
        tm.group_norm.weight.normal_(1.0, 0.2, generator=g)
        tm.group_norm.bias.normal_(0.0, 0.2, generator=g)
        for ln in (layer.input_layernorm, layer.pre_mlp_layernorm):
            ln.weight.normal_(1.0, 0.1, generator=g)
            ln.bias.normal_(0.0, 0.1, generator=g)
    return cfg, layer


@pytest.mark.parametrize("cfg_name", list(WIDTHS))
def test_full_width_layer_parity(pkg, cfg_name):
    C, H, F, _, _ = WIDTHS[cfg_name]
    T, B = 130, 2
    print(f"{cfg_name}: one layer C={C} H={H} F={F}, T={T} B={B}", flush=True)
    cfg, layer = _layer(pkg, C, H, F)
    g = torch.Generator().manual_seed(2)
    x = torch.randn(T, B, C, generator=g).to(torch.bfloat16)
    dy = torch.randn(T, B, C, generator=g).to(torch.bfloat16)
    xg = x.to(DEV).requires_grad_(True)
    out = layer(xg)
    out.backward(dy.to(DEV))
    torch.cuda.synchronize()

    def reference(storage):
        p = lm.params_from_state_dict(layer.state_dict())
        xr = x.double().requires_grad_(True)
        if storage:
            with lm.bf16_storage():
                y = lm.layer(p, xr, H, cfg.layernorm_epsilon)
                y.backward(dy.double())
        else:
            y = lm.layer(p, xr, H, cfg.layernorm_epsilon)
            y.backward(dy.double())
        # parameter gradients are stored in the parameters' dtype (bf16) by both
        grads = {k: t.grad.to(torch.bfloat16) if storage else t.grad for k, t in p.items()}
        return y, xr.grad, grads

    ref, ref_dx, ref_g = reference(False)
    emu, emu_dx, emu_g = reference(True)

    n = lambda t: t.detach().double().cpu().numpy()
    # out and dx are stored in bf16, rounded at the scale of x and dy (2^-9 of it), while the
    # block's own parts y - x and dx - dy are several times smaller: their errors carry that
    # storage rounding on top of the block's own
    parity.check_block("y - x", n(out) - n(x), n(ref) - n(x), n(emu) - n(x), **BARS)
    parity.check_block("dx - dy", n(xg.grad) - n(dy), n(ref_dx) - n(dy), n(emu_dx) - n(dy), **BARS)
    got = {name: n(prm.grad) for name, prm in layer.named_parameters()}
    parity.check_all_block(got, {k: n(ref_g[k]) for k in got}, {k: n(emu_g[k]) for k in got},
                           sorted(got), **BARS)


@pytest.mark.parametrize("cfg_name", list(WIDTHS))
def test_full_shape_layer_properties(pkg, cfg_name):
    C, H, F, B, T = WIDTHS[cfg_name]
    print(f"{cfg_name}: one layer C={C} H={H} F={F}, full T={T} B={B}", flush=True)
    _, layer = _layer(pkg, C, H, F)
    g = torch.Generator(device=DEV).manual_seed(3)
    x = torch.randn(T, B, C, device=DEV, generator=g).to(torch.bfloat16)
    dy = torch.randn(T, B, C, device=DEV, generator=g).to(torch.bfloat16)

    def run():
        xg = x.clone().requires_grad_(True)
        out = layer(xg)
        out.backward(dy)
        grads = {name: prm.grad.clone() for name, prm in layer.named_parameters()}
        for prm in layer.parameters():
            prm.grad = None
        return out.detach(), xg.grad, grads

    a, b = run(), run()
    torch.cuda.synchronize()
    assert torch.isfinite(a[0].float()).all() and torch.isfinite(a[1].float()).all()
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    assert len(a[2]) == len(list(layer.parameters()))
    for name, gr in a[2].items():
        assert torch.isfinite(gr.float()).all(), name
        assert gr.abs().max() > 0, name
        assert torch.equal(gr, b[2][name]), name
