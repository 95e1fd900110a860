"""CPU restatement of the RWKV-6 language model of RWKV-Megatron (TEST INFRASTRUCTURE ONLY).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this module: it is a checker and a CPU baseline, never the product.

torch-CPU code shaped like the reference's own forward (cat-based token shift, the einsum
patterns of the bottleneck, ``unbind`` of the mixes, ``torch.nn.functional.group_norm``),
written against the parameter names of the reference's modules (which the package keeps),
in any float dtype (fp64 for parity, fp32 for the CPU baseline).  The WKV of :339 is the C
oracle (fp64 recurrence) behind an autograd Function, so torch.autograd gives the backward
of the whole model:

  token shift            rwkv6_layer_specs.py:290-300
  RWKV6Bottleneck        :177-195
  RWKV6TimeMix.forward   :431-468 (WKV6 layout glue :330-341)
  RWKV6ChannelMix        :512-536
  layer (pre-LN residual, dropout 0; get_rwkv6_layer_spec) :539-550
  RWKV6Model             rwkv6_model.py:28-37, :108-112 (embedding, pre_norm, layers, final
                         LayerNorm, untied output head: example_config.yaml:184-185)
  loss                   pretrain_rwkv6.py:144-160 (masked sum of per-token CE / token count)

Pinned in tests/test_oracle.py: the model forward against tests/rwkv_lm_reference.py (an fp64
numpy forward written against RWKV-LM's own parameter names, from the numpy oracle pieces),
the WKV autograd wrapper against the C oracle's forward and backward, and the loss against
torch.nn.functional.cross_entropy.

``bf16_storage()`` turns the same functions into an emulation of the reference as it runs in
bf16 on a GPU: every op computes in the tensors' own (higher) precision and its output is
rounded to bf16 once, and so is the gradient reaching each op's output in the backward (the
storage points of bf16 autograd; fla's WKV computes in fp32 and returns bf16; the gradients of
a tensor that several ops read are summed unrounded where they meet).  Its error
against the plain fp64 run is the rounding error the reference itself carries in bf16, which
the block tests use as the scale of an acceptable error.  (torch's own bf16 CPU kernels are
not that reference: some accumulate in bf16.)
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from . import oracle as orc

_ROUND = [False]


class _RoundBF16(torch.autograd.Function):
    """Rounds a tensor to bf16 (keeping its dtype) and the gradient flowing back through it."""

    @staticmethod
    def forward(ctx, t):
        return t.to(torch.bfloat16).to(t.dtype)

    @staticmethod
    def backward(ctx, g):
        return g.to(torch.bfloat16).to(g.dtype)


def rb(t):
    """A bf16 storage point: identity unless inside bf16_storage()."""
    return _RoundBF16.apply(t) if _ROUND[0] else t


class bf16_storage:
    """Context manager: the functions of this module round at every op boundary (above)."""

    def __enter__(self):
        _ROUND[0] = True
        return self

    def __exit__(self, *exc):
        _ROUND[0] = False


class OracleWKV(torch.autograd.Function):
    """fla's RWKV-6 op as the reference calls it (:339, scale 1): r, k, v, w [B,H,T,64],
    u [H,64] -> o [B,H,T,64], on the C oracle (fp64 recurrence, exact reverse backward)."""

    @staticmethod
    def forward(ctx, r, k, v, w, u):
        n = lambda t: t.detach().double().numpy()
        o, _ = orc.wkv6_fwd(n(r), n(k), n(v), n(w), n(u), None, 1.0)
        ctx.save_for_backward(r, k, v, w, u)
        return torch.from_numpy(np.asarray(o)).to(r.dtype)

    @staticmethod
    def backward(ctx, do):
        n = lambda t: t.detach().double().numpy()
        r, k, v, w, u = ctx.saved_tensors
        g = orc.wkv6_bwd(n(r), n(k), n(v), n(w), n(u), n(do), None, None, 1.0)
        return tuple(torch.from_numpy(np.asarray(g[x])).to(t.dtype)
                     for x, t in zip(("dr", "dk", "dv", "dw", "du"), (r, k, v, w, u)))


def token_shift(x):
    """:290-300 (no sequence parallelism): x[t-1], zeros at t = 0, along dim 0 of [T,B,C]."""
    return torch.cat([torch.zeros_like(x.narrow(0, 0, 1)), x.narrow(0, 0, x.shape[0] - 1)], 0)


def bottleneck(p, pre, z):
    """RWKV6Bottleneck.forward (:177-195, TP = 1): [T,B,C] -> [T,B,E,C]."""
    neck = rb(rb(torch.einsum("tbd,der->tber", z, p[pre + ".weight_down"])).tanh())
    return rb(rb(torch.einsum("tber,erd->tbed", neck, p[pre + ".weight_up"])) + p[pre + ".bias"])


def linear(p, name, x):
    """Column/RowParallelLinear at TP = 1: x W^T, plus the bias when the layer has one
    (add_bias_linear / add_qkv_bias, :393, :416, :484-505)."""
    y = rb(x @ p[name + ".weight"].t())
    b = p.get(name + ".bias")
    return y if b is None else rb(y + b)


def time_mix(p, x, H, eps):
    """RWKV6TimeMix.forward (:440-466); p maps the module's parameter names to tensors.  The
    output projection's bias, which the reference hands back separately (skip_bias_add, :418)
    for the layer's bias-dropout-add, is included in the returned output."""
    delta = rb(token_shift(x) - x)
    mixed_input = rb(x + rb(delta * p["mix_coeff_input"]))
    mix = bottleneck(p, "bottleneck_token_shift", mixed_input)
    m_w, m_k, m_v, m_r, m_g = rb(x.unsqueeze(-2) + rb(delta.unsqueeze(-2) * mix)).unbind(-2)
    decay = bottleneck(p, "bottleneck_decay", m_w).squeeze(-2)
    key = linear(p, "linear_key", m_k)
    value = linear(p, "linear_value", m_v)
    rec = linear(p, "linear_receptance", m_r)
    gate = rb(F.silu(linear(p, "linear_gate", m_g)))
    T, B, C = x.shape
    hf = lambda t: t.reshape(T, B, H, C // H).permute(1, 2, 0, 3).contiguous()   # :333-336
    o = rb(OracleWKV.apply(hf(rec), hf(key), hf(value), -rb(torch.exp(hf(decay))),
                           p["core_attention.time_first"].reshape(H, -1)))
    o = o.permute(2, 0, 1, 3).reshape(T * B, C)                                    # :341, :462
    y = rb(F.group_norm(o, H, p["group_norm.weight"], p["group_norm.bias"], eps=eps)).reshape(T, B, C)
    return linear(p, "linear_proj", rb(y * gate))


def channel_mix(p, x):
    """RWKV6ChannelMix.forward (:512-536)."""
    delta = rb(token_shift(x) - x)
    mixed_up, mixed_gate = rb(x.unsqueeze(-2) + rb(delta.unsqueeze(-2) * p["mix_coeffs"])).unbind(-2)
    h = rb(torch.square(torch.relu(linear(p, "linear_up", mixed_up))))
    out = linear(p, "linear_down", h)
    return rb(out * rb(torch.sigmoid(linear(p, "linear_gate", mixed_gate))))


def _sub(p, prefix):
    return {k[len(prefix):]: v for k, v in p.items() if k.startswith(prefix)}


def layer(p, x, H, eps):
    """The TransformerLayer of get_rwkv6_layer_spec() (:539-550): pre-LN residual blocks."""
    C = x.shape[-1]
    ln = lambda z, n: rb(F.layer_norm(z, (C,), p[n + ".weight"], p[n + ".bias"], eps))
    x = rb(x + time_mix(_sub(p, "self_attention."), ln(x, "input_layernorm"), H, eps))
    return rb(x + channel_mix(_sub(p, "mlp."), ln(x, "pre_mlp_layernorm")))


def model_forward(p, tokens, n_layers, H, eps=1e-5):
    """RWKV6Model (rwkv6_model.py:28-37, :108-112): tokens [B,T] -> logits [T,B,V]."""
    C = p["embedding.weight"].shape[1]
    ln = lambda z, n: rb(F.layer_norm(z, (C,), p[n + ".weight"], p[n + ".bias"], eps))
    x = ln(rb(p["embedding.weight"][tokens.t()]), "pre_norm")
    for i in range(n_layers):
        x = layer(_sub(p, f"layers.{i}."), x, H, eps)
    return rb(ln(x, "final_layernorm") @ p["output_layer.weight"].t())


def lm_loss(logits, targets, loss_mask):
    """pretrain_rwkv6.py:144-160: per-token cross entropy (Megatron's vocab-parallel CE at
    TP = 1), summed under the loss mask and divided by the number of unmasked tokens.
    logits [T,B,V], targets and loss_mask [B,T]."""
    V = logits.shape[-1]
    flat = logits.transpose(0, 1).reshape(-1, V)
    losses = F.cross_entropy(flat.to(torch.promote_types(flat.dtype, torch.float32)),
                             targets.reshape(-1), reduction="none")
    mask = loss_mask.reshape(-1).to(losses.dtype)
    return (losses * mask).sum() / mask.sum()


def params_from_state_dict(sd, dtype=torch.float64, requires_grad=True):
    """A module state_dict (any device/dtype) as CPU leaf tensors of `dtype`."""
    return {k: v.detach().to("cpu", dtype).clone().requires_grad_(requires_grad) for k, v in sd.items()}
