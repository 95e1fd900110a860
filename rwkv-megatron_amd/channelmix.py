"""Fused channel-mix building blocks (HIP kernels) as autograd Functions.

RWKV6ChannelMix.forward (/root/reference/rwkv_megatron/rwkv6_layer_specs.py:512-536):

    delta = shift(x) - x                                   :513-516
    mixed_up, mixed_gate = x + delta * mix_coeffs[e]       :517-520
    h = relu(linear_up(mixed_up)) ** 2                     :522-524
    out = linear_down(h)                                   :525
    y = out * sigmoid(linear_gate(mixed_gate))             :528-536

* ``cmix_lerp``: the shift and both lerps in one pass, written as two separate [T,B,C]
  tensors, each a contiguous GEMM operand (the reference's ``unbind`` + ``.contiguous()``
  copies, and the stack of their gradients, disappear).  Its backward is one pass
  producing dx and d mix_coeffs from the two gradients where they lie.
* ``relu_sq`` and ``sigmoid_gate``: single-pass epilogues with single-pass backwards.

The projections stay on hipBLASLt (torch.nn.functional.linear).  Every function raises
if the HIP library is missing; there is no fallback.
"""
from __future__ import annotations

import torch

from . import _lib
from .timemix import _c, _check_act, _p, _param, _ptrs, _stream

NE = 2  # (up, gate)


class _CmixLerp(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, mix):
        T, B, C = x.shape
        x = _c(x)
        m, pdt = _param(mix)
        mixed = tuple(torch.empty(T, B, C, dtype=torch.bfloat16, device=x.device) for _ in range(NE))
        _lib.check(_lib.load().rwkv6_cmix_lerp_fwd(_p(x), _p(m), pdt, _ptrs(mixed), T, B, C,
                                                   _stream(x.device)), "rwkv6_cmix_lerp_fwd")
        ctx.save_for_backward(x, m)
        ctx.pdt, ctx.mix_dtype = pdt, mix.dtype
        return mixed

    @staticmethod
    def backward(ctx, *d_mixed):
        x, m = ctx.saved_tensors
        T, B, C = x.shape
        L = _lib.load()
        d_mixed = [torch.zeros_like(x) if d is None else _c(d.to(torch.bfloat16)) for d in d_mixed]
        dx = torch.empty_like(x)
        d_mix = torch.empty(NE, C, dtype=m.dtype, device=x.device)
        ws = torch.empty(L.rwkv6_cmix_lerp_bwd_workspace_bytes(T, B, C), dtype=torch.uint8,
                         device=x.device)
        _lib.check(L.rwkv6_cmix_lerp_bwd(_p(x), _p(m), ctx.pdt, _ptrs(d_mixed), _p(dx), _p(d_mix),
                                         _p(ws), T, B, C, _stream(x.device)), "rwkv6_cmix_lerp_bwd")
        return dx, d_mix.to(ctx.mix_dtype)


def cmix_lerp(x: torch.Tensor, mix: torch.Tensor) -> torch.Tensor:
    """[T,B,C] bf16, mix_coeffs [2,C] -> (mixed_up, mixed_gate), each [T,B,C] (the inputs of
    linear_up and linear_gate)."""
    _check_act("x", x, 3)
    if tuple(mix.shape) != (NE, x.shape[-1]):
        raise ValueError(f"mix must be [2,C] = {(NE, x.shape[-1])}, got {tuple(mix.shape)}")
    if x.shape[-1] % 8:
        raise NotImplementedError("C must be a multiple of 8")
    return _CmixLerp.apply(x, mix)


def _n_check(*ts):
    for t in ts:
        if t.device.type != "cuda" or t.dtype != torch.bfloat16:
            raise TypeError("channel-mix epilogues take bfloat16 CUDA tensors")
        if t.shape != ts[0].shape:
            raise ValueError("operand shapes differ")
    if ts[0].numel() % 8:
        raise NotImplementedError("element count must be a multiple of 8")


class _ReluSq(torch.autograd.Function):
    @staticmethod
    def forward(ctx, up):
        up = _c(up)
        h = torch.empty_like(up)
        _lib.check(_lib.load().rwkv6_relu_sq_fwd(_p(up), _p(h), up.numel(), _stream(up.device)),
                   "rwkv6_relu_sq_fwd")
        ctx.save_for_backward(up)
        return h

    @staticmethod
    def backward(ctx, dh):
        (up,) = ctx.saved_tensors
        dh = _c(dh.to(torch.bfloat16))
        d_up = torch.empty_like(up)
        _lib.check(_lib.load().rwkv6_relu_sq_bwd(_p(up), _p(dh), _p(d_up), up.numel(),
                                                 _stream(up.device)), "rwkv6_relu_sq_bwd")
        return d_up


def relu_sq(up: torch.Tensor) -> torch.Tensor:
    """square(relu(up)) (rwkv6_layer_specs.py:524), bf16 in and out, fp32 inside."""
    _n_check(up)
    return _ReluSq.apply(up)


class _SigmoidGate(torch.autograd.Function):
    @staticmethod
    def forward(ctx, out, gate_pre):
        out, gate_pre = _c(out), _c(gate_pre)
        y = torch.empty_like(out)
        _lib.check(_lib.load().rwkv6_sigmoid_gate_fwd(_p(out), _p(gate_pre), _p(y), out.numel(),
                                                      _stream(out.device)), "rwkv6_sigmoid_gate_fwd")
        ctx.save_for_backward(out, gate_pre)
        return y

    @staticmethod
    def backward(ctx, dy):
        out, gate_pre = ctx.saved_tensors
        dy = _c(dy.to(torch.bfloat16))
        d_out, d_gp = torch.empty_like(out), torch.empty_like(gate_pre)
        _lib.check(_lib.load().rwkv6_sigmoid_gate_bwd(_p(out), _p(gate_pre), _p(dy), _p(d_out),
                                                      _p(d_gp), out.numel(), _stream(out.device)),
                   "rwkv6_sigmoid_gate_bwd")
        return d_out, d_gp


def sigmoid_gate(out: torch.Tensor, gate_pre: torch.Tensor) -> torch.Tensor:
    """out * sigmoid(gate_pre) (rwkv6_layer_specs.py:533-536), bf16 in and out."""
    _n_check(out, gate_pre)
    return _SigmoidGate.apply(out, gate_pre)
