"""Drop-in for fla's RWKV-6 ops, backed by the HIP kernels of librwkv6_amd.so.

The reference calls ``fused_recurrent_rwkv6(r, k, v, w, u, scale=1.)[0]`` at
/root/reference/rwkv_megatron/rwkv6_layer_specs.py:339 after laying its
tensors out head-first (:333-337).  fla also exports ``chunk_rwkv6`` with the
same contract (4th argument named ``g``).  Both names are provided here:

    o, final_state = chunk_rwkv6(r, k, v, g, u, scale=None, initial_state=None,
                                 output_final_state=False)

* r, k, g(=w): [B,H,T,K]; v: [B,H,T,V]; u: [H,K]; K == V == 64.
* g / w is LOG-space decay (the caller passes ``-exp(decay)``, :336).
* scale None or -1 means K**-0.5 (fla's convention); any other float is used as is.
* initial_state: [B,H,K,V] (computed in fp32); final_state is fp32 or None.
* o has r's dtype.  Arithmetic: bf16 operands on MFMA, fp32 accumulation and fp32
  carried state.  bf16 r, k, v, g are used as they are; fp32 / fp16 ones are rounded to
  bf16 on entry (one rounding each, 2^-9 relative), so an fp32 caller gets bf16-operand
  arithmetic, not fp32 arithmetic.  u is used in its own dtype (fp32 or bf16).
* Backward returns gradients for r, k, v, g, u and initial_state, and accepts a
  gradient on final_state.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

_HEAD = 64


def _stream_ptr(device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _p(t):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _aligned(t: torch.Tensor) -> torch.Tensor:
    t = t.contiguous()
    if t.data_ptr() % 16:
        t = t.clone()
    return t


def _bf16(t: torch.Tensor) -> torch.Tensor:
    return _aligned(t if t.dtype == torch.bfloat16 else t.to(torch.bfloat16))


def _u_arg(u: torch.Tensor):
    if u.dtype == torch.bfloat16:
        return _aligned(u), _lib.RWKV6_BF16
    return _aligned(u.float()), _lib.RWKV6_F32


class _WKV6(torch.autograd.Function):
    @staticmethod
    def forward(ctx, r, k, v, w, u, scale, h0, output_final_state):
        B, H, T, K = r.shape
        V = v.shape[-1]
        dev = r.device
        out_dtype = r.dtype
        rb, kb, vb, wb = _bf16(r), _bf16(k), _bf16(v), _bf16(w)
        ua, u_code = _u_arg(u)
        h0f = None if h0 is None else _aligned(h0.float())
        L = _lib.load()
        saved = torch.empty(L.rwkv6_wkv_saved_bytes(B, H, T, K, V), dtype=torch.uint8, device=dev)
        work = torch.empty(L.rwkv6_wkv_workspace_bytes(B, H, T, K, V, 0), dtype=torch.uint8, device=dev)
        o = torch.empty(B, H, T, V, dtype=torch.bfloat16, device=dev)
        hT = torch.empty(B, H, K, V, dtype=torch.float32, device=dev) if output_final_state else None
        _lib.check(L.rwkv6_wkv_fwd(_p(rb), _p(kb), _p(vb), _p(wb), _p(ua), u_code, _p(h0f), _p(o),
                                   _p(hT), _p(saved), _p(work), B, H, T, K, V, float(scale),
                                   _stream_ptr(dev)), "rwkv6_wkv_fwd")
        ctx.save_for_backward(rb, kb, vb, wb, ua, saved)
        ctx.meta = (scale, u_code, h0 is not None, u.dtype, out_dtype, r.dtype, k.dtype, v.dtype,
                    w.dtype, None if h0 is None else h0.dtype)
        if out_dtype != torch.bfloat16:
            o = o.to(out_dtype)
        return o, hT

    @staticmethod
    def backward(ctx, do, dht):
        rb, kb, vb, wb, ua, saved = ctx.saved_tensors
        scale, u_code, has_h0, u_dtype, _, r_dt, k_dt, v_dt, w_dt, h0_dt = ctx.meta
        B, H, T, K = rb.shape
        V = vb.shape[-1]
        dev = rb.device
        L = _lib.load()
        dob = _bf16(do) if do is not None else torch.zeros(B, H, T, V, dtype=torch.bfloat16, device=dev)
        dhtf = None if dht is None else _aligned(dht.float())
        dr = torch.empty_like(rb)
        dk = torch.empty_like(kb)
        dv = torch.empty_like(vb)
        dw = torch.empty_like(wb)
        du = torch.empty(H, K, dtype=ua.dtype, device=dev)
        need_h0 = has_h0 and ctx.needs_input_grad[6]
        dh0 = torch.empty(B, H, K, V, dtype=torch.float32, device=dev) if need_h0 else None
        work = torch.empty(L.rwkv6_wkv_workspace_bytes(B, H, T, K, V, 1), dtype=torch.uint8, device=dev)
        _lib.check(L.rwkv6_wkv_bwd(_p(rb), _p(kb), _p(vb), _p(wb), _p(ua), u_code, _p(dob), _p(dhtf),
                                   _p(saved), _p(dr), _p(dk), _p(dv), _p(dw), _p(du), _p(dh0), _p(work),
                                   B, H, T, K, V, float(scale), _stream_ptr(dev)), "rwkv6_wkv_bwd")
        cast = lambda t, dt: t if t.dtype == dt else t.to(dt)
        return (cast(dr, r_dt), cast(dk, k_dt), cast(dv, v_dt), cast(dw, w_dt), cast(du, u_dtype),
                None, None if dh0 is None else cast(dh0, h0_dt), None)


def _validate(r, k, v, w, u, initial_state):
    for name, t in (("r", r), ("k", k), ("v", v), ("w", w), ("u", u)):
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor")
        if t.device.type != "cuda":
            raise ValueError(f"{name} must live on the GPU (got {t.device})")
        if t.dtype not in (torch.bfloat16, torch.float16, torch.float32):
            raise TypeError(f"{name}: unsupported dtype {t.dtype}")
    if r.dim() != 4:
        raise ValueError(f"r must be [B,H,T,K], got shape {tuple(r.shape)}")
    B, H, T, K = r.shape
    if k.shape != r.shape or w.shape != r.shape:
        raise ValueError(f"k and w must match r's shape {tuple(r.shape)}")
    if v.dim() != 4 or v.shape[:3] != r.shape[:3]:
        raise ValueError(f"v must be [B,H,T,V] with B,H,T of r, got {tuple(v.shape)}")
    V = v.shape[-1]
    if u.shape != (H, K):
        raise ValueError(f"u must be [H,K] = {(H, K)}, got {tuple(u.shape)}")
    if K != _HEAD or V != _HEAD:
        raise NotImplementedError(f"head size must be K == V == {_HEAD}, got K={K}, V={V}")
    if initial_state is not None and tuple(initial_state.shape) != (B, H, K, V):
        raise ValueError(f"initial_state must be [B,H,K,V] = {(B, H, K, V)}")
    devs = {t.device for t in (r, k, v, w, u)}
    if initial_state is not None:
        devs.add(initial_state.device)
    if len(devs) != 1:
        raise ValueError("all tensors must be on the same device")


def chunk_rwkv6(r, k, v, g, u, scale=None, initial_state=None, output_final_state=False,
                checkpoint_level=None, cu_seqlens=None, head_first=True):
    """RWKV-6 WKV, fla ``chunk_rwkv6`` contract.  Returns ``(o, final_state or None)``."""
    if cu_seqlens is not None:
        raise NotImplementedError("variable-length batches (cu_seqlens) are not supported")
    if not head_first:
        raise NotImplementedError("only the head-first [B,H,T,K] layout is supported")
    _validate(r, k, v, g, u, initial_state)
    if scale is None or scale == -1:
        scale = r.shape[-1] ** -0.5
    return _WKV6.apply(r, k, v, g, u, float(scale), initial_state, bool(output_final_state))


def fused_recurrent_rwkv6(r, k, v, w, u, scale=-1, initial_state=None, output_final_state=False,
                          causal=True, cu_seqlens=None, head_first=True):
    """RWKV-6 WKV, fla ``fused_recurrent_rwkv6`` contract (the name the reference imports at
    rwkv6_layer_specs.py:47 and calls at :339).  Same kernels as ``chunk_rwkv6``."""
    if not causal:
        raise NotImplementedError("only causal RWKV-6 is defined")
    return chunk_rwkv6(r, k, v, w, u, scale=scale, initial_state=initial_state,
                       output_final_state=output_final_state, cu_seqlens=cu_seqlens,
                       head_first=head_first)


class _WKV6SeqFirst(torch.autograd.Function):
    """WKV6 on the time-mix module's own layout: r, k, v, decay [T,B,H*64] bf16 (the linear
    outputs, rwkv6_layer_specs.py:454-457), w = -exp(decay) (:336) applied in the kernels,
    output o head-first [B,H,T,64] (what GroupNorm*gate reads)."""

    @staticmethod
    def forward(ctx, r, k, v, decay, u, scale, H, h0, output_final_state):
        T, B, C = r.shape
        K = C // H
        dev = r.device
        rb, kb, vb, db = _bf16(r), _bf16(k), _bf16(v), _bf16(decay)
        ua, u_code = _u_arg(u)
        h0f = None if h0 is None else _aligned(h0.float())
        L = _lib.load()
        saved = torch.empty(L.rwkv6_wkv_saved_bytes(B, H, T, K, K), dtype=torch.uint8, device=dev)
        work = torch.empty(L.rwkv6_wkv_workspace_bytes(B, H, T, K, K, 0), dtype=torch.uint8, device=dev)
        o = torch.empty(B, H, T, K, dtype=torch.bfloat16, device=dev)
        hT = torch.empty(B, H, K, K, dtype=torch.float32, device=dev) if output_final_state else None
        _lib.check(L.rwkv6_wkv_fwd_seqfirst(_p(rb), _p(kb), _p(vb), _p(db), _p(ua), u_code, _p(h0f), _p(o),
                                            _p(hT), _p(saved), _p(work), B, H, T, K, K, float(scale),
                                            _stream_ptr(dev)), "rwkv6_wkv_fwd_seqfirst")
        ctx.save_for_backward(rb, kb, vb, db, ua, saved)
        ctx.meta = (scale, u_code, H, h0 is not None, u.dtype, r.dtype, k.dtype, v.dtype, decay.dtype,
                    None if h0 is None else h0.dtype)
        return o, hT

    @staticmethod
    def backward(ctx, do, dht):
        rb, kb, vb, db, ua, saved = ctx.saved_tensors
        scale, u_code, H, has_h0, u_dt, r_dt, k_dt, v_dt, d_dt, h0_dt = ctx.meta
        T, B, C = rb.shape
        K = C // H
        dev = rb.device
        L = _lib.load()
        dob = _bf16(do) if do is not None else torch.zeros(B, H, T, K, dtype=torch.bfloat16, device=dev)
        dhtf = None if dht is None else _aligned(dht.float())
        dr, dk, dv, ddec = (torch.empty_like(rb) for _ in range(4))
        du = torch.empty(H, K, dtype=ua.dtype, device=dev)
        need_h0 = has_h0 and ctx.needs_input_grad[7]
        dh0 = torch.empty(B, H, K, K, dtype=torch.float32, device=dev) if need_h0 else None
        work = torch.empty(L.rwkv6_wkv_workspace_bytes(B, H, T, K, K, 1), dtype=torch.uint8, device=dev)
        _lib.check(L.rwkv6_wkv_bwd_seqfirst(_p(rb), _p(kb), _p(vb), _p(db), _p(ua), u_code, _p(dob),
                                            _p(dhtf), _p(saved), _p(dr), _p(dk), _p(dv), _p(ddec), _p(du),
                                            _p(dh0), _p(work), B, H, T, K, K, float(scale),
                                            _stream_ptr(dev)), "rwkv6_wkv_bwd_seqfirst")
        cast = lambda t, dt: t if t.dtype == dt else t.to(dt)
        return (cast(dr, r_dt), cast(dk, k_dt), cast(dv, v_dt), cast(ddec, d_dt), cast(du, u_dt),
                None, None, None if dh0 is None else cast(dh0, h0_dt), None)


def wkv6_seqfirst(r, k, v, decay, u, num_heads, scale=1.0, initial_state=None,
                  output_final_state=False):
    """WKV6 for the time-mix module: r, k, v, decay [T,B,H*64] (decay before -exp) ->
    (o [B,H,T,64] head-first, final_state or None).  Same arithmetic as chunk_rwkv6 with
    w = -exp(decay)."""
    for name, t in (("r", r), ("k", k), ("v", v), ("decay", decay)):
        if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
            raise ValueError(f"{name} must be a CUDA tensor")
        if t.dim() != 3 or t.shape != r.shape:
            raise ValueError(f"{name} must be [T,B,C] like r, got {tuple(t.shape)}")
    T, B, C = r.shape
    if C % num_heads or C // num_heads != _HEAD:
        raise NotImplementedError(f"head size must be {_HEAD} (C={C}, heads={num_heads})")
    if tuple(u.shape) != (num_heads, _HEAD):
        raise ValueError(f"u must be [H,64], got {tuple(u.shape)}")
    if initial_state is not None and tuple(initial_state.shape) != (B, num_heads, _HEAD, _HEAD):
        raise ValueError("initial_state must be [B,H,64,64]")
    return _WKV6SeqFirst.apply(r, k, v, decay, u, float(scale), int(num_heads), initial_state,
                               bool(output_final_state))
