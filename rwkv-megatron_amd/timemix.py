"""Fused time-mix building blocks (HIP kernels) as autograd Functions.

* ``token_shift_mix``: token shift + static lerp + LoRA bottleneck + data-dependent
  lerp of RWKV6TimeMix.forward (/root/reference/rwkv_megatron/rwkv6_layer_specs.py
  :440-452, bottleneck :177-195).  The shift/lerp, the LoRA up-projection fused with
  the ddlerp (MFMA) and their backwards are HIP kernels; the LoRA down-projection and the
  weight-gradient GEMMs run on hipBLASLt through torch.matmul / torch.bmm.
* ``decay_lora``: the decay bottleneck (:454) with its up-projection + bias on MFMA;
  ``lora``: the same for either bottleneck as RWKV6Bottleneck.forward returns it (:177-195).
* ``group_norm_gate``: GroupNorm over heads (:90-97, applied at :461-465) times
  silu(gate) (:458, :466), reading the WKV output head-first so the layout copy
  of :341 disappears; ``group_norm``: the same kernels without the gate (GroupNorm.forward,
  :90-97).

Every function raises if the HIP library is missing; there is no fallback.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

NE = 5  # data-dependent mixes, order w, k, v, r, g (rwkv6_layer_specs.py:450)


def _p(t):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _stream(dev):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _c(t: torch.Tensor) -> torch.Tensor:
    t = t.contiguous()
    return t.clone() if t.data_ptr() % 16 else t


def _param(t: torch.Tensor):
    """Parameters may be fp32 or bf16; anything else is computed as fp32."""
    if t.dtype == torch.bfloat16:
        return _c(t), _lib.RWKV6_BF16
    return _c(t.float()), _lib.RWKV6_F32


def _ptrs(ts):
    """Host array of device pointers (the C ABI's `void* const*` arguments)."""
    return (ctypes.c_void_p * len(ts))(*[t.data_ptr() for t in ts])


def _check_act(name, x, ndim):
    if x.device.type != "cuda":
        raise ValueError(f"{name} must live on the GPU")
    if x.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bfloat16, got {x.dtype}")
    if x.dim() != ndim:
        raise ValueError(f"{name} must have {ndim} dims, got shape {tuple(x.shape)}")


# ---------------------------------------------------------------------------
# raw kernel calls
# ---------------------------------------------------------------------------

def shift_lerp(x: torch.Tensor, maa: torch.Tensor) -> torch.Tensor:
    """xxx = x + (shift(x) - x) * maa, x [T,B,C] bf16 (rwkv6_layer_specs.py:440-444)."""
    _check_act("x", x, 3)
    T, B, C = x.shape
    x = _c(x)
    m, pdt = _param(maa)
    out = torch.empty_like(x)
    _lib.check(_lib.load().rwkv6_shift_lerp_fwd(_p(x), _p(m), pdt, _p(out), T, B, C,
                                                _stream(x.device)), "rwkv6_shift_lerp_fwd")
    return out


def tanh_bwd(d_neck, sE, sN, neck, N, E, R):
    """d_pre [N, E*R] = d_neck * (1 - neck^2), the bottleneck's tanh backward (:195), with
    d_neck(e, n, r) at element e*sE + n*sN + r of the contiguous bf16 tensor d_neck."""
    d_neck = _c(d_neck.to(torch.bfloat16))
    d_pre = torch.empty(N, E * R, dtype=torch.bfloat16, device=neck.device)
    _lib.check(_lib.load().rwkv6_lora_tanh_bwd(_p(d_neck), sE, sN, _p(neck), _p(d_pre), N, E, R,
                                               _stream(neck.device)), "rwkv6_lora_tanh_bwd")
    return d_pre


def col_sum(x, dtype):
    """Sum over the rows of x [N, M] bf16 (fixed order, fp32 accumulation), as `dtype` (fp32 or
    bf16): a bottleneck's bias gradient."""
    L = _lib.load()
    N, M = x.shape
    x = _c(x)
    pdt = _lib.RWKV6_BF16 if dtype == torch.bfloat16 else _lib.RWKV6_F32
    out = torch.empty(M, dtype=torch.bfloat16 if pdt == _lib.RWKV6_BF16 else torch.float32, device=x.device)
    ws = torch.empty(L.rwkv6_col_sum_workspace_bytes(N, M), dtype=torch.uint8, device=x.device)
    _lib.check(L.rwkv6_col_sum(_p(x), N, M, pdt, _p(out), _p(ws), _stream(x.device)), "rwkv6_col_sum")
    return out


def gn_gate_fwd(o, head_first, g_pre, gamma, beta, eps):
    """GroupNorm over heads of 64 channels times silu(g_pre); g_pre None: GroupNorm alone."""
    if head_first:
        B, H, T, K = o.shape
    else:
        T, B, C = o.shape
        K = 64
        H = C // K
    o = _c(o)
    g_pre = None if g_pre is None else _c(g_pre)
    ga, pdt = _param(gamma)
    be, pdt_b = _param(beta)
    if pdt_b != pdt:
        be = _c(be.to(ga.dtype))
    y = torch.empty(T, B, H * K, dtype=torch.bfloat16, device=o.device)
    mean = torch.empty(T * B * H, dtype=torch.float32, device=o.device)
    rstd = torch.empty_like(mean)
    _lib.check(_lib.load().rwkv6_gn_gate_fwd(_p(o), int(head_first), _p(g_pre), _p(ga), _p(be), pdt,
                                             float(eps), _p(y), _p(mean), _p(rstd), T, B, H, K,
                                             _stream(o.device)), "rwkv6_gn_gate_fwd")
    return y, mean, rstd


# ---------------------------------------------------------------------------
# autograd Functions
# ---------------------------------------------------------------------------

def sum_partials(part: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """part [S, ...] fp32 -> sum over S in a fixed order, in `dtype` (bf16, else fp32), by
    rwkv6_sum_partials: one pass instead of a reduction and a cast."""
    if part.dtype != torch.float32 or part.device.type != "cuda":
        raise TypeError("sum_partials takes fp32 partials on the GPU")
    part = _c(part)
    bf = dtype == torch.bfloat16
    out = torch.empty(part.shape[1:], dtype=torch.bfloat16 if bf else torch.float32, device=part.device)
    _lib.check(_lib.load().rwkv6_sum_partials(_p(part), part.shape[0], out.numel(),
                                              _lib.RWKV6_BF16 if bf else _lib.RWKV6_F32, _p(out),
                                              _stream(part.device)), "rwkv6_sum_partials")
    return out if bf else out.to(dtype)


def _wgrad(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """a^T @ b for a [N,P], b [N,Q] bf16 with fp32 accumulation, split over N into s batched
    products (a weight gradient has a small output and a long reduction: one GEMM leaves most
    CUs idle), the s fp32 partials summed in a fixed order."""
    N = a.shape[0]
    s = next(d for d in (8, 4, 2, 1) if N % d == 0)
    part = torch.bmm(a.reshape(s, N // s, a.shape[1]).transpose(1, 2),
                     b.reshape(s, N // s, b.shape[1]), out_dtype=torch.float32)
    return sum_partials(part, torch.float32)


class _TokenShiftMix(torch.autograd.Function):
    """x [T,B,C] -> five [T,B,C] mixes (w,k,v,r,g); params maa [C], w_down [C,5,R],
    w_up [5,R,C], bias [5,C] with the shapes of rwkv6_layer_specs.py:126-170, :377-385.

    Forward: shift_lerp (HIP) -> neck = tanh(xxx W_down) (hipBLASLt) -> the up-projection,
    bias and ddlerp in one MFMA kernel writing the five mixes (rwkv6_ddlerp_lora_fwd).
    Backward: rwkv6_ddlerp_lora_bwd (recomputes the up-projection) -> LoRA GEMMs ->
    rwkv6_shift_lerp_bwd for dx and d_maa."""

    @staticmethod
    def forward(ctx, x, maa, w_down, w_up, bias):
        T, B, C = x.shape
        R = w_down.shape[-1]
        N = T * B
        x = _c(x)
        wd = w_down.to(torch.bfloat16).reshape(C, NE * R)
        wut = w_up.to(torch.bfloat16).transpose(1, 2).contiguous()             # [5, C, R]
        xxx = shift_lerp(x, maa)
        neck = _c(torch.tanh(xxx.view(N, C) @ wd))                              # [N, 5R]
        b, pdt = _param(bias)
        mixed = tuple(torch.empty(T, B, C, dtype=torch.bfloat16, device=x.device) for _ in range(NE))
        _lib.check(_lib.load().rwkv6_ddlerp_lora_fwd(_p(x), _p(neck), _p(wut), _p(b), pdt, _ptrs(mixed),
                                                     T, B, C, R, _stream(x.device)),
                   "rwkv6_ddlerp_lora_fwd")
        ctx.save_for_backward(x, maa, w_down, w_up, bias, xxx, neck, wut)
        return mixed

    @staticmethod
    def backward(ctx, *d_mixed):
        x, maa, w_down, w_up, bias, xxx, neck, wut = ctx.saved_tensors
        T, B, C = x.shape
        R = w_down.shape[-1]
        N = T * B
        L = _lib.load()
        dev = x.device
        d_mixed = [torch.zeros_like(x) if d is None else _c(d.to(torch.bfloat16)) for d in d_mixed]
        b, pdt = _param(bias)
        d_mexp = torch.empty(NE, N, C, dtype=torch.bfloat16, device=dev)
        dd = torch.empty(N, C, dtype=torch.bfloat16, device=dev)
        dsum = torch.empty_like(dd)
        d_bias = torch.empty(NE, C, dtype=b.dtype, device=dev)
        ws = torch.empty(L.rwkv6_ddlerp_lora_bwd_workspace_bytes(T, B, C), dtype=torch.uint8, device=dev)
        _lib.check(L.rwkv6_ddlerp_lora_bwd(_p(x), _p(neck), _p(wut), _p(b), pdt, _ptrs(d_mixed),
                                           _p(d_mexp), _p(dd), _p(dsum), _p(d_bias), _p(ws), T, B, C,
                                           R, _stream(dev)), "rwkv6_ddlerp_lora_bwd")
        neck_t = neck.view(N, NE, R).permute(1, 0, 2).contiguous()              # [5, N, R]
        s = next(d for d in (8, 4, 2, 1) if N % d == 0)
        d_w_up = torch.bmm(neck_t.view(NE * s, N // s, R).transpose(1, 2),
                           d_mexp.view(NE * s, N // s, C),
                           out_dtype=torch.float32).view(NE, s, R, C).sum(1)    # [5, R, C]
        d_neck_t = torch.bmm(d_mexp, wut)                                       # [5, N, R]
        d_pre = tanh_bwd(d_neck_t, N * R, R, neck, N, NE, R)                    # [N, 5R]
        wd = w_down.to(torch.bfloat16).reshape(C, NE * R)
        d_w_down = _wgrad(xxx.view(N, C), d_pre).view(C, NE, R)
        d_xxx = _c(d_pre @ wd.t())
        m, pdt_m = _param(maa)
        dx = torch.empty_like(x)
        d_maa = torch.empty(C, dtype=m.dtype, device=dev)
        ws2 = torch.empty(L.rwkv6_shift_lerp_bwd_workspace_bytes(T, B, C), dtype=torch.uint8, device=dev)
        _lib.check(L.rwkv6_shift_lerp_bwd(_p(x), _p(m), pdt_m, _p(dd), _p(dsum), _p(d_xxx), _p(dx),
                                          _p(d_maa), _p(ws2), T, B, C, _stream(dev)),
                   "rwkv6_shift_lerp_bwd")
        return (dx, d_maa.to(maa.dtype), d_w_down.to(w_down.dtype), d_w_up.to(w_up.dtype),
                d_bias.to(bias.dtype))


class _Lora(torch.autograd.Function):
    """out = tanh(x W_down) W_up + bias, RWKV6Bottleneck.forward (rwkv6_layer_specs.py:177-195):
    x [T,B,C], W_down [C,E,R], W_up [E,R,C], bias [E,C] -> [T,B,E,C], E = 1 (decay, :370-375)
    or 5 (token shift, :364-369).  The up-projection and bias run in one MFMA kernel
    (rwkv6_lora_bias_fwd); the down-projection and the weight-gradient GEMMs on hipBLASLt."""

    @staticmethod
    def forward(ctx, x, w_down, w_up, bias):
        T, B, C = x.shape
        E, R = w_down.shape[1], w_down.shape[2]
        N = T * B
        x = _c(x)
        wd = w_down.to(torch.bfloat16).reshape(C, E * R)
        wut = w_up.to(torch.bfloat16).transpose(1, 2).contiguous()             # [E, C, R]
        neck = _c(torch.tanh(x.view(N, C) @ wd))                                # [N, E*R]
        b, pdt = _param(bias)
        out = torch.empty(T, B, E, C, dtype=torch.bfloat16, device=x.device)
        _lib.check(_lib.load().rwkv6_lora_bias_fwd(_p(neck), _p(wut), _p(b), pdt, _p(out), N, E, C, R,
                                                   _stream(x.device)), "rwkv6_lora_bias_fwd")
        ctx.save_for_backward(x, w_down, w_up, bias, neck, wut)
        return out

    @staticmethod
    def backward(ctx, d_out):
        x, w_down, w_up, bias, neck, wut = ctx.saved_tensors
        T, B, C = x.shape
        E, R = w_down.shape[1], w_down.shape[2]
        N = T * B
        g = _c(d_out.to(torch.bfloat16)).view(N, E, C)
        d_bias = col_sum(g.view(N, E * C), bias.dtype).view(E, C)              # [E, C]
        neck3 = neck.view(N, E, R)
        d_w_up = torch.stack([_wgrad(_c(neck3[:, e]), _c(g[:, e])) for e in range(E)])   # [E, R, C]
        d_neck = torch.stack([_c(g[:, e]) @ wut[e] for e in range(E)], 1)       # [N, E, R]
        d_pre = tanh_bwd(d_neck, R, E * R, neck, N, E, R)                       # [N, E*R]
        d_w_down = _wgrad(x.view(N, C), d_pre).view(C, E, R)
        wd = w_down.to(torch.bfloat16).reshape(C, E * R)
        dx = (d_pre @ wd.t()).view(T, B, C)
        return dx, d_w_down.to(w_down.dtype), d_w_up.to(w_up.dtype), d_bias.to(bias.dtype)


def lora(x, w_down, w_up, bias):
    """RWKV6Bottleneck.forward (:177-195): tanh(x W_down) W_up + bias, x [T,B,C] bf16 ->
    [T,B,E,C] bf16 (E = 1 or 5)."""
    _check_act("x", x, 3)
    if w_down.dim() != 3 or w_up.dim() != 3 or w_down.shape[1] != w_up.shape[0]:
        raise ValueError("expected w_down [C,E,R], w_up [E,R,C]")
    return _Lora.apply(x, w_down, w_up, bias)


def decay_lora(x, w_down, w_up, bias):
    """The decay bottleneck of RWKV6TimeMix (:454): tanh(x W_down) W_up + bias, [T,B,C] bf16."""
    _check_act("x", x, 3)
    if w_down.dim() != 3 or w_down.shape[1] != 1:
        raise ValueError("decay_lora expects the E = 1 bottleneck (w_down [C,1,R])")
    return _Lora.apply(x, w_down, w_up, bias).view(x.shape)


def token_shift_mix(x, maa, w_down, w_up, bias):
    """Returns the five [T,B,C] mixes (w, k, v, r, g), the inputs of RWKV6TimeMix's
    projections (:440-452)."""
    _check_act("x", x, 3)
    return _TokenShiftMix.apply(x, maa, w_down, w_up, bias)


class _GroupNormGate(torch.autograd.Function):
    """y = GroupNorm_heads(o) * silu(g_pre), or GroupNorm alone when g_pre is None."""

    @staticmethod
    def forward(ctx, o, head_first, g_pre, gamma, beta, eps):
        y, mean, rstd = gn_gate_fwd(o, head_first, g_pre, gamma, beta, eps)
        ctx.save_for_backward(o, g_pre, gamma, beta, mean, rstd)
        ctx.head_first = head_first
        return y

    @staticmethod
    def backward(ctx, dy):
        o, g_pre, gamma, beta, mean, rstd = ctx.saved_tensors
        head_first = ctx.head_first
        if head_first:
            B, H, T, K = o.shape
        else:
            T, B, C = o.shape
            K = 64
            H = C // K
        L = _lib.load()
        o, dy = _c(o), _c(dy.to(torch.bfloat16))
        g_pre = None if g_pre is None else _c(g_pre)
        ga, pdt = _param(gamma)
        be, pdt_b = _param(beta)
        if pdt_b != pdt:
            be = _c(be.to(ga.dtype))
        d_o = torch.empty_like(o)
        d_g = None if g_pre is None else torch.empty_like(g_pre)
        dgamma = torch.empty(H * K, dtype=ga.dtype, device=o.device)
        dbeta = torch.empty_like(dgamma)
        ws = torch.empty(L.rwkv6_gn_gate_bwd_workspace_bytes(T, B, H, K), dtype=torch.uint8,
                         device=o.device)
        _lib.check(L.rwkv6_gn_gate_bwd(_p(o), int(head_first), _p(g_pre), _p(ga), _p(be), pdt,
                                       _p(mean), _p(rstd), _p(dy), _p(d_o), _p(d_g), _p(dgamma),
                                       _p(dbeta), _p(ws), T, B, H, K, _stream(o.device)),
                   "rwkv6_gn_gate_bwd")
        return d_o, None, d_g, dgamma.to(gamma.dtype), dbeta.to(beta.dtype), None


def group_norm_gate(o, g_pre, gamma, beta, eps, head_first=True):
    """y [T,B,C] = GroupNorm_heads(o) * silu(g_pre); o is [B,H,T,64] (head_first) or [T,B,C]."""
    _check_act("o", o, 4 if head_first else 3)
    _check_act("g_pre", g_pre, 3)
    return _group_norm(o, g_pre, gamma, beta, eps, head_first)


def group_norm(x, num_groups, gamma, beta, eps):
    """The reference's GroupNorm.forward (rwkv6_layer_specs.py:90-97) over x [N, C] bf16 with
    groups of 64 channels (the RWKV-6 head size; other group sizes raise)."""
    _check_act("x", x, 2)
    N, C = x.shape
    if C % num_groups or C // num_groups != 64:
        raise NotImplementedError(f"GroupNorm kernels support groups of 64 channels (C={C}, "
                                  f"groups={num_groups})")
    return _group_norm(x.view(N, 1, C), None, gamma, beta, eps, False).view(N, C)


def _group_norm(o, g_pre, gamma, beta, eps, head_first):
    if head_first:
        B, H, T, K = o.shape
    else:
        T, B, C = o.shape
        K, H = 64, o.shape[-1] // 64
    if K != 64 or (not head_first and o.shape[-1] % 64):
        raise NotImplementedError("GroupNorm gate supports head size 64 only")
    if g_pre is not None and tuple(g_pre.shape) != (T, B, H * K):
        raise ValueError(f"g_pre must be [T,B,C] = {(T, B, H * K)}, got {tuple(g_pre.shape)}")
    return _GroupNormGate.apply(o, bool(head_first), g_pre, gamma, beta, float(eps))
