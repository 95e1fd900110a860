"""CPU oracle for the RWKV-6 time-mix hot path (TEST INFRASTRUCTURE ONLY).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module.  It is the checker, never the product:
the GPU package fails loudly when its HIP library is missing and never routes
through anything here.

Contents
--------
* ``wkv6_fwd`` / ``wkv6_bwd``: ctypes front-end of ``wkv6_oracle.c``, the fp64
  naive-recurrent RWKV-6 (fla ``fused_recurrent_rwkv6`` contract as called at
  /root/reference/rwkv_megatron/rwkv6_layer_specs.py:339).
* numpy fp64 restatements (forward and explicit backward) of the elementwise
  parts of ``RWKV6TimeMix.forward``:
    - token shift            rwkv6_layer_specs.py:290-300
    - shift + static lerp    rwkv6_layer_specs.py:443-444
    - data-dependent lerp    rwkv6_layer_specs.py:447-452 (bias of :195 folded in)
    - GroupNorm * silu gate  rwkv6_layer_specs.py:90-97, :458, :461-466
    - LoRA bottleneck        rwkv6_layer_specs.py:177-195
  and of ``RWKV6ChannelMix.forward`` (rwkv6_layer_specs.py:512-536): shift + static
  lerp, relu^2, sigmoid gate, and the whole block with its projections.

Pinning (each checked in tests/test_oracle.py, never by retyping a formula):
WKV forward against the quadratic (attention-form) closed form, w=0 causal
linear attention, w->-inf bonus-only output, T=1, segment splitting and
linearity; WKV backward against torch.autograd of an independent fp64 torch
formulation; GroupNorm against ``torch.nn.functional.group_norm`` (the
routine the reference calls); the elementwise backward passes against
torch.autograd of the reference-shaped torch code; the channel-mix lerp against
its end points (mix = 0 gives x, mix = 1 gives shift(x)).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libwkv6_oracle.so")
_lib = None


def build(force: bool = False) -> str:
    """Compile the C oracle with its Makefile (gcc).  Returns the .so path."""
    if force or not os.path.exists(_LIB_PATH):
        cmd = ["make", "-C", _HERE, "-B" if force else "all"]
        subprocess.run([c for c in cmd if c], check=True, capture_output=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        fp = ctypes.POINTER(ctypes.c_float)
        i64 = ctypes.c_int64
        L.wkv6_oracle_fwd.argtypes = [fp] * 6 + [ctypes.c_float] + [i64] * 5 + [fp, fp, ctypes.c_int]
        L.wkv6_oracle_fwd.restype = None
        L.wkv6_oracle_bwd.argtypes = (
            [fp] * 8 + [ctypes.c_float] + [i64] * 5 + [fp] * 6 + [ctypes.c_int]
        )
        L.wkv6_oracle_bwd.restype = None
        L.wkv6_oracle_max_threads.argtypes = []
        L.wkv6_oracle_max_threads.restype = ctypes.c_int
        _lib = L
    return _lib


def max_threads() -> int:
    return int(lib().wkv6_oracle_max_threads())


def _f32(a):
    if a is None:
        return None
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _ptr(a):
    if a is None:
        return ctypes.POINTER(ctypes.c_float)()
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def wkv6_fwd(r, k, v, w, u, h0=None, scale=1.0, nthreads=0):
    """Naive recurrent RWKV-6 forward.

    r, k, w: [B,H,T,K]; v: [B,H,T,V]; u: [H,K]; h0: [B,H,K,V] or None.
    ``w`` is log-space decay.  Returns (o [B,H,T,V] f32, hT [B,H,K,V] f32).
    """
    r, k, v, w, u, h0 = (_f32(x) for x in (r, k, v, w, u, h0))
    B, H, T, K = r.shape
    V = v.shape[-1]
    assert k.shape == (B, H, T, K) and w.shape == (B, H, T, K) and v.shape == (B, H, T, V)
    assert u.shape == (H, K)
    o = np.empty((B, H, T, V), np.float32)
    hT = np.empty((B, H, K, V), np.float32)
    lib().wkv6_oracle_fwd(
        _ptr(r), _ptr(k), _ptr(v), _ptr(w), _ptr(u), _ptr(h0), float(scale),
        B, H, T, K, V, _ptr(o), _ptr(hT), int(nthreads),
    )
    return o, hT


def wkv6_bwd(r, k, v, w, u, dO, h0=None, dhT=None, scale=1.0, nthreads=0):
    """Exact reverse-time backward of ``wkv6_fwd``.

    Returns dict with dr, dk, dv, dw ([B,H,T,*]), du ([H,K]) and dh0 ([B,H,K,V]).
    """
    r, k, v, w, u, h0, dO, dhT = (_f32(x) for x in (r, k, v, w, u, h0, dO, dhT))
    B, H, T, K = r.shape
    V = v.shape[-1]
    dr = np.empty_like(r)
    dk = np.empty_like(k)
    dv = np.empty_like(v)
    dw = np.empty_like(w)
    du = np.empty((H, K), np.float32)
    dh0 = np.empty((B, H, K, V), np.float32)
    lib().wkv6_oracle_bwd(
        _ptr(r), _ptr(k), _ptr(v), _ptr(w), _ptr(u), _ptr(h0), _ptr(dO), _ptr(dhT),
        float(scale), B, H, T, K, V,
        _ptr(dr), _ptr(dk), _ptr(dv), _ptr(dw), _ptr(du), _ptr(dh0), int(nthreads),
    )
    return dict(dr=dr, dk=dk, dv=dv, dw=dw, du=du, dh0=dh0)


# ---------------------------------------------------------------------------
# Elementwise parts of RWKV6TimeMix (numpy, fp64), sequence-first [T, B, C]
# ---------------------------------------------------------------------------

def token_shift(x):
    """x_prev[t] = x[t-1], x_prev[0] = 0 along dim 0 (rwkv6_layer_specs.py:294-300)."""
    x = np.asarray(x, np.float64)
    out = np.zeros_like(x)
    out[1:] = x[:-1]
    return out


def token_shift_bwd(dy):
    """Adjoint of ``token_shift``: dx[t] = dy[t+1], dx[T-1] = 0."""
    dy = np.asarray(dy, np.float64)
    out = np.zeros_like(dy)
    out[:-1] = dy[1:]
    return out


def shift_lerp_fwd(x, maa):
    """xxx = x + (shift(x) - x) * maa   (rwkv6_layer_specs.py:443-444)."""
    x = np.asarray(x, np.float64)
    delta = token_shift(x) - x
    return x + delta * np.asarray(maa, np.float64)


def ddlerp_fwd(x, mexp, bias):
    """mixed[e] = x + (shift(x) - x) * (mexp[:, :, e] + bias[e]) for e in w,k,v,r,g.

    rwkv6_layer_specs.py:446-452 with the bottleneck bias of :195 folded in.
    x: [T,B,C]; mexp: [T,B,5,C] (LoRA up-projection without bias); bias: [5,C].
    Returns [5,T,B,C].
    """
    x = np.asarray(x, np.float64)
    m = np.asarray(mexp, np.float64) + np.asarray(bias, np.float64)
    delta = token_shift(x) - x
    return np.moveaxis(x[:, :, None, :] + delta[:, :, None, :] * m, 2, 0)


def mix_bwd(x, maa, mexp, bias, d_mixed, d_xxx):
    """Backward of shift_lerp_fwd + ddlerp_fwd sharing one input x.

    Returns (dx [T,B,C], d_mexp [T,B,5,C], d_bias [5,C], d_maa [C]).
    """
    x = np.asarray(x, np.float64)
    maa = np.asarray(maa, np.float64)
    m = np.asarray(mexp, np.float64) + np.asarray(bias, np.float64)
    dmix = np.moveaxis(np.asarray(d_mixed, np.float64), 0, 2)  # [T,B,5,C]
    dxxx = np.asarray(d_xxx, np.float64)
    delta = token_shift(x) - x
    # mixed_e = x + delta*m_e ; xxx = x + delta*maa ; delta = shift(x) - x
    d_delta = (dmix * m).sum(axis=2) + dxxx * maa
    dx = dmix.sum(axis=2) + dxxx - d_delta + token_shift_bwd(d_delta)
    d_mexp = dmix * delta[:, :, None, :]
    d_bias = d_mexp.sum(axis=(0, 1))
    d_maa = (dxxx * delta).sum(axis=(0, 1))
    return dx, d_mexp, d_bias, d_maa


def cmix_lerp_fwd(x, mix):
    """Channel-mix inputs (rwkv6_layer_specs.py:512-520): mixed[e] = x + (shift(x) - x) * mix[e],
    e = 0 (up), 1 (gate).  x: [T,B,C]; mix: [2,C] (mix_coeffs).  Returns [2,T,B,C]."""
    x = np.asarray(x, np.float64)
    delta = token_shift(x) - x
    return x[None] + delta[None] * np.asarray(mix, np.float64)[:, None, None, :]


def cmix_lerp_bwd(x, mix, d_mixed):
    """Adjoint of ``cmix_lerp_fwd``: returns (dx [T,B,C], d_mix [2,C])."""
    x = np.asarray(x, np.float64)
    mix = np.asarray(mix, np.float64)
    g = np.asarray(d_mixed, np.float64)
    delta = token_shift(x) - x
    d_delta = (g * mix[:, None, None, :]).sum(axis=0)
    dx = g.sum(axis=0) - d_delta + token_shift_bwd(d_delta)
    d_mix = (g * delta[None]).sum(axis=(1, 2))
    return dx, d_mix


def relu_sq_fwd(up):
    """square(relu(up)) (rwkv6_layer_specs.py:524)."""
    return np.maximum(np.asarray(up, np.float64), 0.0) ** 2


def relu_sq_bwd(up, dh):
    return 2.0 * np.maximum(np.asarray(up, np.float64), 0.0) * np.asarray(dh, np.float64)


def sigmoid_gate_fwd(out, gate_pre):
    """out * sigmoid(gate_pre) (rwkv6_layer_specs.py:533-536)."""
    return np.asarray(out, np.float64) * _sigmoid(np.asarray(gate_pre, np.float64))


def sigmoid_gate_bwd(out, gate_pre, dy):
    """Returns (d_out, d_gate_pre)."""
    sg = _sigmoid(np.asarray(gate_pre, np.float64))
    dy = np.asarray(dy, np.float64)
    return dy * sg, dy * np.asarray(out, np.float64) * sg * (1.0 - sg)


def channel_mix_fwd(x, mix, w_up, w_gate, w_down):
    """RWKV6ChannelMix.forward (rwkv6_layer_specs.py:512-536, TP=1, no biases); weights in the
    Megatron [out, in] layout.  x: [T,B,C] -> [T,B,C]."""
    mixed = cmix_lerp_fwd(x, mix)
    h = relu_sq_fwd(mixed[0] @ np.asarray(w_up, np.float64).T)
    out = h @ np.asarray(w_down, np.float64).T
    return sigmoid_gate_fwd(out, mixed[1] @ np.asarray(w_gate, np.float64).T)


def channel_mix_bwd(x, mix, w_up, w_gate, w_down, dy):
    """Backward of ``channel_mix_fwd``: returns (dx, d_mix, d_w_up, d_w_gate, d_w_down)."""
    w_up, w_gate, w_down = (np.asarray(w, np.float64) for w in (w_up, w_gate, w_down))
    mixed = cmix_lerp_fwd(x, mix)
    up = mixed[0] @ w_up.T
    h = relu_sq_fwd(up)
    out = h @ w_down.T
    gp = mixed[1] @ w_gate.T
    d_out, d_gp = sigmoid_gate_bwd(out, gp, dy)
    C, F = x.shape[-1], w_up.shape[0]
    d_w_down = d_out.reshape(-1, C).T @ h.reshape(-1, F)
    d_up = relu_sq_bwd(up, d_out @ w_down)
    d_w_up = d_up.reshape(-1, F).T @ mixed[0].reshape(-1, C)
    d_w_gate = d_gp.reshape(-1, C).T @ mixed[1].reshape(-1, C)
    d_mixed = np.stack([d_up @ w_up, d_gp @ w_gate])
    dx, d_mix = cmix_lerp_bwd(x, mix, d_mixed)
    return dx, d_mix, d_w_up, d_w_gate, d_w_down


def group_norm_fwd(x, groups, gamma, beta, eps):
    """Per-group normalisation over the channel dim of x [N, C] (rwkv6_layer_specs.py:90-97)."""
    x = np.asarray(x, np.float64)
    N, C = x.shape
    xg = x.reshape(N, groups, C // groups)
    mean = xg.mean(axis=-1, keepdims=True)
    var = ((xg - mean) ** 2).mean(axis=-1, keepdims=True)
    rstd = 1.0 / np.sqrt(var + eps)
    xhat = ((xg - mean) * rstd).reshape(N, C)
    return xhat * np.asarray(gamma, np.float64) + np.asarray(beta, np.float64), mean[..., 0], rstd[..., 0]


def _sigmoid(z):
    return 1.0 / (1.0 + np.exp(-z))


def gn_gate_fwd(o, g_pre, groups, gamma, beta, eps):
    """y = GroupNorm(o) * silu(g_pre) over o, g_pre [N, C] (rwkv6_layer_specs.py:458, :461-466)."""
    y, mean, rstd = group_norm_fwd(o, groups, gamma, beta, eps)
    z = np.asarray(g_pre, np.float64)
    return y * (z * _sigmoid(z)), mean, rstd


def gn_gate_bwd(o, g_pre, groups, gamma, beta, eps, dy):
    """Returns (do, dg_pre, dgamma, dbeta) for ``gn_gate_fwd``."""
    o = np.asarray(o, np.float64)
    z = np.asarray(g_pre, np.float64)
    dy = np.asarray(dy, np.float64)
    gamma = np.asarray(gamma, np.float64)
    N, C = o.shape
    D = C // groups
    y, mean, rstd = group_norm_fwd(o, groups, gamma, beta, eps)
    sig = _sigmoid(z)
    gate = z * sig
    dg_pre = dy * y * sig * (1.0 + z * (1.0 - sig))
    dn = dy * gate
    xhat = ((o.reshape(N, groups, D) - mean[..., None]) * rstd[..., None])
    dgamma = (dn.reshape(N, groups, D) * xhat).reshape(N, C).sum(axis=0)
    dbeta = dn.sum(axis=0)
    dxhat = (dn * gamma).reshape(N, groups, D)
    do = rstd[..., None] * (
        dxhat - dxhat.mean(axis=-1, keepdims=True) - xhat * (dxhat * xhat).mean(axis=-1, keepdims=True)
    )
    return do.reshape(N, C), dg_pre, dgamma, dbeta


def bottleneck_bwd(x, w_down, w_up, dm):
    """Backward of ``bottleneck_fwd`` for dm = dL/d(output) [T,B,E,C].

    Returns (dx [T,B,C], d_w_down [C,E,R], d_w_up [E,R,C], d_bias [E,C]).
    """
    x = np.asarray(x, np.float64)
    wd = np.asarray(w_down, np.float64)
    wu = np.asarray(w_up, np.float64)
    dm = np.asarray(dm, np.float64)
    neck = np.tanh(np.einsum("tbd,der->tber", x, wd))
    d_bias = dm.sum(axis=(0, 1))
    d_wu = np.einsum("tber,tbed->erd", neck, dm)
    d_pre = np.einsum("tbed,erd->tber", dm, wu) * (1.0 - neck ** 2)
    d_wd = np.einsum("tbd,tber->der", x, d_pre)
    dx = np.einsum("tber,der->tbd", d_pre, wd)
    return dx, d_wd, d_wu, d_bias


def bottleneck_fwd(x, w_down, w_up, bias):
    """tanh(x . W_down) . W_up + bias  (rwkv6_layer_specs.py:177-195, TP=1).

    x: [T,B,C]; w_down: [C,E,R]; w_up: [E,R,C]; bias: [E,C].  Returns [T,B,E,C].
    """
    x = np.asarray(x, np.float64)
    neck = np.tanh(np.einsum("tbd,der->tber", x, np.asarray(w_down, np.float64)))
    return np.einsum("tber,erd->tbed", neck, np.asarray(w_up, np.float64)) + np.asarray(bias, np.float64)
