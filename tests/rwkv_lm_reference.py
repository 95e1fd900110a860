"""RWKV-6 LM forward written against RWKV-LM's own (BlinkDL) parameter names, for the
checkpoint-interop tests: the converter must put every RWKV-LM tensor where this forward
uses it.  fp64 numpy on the CPU, built from the oracle's pieces (token shift, LoRA
bottleneck, ddlerp, WKV6 recurrence, GroupNorm); the block follows RWKV-LM's RWKV-6
time mix / channel mix with the reference's eps choices (config.layernorm_epsilon for both
LayerNorm and the head GroupNorm, rwkv6_layer_specs.py:68)."""
import numpy as np

from oracle import oracle as orc


def make_state_dict(C, H, F, L, V, r_mix=32, r_decay=64, seed=0):
    """A random RWKV-LM RWKV-6 state dict (torch fp32 CPU tensors, RWKV-LM shapes)."""
    import torch
    g = torch.Generator().manual_seed(seed)
    rn = lambda *s, std=0.1: (std * torch.randn(*s, generator=g)).float()
    ru = lambda *s: torch.rand(*s, generator=g).float()
    sd = {"emb.weight": rn(V, C, std=0.5), "blocks.0.ln0.weight": 1 + rn(C), "blocks.0.ln0.bias": rn(C),
          "ln_out.weight": 1 + rn(C), "ln_out.bias": rn(C), "head.weight": rn(V, C, std=0.1)}
    for i in range(L):
        p = f"blocks.{i}."
        sd.update({p + "ln1.weight": 1 + rn(C), p + "ln1.bias": rn(C),
                   p + "ln2.weight": 1 + rn(C), p + "ln2.bias": rn(C)})
        a = p + "att."
        sd.update({a + "time_maa_x": ru(1, 1, C), a + "time_maa_w1": rn(C, 5 * r_mix, std=0.3),
                   a + "time_maa_w2": rn(5, r_mix, C, std=0.3)})
        for n in "wkvrg":
            sd[a + "time_maa_" + n] = ru(1, 1, C)
        sd.update({a + "time_decay": (-6 + 5 * ru(1, 1, C)), a + "time_decay_w1": rn(C, r_decay, std=0.3),
                   a + "time_decay_w2": rn(r_decay, C, std=0.3), a + "time_faaaa": rn(H, 64, std=0.5)})
        for n in ("receptance", "key", "value", "gate", "output"):
            sd[a + n + ".weight"] = rn(C, C, std=C ** -0.5)
        sd.update({a + "ln_x.weight": 1 + rn(C), a + "ln_x.bias": rn(C)})
        f = p + "ffn."
        sd.update({f + "time_maa_k": ru(1, 1, C), f + "time_maa_r": ru(1, 1, C),
                   f + "key.weight": rn(F, C, std=C ** -0.5), f + "receptance.weight": rn(C, C, std=C ** -0.5),
                   f + "value.weight": rn(C, F, std=F ** -0.5)})
    return sd


def _ln(x, w, b, eps):
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * w + b


def _time_mix(x, P, H, eps):
    T, B, C = x.shape
    xxx = orc.shift_lerp_fwd(x, P["time_maa_x"].reshape(C))
    w1 = P["time_maa_w1"]
    R = w1.shape[1] // 5
    m = orc.bottleneck_fwd(xxx, w1.reshape(C, 5, R), P["time_maa_w2"], np.zeros((5, C)))
    bias = np.stack([P["time_maa_" + n].reshape(C) for n in "wkvrg"])
    xw, xk, xv, xr, xg = orc.ddlerp_fwd(x, m, bias)
    decay = P["time_decay"].reshape(C) + np.tanh(xw @ P["time_decay_w1"]) @ P["time_decay_w2"]
    r, k, v = xr @ P["receptance.weight"].T, xk @ P["key.weight"].T, xv @ P["value.weight"].T
    gz = xg @ P["gate.weight"].T
    hf = lambda t: t.reshape(T, B, H, 64).transpose(1, 2, 0, 3)
    o, _ = orc.wkv6_fwd(hf(r), hf(k), hf(v), hf(-np.exp(decay)), P["time_faaaa"].reshape(H, 64), None, 1.0)
    o = o.transpose(2, 0, 1, 3).reshape(T * B, C)
    y, _, _ = orc.group_norm_fwd(o, H, P["ln_x.weight"], P["ln_x.bias"], eps)
    y = y.reshape(T, B, C) * (gz / (1 + np.exp(-gz)))
    return y @ P["output.weight"].T


def _channel_mix(x, P):
    C = x.shape[-1]
    mix = np.stack([P["time_maa_k"].reshape(C), P["time_maa_r"].reshape(C)])
    return orc.channel_mix_fwd(x, mix, P["key.weight"], P["receptance.weight"], P["value.weight"])


def forward(sd, tokens, n_layer, H, eps=1e-5):
    """tokens [B,T] int -> logits [T,B,V] (fp64)."""
    S = {k: v.double().numpy() for k, v in sd.items()}
    x = S["emb.weight"][tokens.T]                                     # [T,B,C]
    x = _ln(x, S["blocks.0.ln0.weight"], S["blocks.0.ln0.bias"], eps)
    for i in range(n_layer):
        p = f"blocks.{i}."
        att = {k[len(p) + 4:]: v for k, v in S.items() if k.startswith(p + "att.")}
        ffn = {k[len(p) + 4:]: v for k, v in S.items() if k.startswith(p + "ffn.")}
        x = x + _time_mix(_ln(x, S[p + "ln1.weight"], S[p + "ln1.bias"], eps), att, H, eps)
        x = x + _channel_mix(_ln(x, S[p + "ln2.weight"], S[p + "ln2.bias"], eps), ffn)
    x = _ln(x, S["ln_out.weight"], S["ln_out.bias"], eps)
    return x @ S["head.weight"].T
