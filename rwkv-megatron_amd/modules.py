"""Host-side mirror of the reference's RWKV-6 layer modules (TP = 1, one GPU).

Same class names, constructor/forward contracts and parameter names/shapes as
/root/reference/rwkv_megatron/rwkv6_layer_specs.py, so state_dicts load either
way (Megatron's module prefix aside).  The hot path runs on the HIP kernels:

  RWKV6TimeMix.forward  (:431-468)
    token shift + lerp + LoRA + ddlerp   -> timemix.token_shift_mix   (HIP + HIP MFMA + hipBLASLt)
    decay LoRA                           -> timemix.decay_lora        (hipBLASLt + HIP MFMA)
    r/k/v/gate projections               -> torch.matmul (hipBLASLt)
    WKV6 (incl. -exp(decay), layout)     -> wkv.wkv6_seqfirst         (HIP, sequence-first entry)
    GroupNorm * silu(gate)               -> timemix.group_norm_gate   (HIP, head-first read)
    output projection                    -> torch.matmul

  RWKV6ChannelMix.forward  (:512-536)
    token shift + 2 static lerps         -> channelmix.cmix_lerp      (HIP)
    relu^2, sigmoid(gate) * out          -> channelmix.relu_sq / sigmoid_gate (HIP)
    up / gate / down projections         -> torch.matmul

Construction from Megatron's own TransformerConfig.  The layer spec (:539-550) builds
``RWKV6TimeMix(config, layer_number)`` and ``RWKV6ChannelMix(config)``; the config then carries
Megatron's fields plus the two bottleneck sizes pretrain_rwkv6.py:61-69 adds.  Every field
read here is one of those, or is read with getattr and a default:
  hidden_size, num_attention_heads, ffn_hidden_size, num_layers, layernorm_epsilon,
  params_dtype, perform_initialization, init_method_std, token_shift_bottleneck_size,
  decay_bottleneck_size; optional: init_method / output_layer_init_method (callables, as
  Megatron's config sets them; else normal(0, std) and normal(0, std / sqrt(2 L))),
  add_bias_linear / add_qkv_bias (default False), sequence_parallel (must be False: one
  GPU, no token-shift halo), rwkv_lm_decay_init (this package's own switch, default False).

Deliberate differences, all documented in the reference's own terms:
  * ``mix_coeff_input`` and ``RWKV6ChannelMix.mix_coeffs`` are left uninitialised by
    the reference (torch.empty, :377-385, :475-477); here they get the RWKV-6 ramp
    ``1 - (c / C) ** (1 - l / L)`` so a freshly built model is finite.  Megatron builds the
    channel mix without a layer number (:547); it then gets the first layer's ramp
    (l = 0) in every layer, and a checkpoint (from_rwkv_lm) sets the real values.
  * The decay bias keeps the reference's uniform(-1, 1) (:173-175) unless
    ``rwkv_lm_decay_init`` asks for RWKV-LM's ramp.
  * LayerNorms and the output head cast their parameters to the activations' dtype, so fp32
    parameters train with bf16 activations (the HIP kernels take bf16 activations).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn

from . import channelmix, timemix
from .wkv import chunk_rwkv6, wkv6_seqfirst


@dataclass
class TransformerConfig:
    """The fields of Megatron's TransformerConfig that the RWKV-6 layers read."""
    hidden_size: int = 2048
    num_attention_heads: int = 32
    ffn_hidden_size: int = 7168
    num_layers: int = 24
    layernorm_epsilon: float = 1e-5              # example_config.yaml:18, used by GroupNorm (:68)
    token_shift_bottleneck_size: int = 32        # example_config.yaml:8
    decay_bottleneck_size: int = 64              # example_config.yaml:9
    init_method_std: float = 0.02                # example_config.yaml:31
    params_dtype: torch.dtype = torch.bfloat16
    perform_initialization: bool = True
    add_bias_linear: bool = False                # example_config.yaml:20
    add_qkv_bias: bool = False                   # example_config.yaml:22
    sequence_parallel: bool = False              # one GPU: no sequence-parallel token shift
    # The reference initialises the decay bottleneck's bias uniform(-1, 1) (:173-175).  True
    # selects RWKV-LM's per-channel ramp -6 + 5 (c/(C-1))^(0.7 + 1.3 l/(L-1)) instead (the
    # tiny-LM benchmark configuration asks for it).  Not a Megatron field: read with getattr.
    rwkv_lm_decay_init: bool = False


def _check_config(config):
    """Megatron options this one-GPU mirror does not implement raise here, at construction."""
    if getattr(config, "sequence_parallel", False):
        raise NotImplementedError(
            "sequence_parallel: the token-shift halo exchange (rwkv6_layer_specs.py:213-287) is "
            "multi-GPU and not built here")


def _ramp(C, layer_id, n_layers, device):
    ratio = 1.0 - layer_id / max(n_layers, 1)
    ddd = torch.arange(C, dtype=torch.float32, device=device) / C
    return 1.0 - torch.pow(ddd, ratio)


def _splitk_wgrad(dy: torch.Tensor, x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """dW = dy^T x for dy [N, O], x [N, I] (N = tokens), fp32-accumulated.

    A projection's weight gradient has a small output (O x I, e.g. 2048 x 2048 = 64 tiles
    of 256 x 256) and a long reduction (16 K tokens): one GEMM occupies a quarter of the
    256 CUs.  The tokens are split into s chunks (s doubles while the tile count stays below
    512, at most 4: measured on MI355X at 16 K tokens, a 2048 x 2048 dW takes 155 us with
    s = 4 against 170 us with s = 8, whose partial sum reads twice the bytes), the chunks run
    as one batched GEMM with fp32 outputs, and the partials are summed in a fixed order."""
    N, O = dy.shape
    I = x.shape[1]
    tiles = -(-O // 256) * -(-I // 256)
    s = 1
    while s < 4 and tiles * s < 512 and N % (2 * s) == 0:
        s *= 2
    if s == 1:
        return (dy.t() @ x).to(dtype)
    part = torch.bmm(dy.view(s, N // s, O).transpose(1, 2), x.view(s, N // s, I),
                     out_dtype=torch.float32)
    return timemix.sum_partials(part, dtype)


class _LinearFn(torch.autograd.Function):
    """y = x W^T; backward dx = dy W on hipBLASLt, dW by the split-token GEMM above."""

    @staticmethod
    def forward(ctx, x, w):
        wc = w.to(x.dtype)
        ctx.save_for_backward(x, wc)
        ctx.w_dtype = w.dtype
        return F.linear(x, wc)

    @staticmethod
    def backward(ctx, dy):
        x, wc = ctx.saved_tensors
        dy2 = dy.reshape(-1, dy.shape[-1]).contiguous()
        dx = (dy2 @ wc).view(x.shape) if ctx.needs_input_grad[0] else None
        dw = None
        if ctx.needs_input_grad[1]:
            dw = _splitk_wgrad(dy2, x.reshape(-1, x.shape[-1]).contiguous(), ctx.w_dtype)
        return dx, dw


class _Linear(nn.Module):
    """Column/RowParallelLinear at TP=1: weight [out, in], y = x @ W^T, optional bias.

    The weight is initialised by the config's Megatron init callable (``init_attr``:
    ``init_method`` or ``output_layer_init_method``) when it has one, else normal(0, std);
    the bias, as Megatron's, with zeros.  forward returns (y + bias, None), or (y, bias) with
    ``skip_bias_add`` (RowParallelLinear of the time mix's output projection, :411-421)."""

    def __init__(self, cfg, n_in, n_out, std, device, init_attr="init_method", bias=False,
                 skip_bias_add=False):
        super().__init__()
        self.weight = nn.Parameter(torch.empty(n_out, n_in, device=device, dtype=cfg.params_dtype))
        self.bias = (nn.Parameter(torch.zeros(n_out, device=device, dtype=cfg.params_dtype))
                     if bias else None)
        self.skip_bias_add = skip_bias_add
        if cfg.perform_initialization:
            init = getattr(cfg, init_attr, None)
            with torch.no_grad():
                if callable(init):
                    init(self.weight)
                else:
                    nn.init.normal_(self.weight, 0.0, std)

    def forward(self, x):
        y = _LinearFn.apply(x, self.weight)
        if self.bias is None:
            return y, None
        b = self.bias.to(y.dtype)
        return (y, b) if self.skip_bias_add else (y + b, None)


class LayerNorm(nn.LayerNorm):
    """Megatron's LayerNorm at TP = 1 (the layer spec's input_layernorm / pre_mlp_layernorm,
    :543, :546, and the model's pre_norm / final_layernorm); the parameters are cast to the
    activations' dtype, so fp32 parameters run with bf16 activations."""

    def forward(self, x):
        return F.layer_norm(x, self.normalized_shape, self.weight.to(x.dtype), self.bias.to(x.dtype),
                            self.eps)


class OutputLayer(nn.Linear):
    """The untied output head (rwkv6_model.py, output_layer) as y = x W^T with the parameter cast
    to the activations' dtype; the weight gradient by the split-token GEMM of _LinearFn."""

    def forward(self, x):
        return _LinearFn.apply(x, self.weight)


class GroupNorm(nn.Module):
    """rwkv6_layer_specs.py:50-109 (eps taken from config.layernorm_epsilon, :68)."""

    def __init__(self, config, num_groups, num_channels, eps=1e-5, device=None):
        super().__init__()
        self.num_groups = num_groups
        self.num_channels = num_channels
        self.eps = config.layernorm_epsilon
        self.weight = nn.Parameter(torch.ones(num_channels, device=device, dtype=config.params_dtype))
        self.bias = nn.Parameter(torch.zeros(num_channels, device=device, dtype=config.params_dtype))

    def forward(self, hidden_states):
        """GroupNorm over [N, C] (the reference's forward), on the HIP GroupNorm kernel
        (groups of 64 channels, bf16 activations)."""
        return timemix.group_norm(hidden_states, self.num_groups, self.weight, self.bias, self.eps)


class RWKV6Bottleneck(nn.Module):
    """rwkv6_layer_specs.py:112-210 (TP = 1): tanh(x W_down) W_up + bias."""

    def __init__(self, config, bottleneck_size, expansion, to_tensor_parallel, device=None):
        super().__init__()
        C = config.hidden_size
        self.bottleneck_size = bottleneck_size
        self.expansion = expansion
        self.to_tensor_parallel = to_tensor_parallel
        dt = config.params_dtype
        self.weight_down = nn.Parameter(torch.empty(C, expansion, bottleneck_size, device=device, dtype=dt))
        self.weight_up = nn.Parameter(torch.empty(expansion, bottleneck_size, C, device=device, dtype=dt))
        self.bias = nn.Parameter(torch.empty(expansion, C, device=device, dtype=dt))
        if config.perform_initialization:
            nn.init.uniform_(self.weight_down, -1e-4, 1e-4)
            nn.init.uniform_(self.weight_up, -1e-4, 1e-4)
            nn.init.uniform_(self.bias, -1, 1)

    def forward(self, x):
        """[T,B,C] -> [T,B,E,C] (reference layout, :177-195), the up-projection and bias on the
        HIP MFMA kernel.  RWKV6TimeMix does not call this: it runs each bottleneck fused with
        its consumer (timemix.token_shift_mix, timemix.decay_lora)."""
        return timemix.lora(x, self.weight_down, self.weight_up, self.bias)


class WKV6(nn.Module):
    """rwkv6_layer_specs.py:303-353: time_first [C] (N(1, 0.02)), forward over [T,B,C]."""

    def __init__(self, config, layer_number=1, device=None):
        super().__init__()
        self.num_heads_local = config.num_attention_heads
        self.time_first = nn.Parameter(torch.empty(config.hidden_size, device=device,
                                                   dtype=config.params_dtype))
        if config.perform_initialization:
            nn.init.normal_(self.time_first, mean=1.0, std=0.02)

    def head_first(self, r, k, v, decay):
        """Layout glue of :333-337: [T,B,(h n)] -> [B,h,T,n]; w = -exp(decay)."""
        H = self.num_heads_local
        T, B, C = r.shape
        hf = lambda t: t.view(T, B, H, C // H).permute(1, 2, 0, 3).contiguous()
        w = hf(-torch.exp(decay.float())).to(torch.bfloat16)
        u = self.time_first.view(H, C // H)
        return hf(r), hf(k), hf(v), w, u

    def forward(self, r, k, v, w):
        """Reference contract: returns [T,B,C]."""
        rr, kk, vv, ww, u = self.head_first(r, k, v, w)
        o, _ = chunk_rwkv6(rr, kk, vv, ww, u, scale=1.0)
        T, B, C = r.shape
        return o.permute(2, 0, 1, 3).reshape(T, B, C)


class RWKV6TimeMix(nn.Module):
    """rwkv6_layer_specs.py:356-468 with the hot path on HIP kernels."""

    def __init__(self, config, layer_number=1, device=None):
        super().__init__()
        _check_config(config)
        self.config = config
        C = config.hidden_size
        self.layer_number = layer_number
        self.bottleneck_token_shift = RWKV6Bottleneck(config, config.token_shift_bottleneck_size, 5,
                                                      False, device)
        self.bottleneck_decay = RWKV6Bottleneck(config, config.decay_bottleneck_size, 1, True, device)
        self.mix_coeff_input = nn.Parameter(torch.empty(C, device=device, dtype=config.params_dtype))
        std = config.init_method_std
        out_std = std / math.sqrt(2.0 * config.num_layers)
        bias_lin = getattr(config, "add_bias_linear", False)
        bias_qkv = bias_lin or getattr(config, "add_qkv_bias", False)       # :393
        col = lambda: _Linear(config, C, C, std, device, bias=bias_qkv)
        self.linear_receptance = col()
        self.linear_key = col()
        self.linear_value = col()
        self.linear_gate = col()
        self.core_attention = WKV6(config, layer_number, device)
        self.group_norm = GroupNorm(config, config.num_attention_heads, C, config.layernorm_epsilon, device)
        self.linear_proj = _Linear(config, C, C, out_std, device, "output_layer_init_method",
                                   bias=bias_lin, skip_bias_add=True)       # :411-421
        self.num_heads_per_partition = config.num_attention_heads
        self.head_size = C // config.num_attention_heads
        if config.perform_initialization:
            with torch.no_grad():
                self.mix_coeff_input.copy_(_ramp(C, layer_number - 1, config.num_layers, device))
                if getattr(config, "rwkv_lm_decay_init", False):
                    # RWKV-LM's decay ramp -6 + 5 (c/(C-1))^(0.7 + 1.3 l/(L-1))
                    L = max(config.num_layers - 1, 1)
                    c = torch.arange(C, dtype=torch.float32, device=device) / max(C - 1, 1)
                    self.bottleneck_decay.bias.copy_(
                        (-6 + 5 * c ** (0.7 + 1.3 * (layer_number - 1) / L))[None])

    def forward(self, hidden_states, attention_mask=None, key_value_states=None,
                inference_params=None, rotary_pos_emb=None, packed_seq_params=None):
        x = hidden_states
        T, B, C = x.shape
        ts = self.bottleneck_token_shift
        mixed_decay, mixed_key, mixed_value, mixed_receptance, mixed_gate = timemix.token_shift_mix(
            x, self.mix_coeff_input, ts.weight_down, ts.weight_up, ts.bias)
        bd = self.bottleneck_decay
        decay = timemix.decay_lora(mixed_decay, bd.weight_down, bd.weight_up, bd.bias)
        key = self.linear_key(mixed_key)[0]
        value = self.linear_value(mixed_value)[0]
        receptance = self.linear_receptance(mixed_receptance)[0]
        gate_pre = self.linear_gate(mixed_gate)[0]
        H = self.num_heads_per_partition
        u = self.core_attention.time_first.view(H, self.head_size)
        # WKV6 straight on the linear outputs: w = -exp(decay) and the head-first layout of
        # :333-337 happen inside the kernels; o comes back head-first for GroupNorm*gate.
        o, _ = wkv6_seqfirst(receptance, key, value, decay.contiguous(), u, H, scale=1.0)
        y = timemix.group_norm_gate(o, gate_pre, self.group_norm.weight, self.group_norm.bias,
                                    self.group_norm.eps, head_first=True)
        output, bias = self.linear_proj(y)
        return output, bias


class RWKV6ChannelMix(nn.Module):
    """rwkv6_layer_specs.py:471-536 (TP = 1)."""

    def __init__(self, config, layer_number=None, device=None):
        """Megatron builds this module as ``RWKV6ChannelMix(config)`` (:471-473, :547): with no
        layer number the mix coefficients get the first layer's ramp."""
        super().__init__()
        _check_config(config)
        self.config = config
        C, Fh = config.hidden_size, config.ffn_hidden_size
        self.mix_coeffs = nn.Parameter(torch.empty(2, C, device=device, dtype=config.params_dtype))
        std = config.init_method_std
        bias = getattr(config, "add_bias_linear", False)                     # :484, :495, :505
        self.linear_up = _Linear(config, C, Fh, std, device, bias=bias)
        self.linear_gate = _Linear(config, C, C, std, device, bias=bias)
        self.linear_down = _Linear(config, Fh, C, std / math.sqrt(2.0 * config.num_layers), device,
                                   "output_layer_init_method", bias=bias)
        if config.perform_initialization:
            with torch.no_grad():
                ramp = _ramp(C, (layer_number or 1) - 1, config.num_layers, device)
                self.mix_coeffs.copy_(torch.stack([ramp, ramp]))

    def forward(self, hidden_states):
        """:512-536 with the shift + lerps, relu^2 and sigmoid gate on HIP kernels."""
        mixed_up, mixed_gate = channelmix.cmix_lerp(hidden_states, self.mix_coeffs)
        h = channelmix.relu_sq(self.linear_up(mixed_up)[0])
        out = self.linear_down(h)[0]
        return channelmix.sigmoid_gate(out, self.linear_gate(mixed_gate)[0]), None


class RWKV6Layer(nn.Module):
    """The TransformerLayer that get_rwkv6_layer_spec() builds (:539-550):
    LN -> time mix -> residual -> LN -> channel mix -> residual (dropout 0)."""

    def __init__(self, config, layer_number=1, device=None):
        super().__init__()
        C = config.hidden_size
        self.input_layernorm = LayerNorm(C, eps=config.layernorm_epsilon, device=device,
                                         dtype=config.params_dtype)
        self.self_attention = RWKV6TimeMix(config, layer_number, device)
        self.pre_mlp_layernorm = LayerNorm(C, eps=config.layernorm_epsilon, device=device,
                                           dtype=config.params_dtype)
        self.mlp = RWKV6ChannelMix(config, layer_number, device)

    def forward(self, x):
        a, a_bias = self.self_attention(self.input_layernorm(x), None)
        x = x + a if a_bias is None else x + (a + a_bias)    # bias-dropout-add, dropout 0
        m, _ = self.mlp(self.pre_mlp_layernorm(x))
        return x + m


def get_rwkv6_layer_spec():
    """Mirror of rwkv6_layer_specs.py:539-550 as a plain description (no Megatron here)."""
    return dict(module=RWKV6Layer,
                submodules=dict(input_layernorm=LayerNorm, self_attention=RWKV6TimeMix,
                                pre_mlp_layernorm=LayerNorm, mlp=RWKV6ChannelMix))


class RWKV6Model(nn.Module):
    """One-GPU RWKV-6 LM mirroring RWKV6Model (rwkv6_model.py:28-184): embedding ->
    pre_norm (ln0, :34-37, :108-112) -> layers -> final LayerNorm -> untied output head.
    Activations are bf16 (the HIP kernels' dtype) whatever the parameters' dtype."""

    def __init__(self, config, vocab_size, device=None):
        super().__init__()
        C = config.hidden_size
        dt = config.params_dtype
        self.embedding = nn.Embedding(vocab_size, C, device=device, dtype=dt)
        nn.init.normal_(self.embedding.weight, 0.0, config.init_method_std)
        self.pre_norm = LayerNorm(C, eps=config.layernorm_epsilon, device=device, dtype=dt)
        self.layers = nn.ModuleList(RWKV6Layer(config, i + 1, device) for i in range(config.num_layers))
        self.final_layernorm = LayerNorm(C, eps=config.layernorm_epsilon, device=device, dtype=dt)
        self.output_layer = OutputLayer(C, vocab_size, bias=False, device=device, dtype=dt)
        nn.init.normal_(self.output_layer.weight, 0.0, config.init_method_std)

    def forward(self, tokens):
        """tokens [B,T] -> logits [T,B,V] (sequence-first inside, as Megatron)."""
        x = self.pre_norm(self.embedding(tokens.t()).to(torch.bfloat16))
        for layer in self.layers:
            x = layer(x)
        return self.output_layer(self.final_layernorm(x))

    @torch.no_grad()
    def from_rwkv_lm(self, sd):
        """Loads RWKV-LM weights into this model (rwkv6_model.py:295-372), cast to the
        parameters' dtype and device; see rwkv_lm_to_state_dict for the key map."""
        own = self.state_dict()
        conv = rwkv_lm_to_state_dict(sd, len(self.layers))
        missing = sorted(set(own) - set(conv))
        if missing:
            raise KeyError(f"no RWKV-LM source for {missing}")
        for name, t in conv.items():
            if tuple(t.shape) != tuple(own[name].shape):
                raise ValueError(f"{name}: checkpoint shape {tuple(t.shape)} != {tuple(own[name].shape)}")
            own[name].copy_(t.to(own[name].dtype))
        return self


def rwkv_lm_to_state_dict(sd, num_layers, head_size=64):
    """RWKV-LM (BlinkDL) RWKV-6 checkpoint keys -> this package's RWKV6Model state_dict.

    Mirrors RWKV6Model.from_rwkv_lm (rwkv6_model.py:295-372) at TP = 1 with
    layernorm_zero_centered_gamma off (norm offset 0):
      emb.weight -> embedding.weight; blocks.0.ln0 -> pre_norm; ln_out -> final_layernorm;
      head.weight -> output_layer.weight; per block i:
      ln1 / ln2 -> input_layernorm / pre_mlp_layernorm;
      att.time_maa_x -> mix_coeff_input; att.time_maa_w1 [C, 5R] -> bottleneck_token_shift
      .weight_down [C, 5, R] ("d (e r) -> d e r"); att.time_maa_w2 -> .weight_up;
      att.time_maa_{w,k,v,r,g} -> .bias[0..4] (order "wkvrg");
      att.time_decay_w1 [C, R] -> bottleneck_decay.weight_down [C, 1, R];
      att.time_decay_w2 [R, C] -> .weight_up [1, R, C]; att.time_decay -> .bias [1, C];
      att.time_faaaa -> core_attention.time_first [C]; att.{receptance,key,value,gate,output}
      -> linear_{receptance,key,value,gate,proj}; att.ln_x -> group_norm;
      ffn.time_maa_k / ffn.time_maa_r -> mlp.mix_coeffs[0] / [1];
      ffn.key / ffn.receptance / ffn.value -> mlp.linear_up / linear_gate / linear_down.
    Tensors are returned as they come (dtype and device of `sd`); shapes are flattened or
    split exactly as the reference does."""
    out = {
        "embedding.weight": sd["emb.weight"],
        "pre_norm.weight": sd["blocks.0.ln0.weight"],
        "pre_norm.bias": sd["blocks.0.ln0.bias"],
        "final_layernorm.weight": sd["ln_out.weight"],
        "final_layernorm.bias": sd["ln_out.bias"],
        "output_layer.weight": sd["head.weight"],
    }
    for i in range(num_layers):
        src = f"blocks.{i}."
        dst = f"layers.{i}."
        att = lambda k: sd[src + "att." + k]
        ffn = lambda k: sd[src + "ffn." + k]
        C = att("time_maa_x").numel()
        w1 = att("time_maa_w1")
        out.update({
            dst + "input_layernorm.weight": sd[src + "ln1.weight"],
            dst + "input_layernorm.bias": sd[src + "ln1.bias"],
            dst + "pre_mlp_layernorm.weight": sd[src + "ln2.weight"],
            dst + "pre_mlp_layernorm.bias": sd[src + "ln2.bias"],
            dst + "self_attention.mix_coeff_input": att("time_maa_x").reshape(C),
            dst + "self_attention.bottleneck_token_shift.weight_down": w1.reshape(C, 5, w1.shape[1] // 5),
            dst + "self_attention.bottleneck_token_shift.weight_up": att("time_maa_w2"),
            dst + "self_attention.bottleneck_token_shift.bias": torch.stack(
                [att("time_maa_" + n).reshape(C) for n in "wkvrg"]),
            dst + "self_attention.bottleneck_decay.weight_down": att("time_decay_w1").unsqueeze(1),
            dst + "self_attention.bottleneck_decay.weight_up": att("time_decay_w2").unsqueeze(0),
            dst + "self_attention.bottleneck_decay.bias": att("time_decay").reshape(1, C),
            dst + "self_attention.core_attention.time_first": att("time_faaaa").reshape(C),
            dst + "self_attention.linear_receptance.weight": att("receptance.weight"),
            dst + "self_attention.linear_key.weight": att("key.weight"),
            dst + "self_attention.linear_value.weight": att("value.weight"),
            dst + "self_attention.linear_gate.weight": att("gate.weight"),
            dst + "self_attention.linear_proj.weight": att("output.weight"),
            dst + "self_attention.group_norm.weight": att("ln_x.weight"),
            dst + "self_attention.group_norm.bias": att("ln_x.bias"),
            dst + "mlp.mix_coeffs": torch.stack([ffn("time_maa_k").reshape(C), ffn("time_maa_r").reshape(C)]),
            dst + "mlp.linear_up.weight": ffn("key.weight"),
            dst + "mlp.linear_gate.weight": ffn("receptance.weight"),
            dst + "mlp.linear_down.weight": ffn("value.weight"),
        })
    return out


def load_rwkv_lm(path):
    """Reads an RWKV-LM .pth checkpoint with torch.load(weights_only=True) (tensors only, no
    code from the file runs); returns the raw state dict for rwkv_lm_to_state_dict."""
    return torch.load(path, map_location="cpu", weights_only=True)
