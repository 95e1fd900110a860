"""CPU checks that the module mirror builds from Megatron's own TransformerConfig.

The reference's layer spec (rwkv6_layer_specs.py:539-550) has Megatron construct
``RWKV6TimeMix(config, layer_number)`` (:356-361) and ``RWKV6ChannelMix(config)`` (:471-473),
with the config Megatron builds plus the two bottleneck sizes pretrain_rwkv6.py:61-69 adds.
These tests build both modules from a ``SimpleNamespace`` carrying exactly those field names
(no field that only this package defines), on the CPU, and check the parameter names and
shapes against the reference's (TP = 1), the use of Megatron's init callables, the linear
biases of add_bias_linear / add_qkv_bias, and the construction-time refusals.
"""
import math
from types import SimpleNamespace

import pytest
import torch


def megatron_config(C=128, H=2, F=448, L=3, **kw):
    """The fields of megatron.core.transformer.TransformerConfig the reference's time-mix and
    channel-mix constructors read (:356-430, :471-510, GroupNorm :50-88, Bottleneck :112-175,
    WKV6 :303-328), plus token_shift_bottleneck_size / decay_bottleneck_size
    (pretrain_rwkv6.py:61-69).  init_method / output_layer_init_method are the callables
    Megatron's __post_init__ derives from init_method_std."""
    std = 0.02
    cfg = dict(
        hidden_size=C, num_attention_heads=H, ffn_hidden_size=F, num_layers=L,
        layernorm_epsilon=1e-5, params_dtype=torch.float32, perform_initialization=True,
        use_cpu_initialization=False, sequence_parallel=False, add_bias_linear=False,
        add_qkv_bias=False, init_method_std=std,
        init_method=lambda t: torch.nn.init.normal_(t, 0.0, std),
        output_layer_init_method=lambda t: torch.nn.init.normal_(t, 0.0, std / math.sqrt(2.0 * L)),
        token_shift_bottleneck_size=32, decay_bottleneck_size=64)
    cfg.update(kw)
    return SimpleNamespace(**cfg)


def expected_time_mix_shapes(C, bias_qkv=False, bias_proj=False):
    """Parameter names and shapes of the reference's RWKV6TimeMix at TP = 1 (:356-430)."""
    s = {
        "bottleneck_token_shift.weight_down": (C, 5, 32), "bottleneck_token_shift.weight_up": (5, 32, C),
        "bottleneck_token_shift.bias": (5, C), "bottleneck_decay.weight_down": (C, 1, 64),
        "bottleneck_decay.weight_up": (1, 64, C), "bottleneck_decay.bias": (1, C),
        "mix_coeff_input": (C,), "linear_receptance.weight": (C, C), "linear_key.weight": (C, C),
        "linear_value.weight": (C, C), "linear_gate.weight": (C, C),
        "core_attention.time_first": (C,), "group_norm.weight": (C,), "group_norm.bias": (C,),
        "linear_proj.weight": (C, C)}
    if bias_qkv:
        s.update({f"linear_{n}.bias": (C,) for n in ("receptance", "key", "value", "gate")})
    if bias_proj:
        s["linear_proj.bias"] = (C,)
    return s


def test_builds_from_megatron_fields_only(pkg):
    M = pkg.modules
    cfg = megatron_config()
    assert not hasattr(cfg, "rwkv_lm_decay_init")
    torch.manual_seed(0)
    tm = M.RWKV6TimeMix(cfg, 2)                  # :356-361 (config, layer_number)
    cm = M.RWKV6ChannelMix(cfg)                  # :471-473 (config) only
    C, F = cfg.hidden_size, cfg.ffn_hidden_size
    assert {n: tuple(t.shape) for n, t in tm.state_dict().items()} == expected_time_mix_shapes(C)
    assert {n: tuple(t.shape) for n, t in cm.state_dict().items()} == {
        "mix_coeffs": (2, C), "linear_up.weight": (F, C), "linear_gate.weight": (C, C),
        "linear_down.weight": (C, F)}
    for mod in (tm, cm):
        for n, t in mod.state_dict().items():
            assert torch.isfinite(t).all(), n
            assert t.dtype == torch.float32, n
    # reference inits (:172-175, :86-88, :327-328): bottleneck weights U(+-1e-4), bias U(-1, 1),
    # GroupNorm ones / zeros, time_first N(1, 0.02)
    assert tm.bottleneck_decay.weight_down.abs().max() <= 1e-4
    assert tm.bottleneck_token_shift.bias.abs().max() <= 1.0
    assert torch.equal(tm.group_norm.weight, torch.ones(C))
    assert torch.equal(tm.group_norm.bias, torch.zeros(C))
    assert abs(tm.core_attention.time_first.mean().item() - 1.0) < 0.01
    assert tm.group_norm.eps == cfg.layernorm_epsilon                           # :68
    # without a layer number the channel mix gets the first layer's ramp 1 - (c/C)^1
    ramp = 1.0 - torch.arange(C, dtype=torch.float32) / C
    assert torch.allclose(cm.mix_coeffs, torch.stack([ramp, ramp]))
    # a layer number, when given (this package's RWKV6Layer passes one), moves the ramp
    cm3 = M.RWKV6ChannelMix(cfg, 3)
    assert not torch.allclose(cm3.mix_coeffs, cm.mix_coeffs)


def test_uses_megatron_init_callables(pkg):
    """Column-parallel layers take config.init_method, the output projections
    config.output_layer_init_method (:389, :413, :481, :492, :503)."""
    M = pkg.modules
    seen = []
    cfg = megatron_config(init_method=lambda t: (seen.append(("in", tuple(t.shape))), t.fill_(0.5)),
                          output_layer_init_method=lambda t: (seen.append(("out", tuple(t.shape))),
                                                              t.fill_(-0.25)))
    tm = M.RWKV6TimeMix(cfg, 1)
    cm = M.RWKV6ChannelMix(cfg)
    C, F = cfg.hidden_size, cfg.ffn_hidden_size
    for n in ("receptance", "key", "value", "gate"):
        assert torch.all(getattr(tm, "linear_" + n).weight == 0.5)
    assert torch.all(tm.linear_proj.weight == -0.25)
    assert torch.all(cm.linear_up.weight == 0.5) and torch.all(cm.linear_gate.weight == 0.5)
    assert torch.all(cm.linear_down.weight == -0.25)
    assert sorted(seen) == sorted([("in", (C, C))] * 4 + [("out", (C, C))]
                                  + [("in", (F, C)), ("in", (C, C)), ("out", (C, F))])


def test_no_initialization_leaves_parameters_alone(pkg):
    M = pkg.modules
    called = []
    cfg = megatron_config(perform_initialization=False,
                          init_method=lambda t: called.append(t))
    M.RWKV6TimeMix(cfg, 1)
    M.RWKV6ChannelMix(cfg)
    assert called == []


@pytest.mark.parametrize("bias_linear,bias_qkv", [(True, False), (False, True)])
def test_linear_biases(pkg, bias_linear, bias_qkv):
    """add_bias_linear / add_qkv_bias add zero-initialised biases where the reference's
    ColumnParallel / RowParallel layers have them (:393, :416, :484, :495, :505)."""
    M = pkg.modules
    cfg = megatron_config(add_bias_linear=bias_linear, add_qkv_bias=bias_qkv)
    tm = M.RWKV6TimeMix(cfg, 1)
    cm = M.RWKV6ChannelMix(cfg)
    C, F = cfg.hidden_size, cfg.ffn_hidden_size
    assert {n: tuple(t.shape) for n, t in tm.state_dict().items()} == expected_time_mix_shapes(
        C, bias_qkv=True, bias_proj=bias_linear)
    cm_keys = {n: tuple(t.shape) for n, t in cm.state_dict().items()}
    if bias_linear:
        assert cm_keys["linear_up.bias"] == (F,) and cm_keys["linear_down.bias"] == (C,)
        assert cm_keys["linear_gate.bias"] == (C,)
    else:
        assert not any(k.endswith(".bias") for k in cm_keys)
    for n, t in tm.state_dict().items():
        if n.startswith("linear_") and n.endswith(".bias"):
            assert torch.equal(t, torch.zeros_like(t)), n
    # the output projection hands its bias back (skip_bias_add, :418); the others add it
    assert tm.linear_proj.skip_bias_add and not tm.linear_key.skip_bias_add


def test_sequence_parallel_refused(pkg):
    M = pkg.modules
    cfg = megatron_config(sequence_parallel=True)
    with pytest.raises(NotImplementedError, match="sequence_parallel"):
        M.RWKV6TimeMix(cfg, 1)
    with pytest.raises(NotImplementedError, match="sequence_parallel"):
        M.RWKV6ChannelMix(cfg)


def test_package_config_decay_ramp_still_selectable(pkg):
    """The package's own TransformerConfig keeps its RWKV-LM decay-ramp switch."""
    M = pkg.modules
    cfg = M.TransformerConfig(hidden_size=128, num_attention_heads=2, ffn_hidden_size=448,
                              num_layers=2, params_dtype=torch.float32, rwkv_lm_decay_init=True)
    tm = M.RWKV6TimeMix(cfg, 1)
    b = tm.bottleneck_decay.bias[0]
    assert abs(b[0].item() + 6.0) < 1e-6 and abs(b[-1].item() + 1.0) < 1e-5
