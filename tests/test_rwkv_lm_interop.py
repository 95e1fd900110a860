"""RWKV-LM checkpoint interop (RWKV6Model.from_rwkv_lm, rwkv6_model.py:295-372).

CPU: the key map covers the whole model, splits/flattens like the reference, rejects wrong
shapes, and round-trips a .pth through torch.load(weights_only=True).
GPU: the converted model's logits equal an fp64 forward written against RWKV-LM's own
parameter names (tests/rwkv_lm_reference.py), max-rel and L2-rel <= 6e-2 (bf16 weights,
activations and residual stream through 2 layers; the reference side uses the same
bf16-rounded weights), while a converter that swaps two mixes lands far outside that.
"""
import os

import numpy as np
import pytest
import torch

import parity
import rwkv_lm_reference as ref

C, H, F, L, V = 128, 2, 448, 2, 256
TOL = 6e-2    # bf16 weights, activations and residual stream through 2 layers vs fp64


def _model(pkg, device):
    M = pkg.modules
    cfg = M.TransformerConfig(hidden_size=C, num_attention_heads=H, ffn_hidden_size=F, num_layers=L,
                              params_dtype=torch.bfloat16)
    return M.RWKV6Model(cfg, V, device=device)


def test_key_map_covers_model_and_follows_reference(pkg):
    sd = ref.make_state_dict(C, H, F, L, V)
    model = _model(pkg, "cpu").from_rwkv_lm(sd)
    own = model.state_dict()
    bf = lambda t: t.to(torch.bfloat16)
    tm = "layers.1.self_attention."
    w1 = sd["blocks.1.att.time_maa_w1"]
    for e in range(5):            # "d (e r) -> d e r"
        assert torch.equal(own[tm + "bottleneck_token_shift.weight_down"][:, e], bf(w1[:, 32 * e:32 * (e + 1)]))
    for e, n in enumerate("wkvrg"):
        assert torch.equal(own[tm + "bottleneck_token_shift.bias"][e], bf(sd["blocks.1.att.time_maa_" + n].flatten()))
    assert torch.equal(own[tm + "bottleneck_decay.weight_down"][:, 0], bf(sd["blocks.1.att.time_decay_w1"]))
    assert torch.equal(own[tm + "core_attention.time_first"], bf(sd["blocks.1.att.time_faaaa"].flatten()))
    assert torch.equal(own[tm + "linear_proj.weight"], bf(sd["blocks.1.att.output.weight"]))
    assert torch.equal(own["layers.0.mlp.mix_coeffs"][1], bf(sd["blocks.0.ffn.time_maa_r"].flatten()))
    assert torch.equal(own["layers.0.mlp.linear_down.weight"], bf(sd["blocks.0.ffn.value.weight"]))
    assert torch.equal(own["output_layer.weight"], bf(sd["head.weight"]))
    conv = pkg.modules.rwkv_lm_to_state_dict(sd, L)
    assert set(conv) == set(own)


def test_rejects_wrong_shapes_and_missing_keys(pkg):
    sd = ref.make_state_dict(C, H, F, L, V)
    bad = dict(sd)
    bad["blocks.0.att.key.weight"] = torch.zeros(C, C + 1)
    with pytest.raises(ValueError):
        _model(pkg, "cpu").from_rwkv_lm(bad)
    bad = dict(sd)
    del bad["blocks.1.ffn.time_maa_k"]
    with pytest.raises(KeyError):
        _model(pkg, "cpu").from_rwkv_lm(bad)


def test_pth_round_trip_weights_only(pkg, tmp_path):
    sd = ref.make_state_dict(C, H, F, L, V)
    path = os.path.join(tmp_path, "rwkv6.pth")
    torch.save(sd, path)
    back = pkg.modules.load_rwkv_lm(path)
    assert set(back) == set(sd) and all(torch.equal(back[k], sd[k]) for k in sd)


@pytest.mark.gpu
def test_converted_model_logits_match_rwkv_lm_forward(pkg):
    sd = ref.make_state_dict(C, H, F, L, V, seed=3)
    sd_bf = {k: v.to(torch.bfloat16).float() for k, v in sd.items()}    # what the model holds
    model = _model(pkg, "cuda:0").from_rwkv_lm(sd)
    tokens = torch.randint(0, V, (2, 96), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        logits = model(tokens.to("cuda:0")).float().cpu().numpy()
    want = ref.forward(sd_bf, tokens.numpy(), L, H)
    err = lambda a: (np.abs(a - want).max() / np.abs(want).max(),
                     np.linalg.norm(a - want) / np.linalg.norm(want))
    parity.check("logits", logits, want, tol_max=TOL, tol_l2=TOL, elem_mean=parity.ELEM_MEAN_BLOCK)
    # control: a converter that swapped two of the five token-shift mixes (k <-> v) is caught
    bad = dict(sd)
    for i in range(L):
        a = f"blocks.{i}.att."
        bad[a + "time_maa_k"], bad[a + "time_maa_v"] = sd[a + "time_maa_v"], sd[a + "time_maa_k"]
    model.from_rwkv_lm(bad)
    with torch.no_grad():
        wrong = model(tokens.to("cuda:0")).float().cpu().numpy()
    print(f"swapped-mix control: {err(wrong)[0]:.1e}/{err(wrong)[1]:.1e}")
    assert err(wrong)[1] > 3 * TOL
