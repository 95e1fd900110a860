"""Pins the CPU oracle (oracle/) before anything is compared against it.

The reference ships no tests or golden vectors for this path (the fla
submodule is empty), so every oracle function is pinned here by mathematics
that an independent computation fixes:

* WKV forward  == quadratic (attention-form) closed form with an explicit
  pairwise decay matrix, computed with torch fp64 einsum;
* special cases: w = 0 (causal linear attention), w -> -inf (only the
  previous token and the u-bonus survive), T = 1, segment splitting with a
  carried state, linearity in v;
* WKV backward == torch.autograd through that quadratic form (fp64),
  including u, h0 and a loss on the final state;
* GroupNorm == torch.nn.functional.group_norm (the routine the reference
  calls at rwkv6_layer_specs.py:91-97);
* shift / lerp / ddlerp / gate backward == torch.autograd through torch code
  shaped like the reference's own (rwkv6_layer_specs.py:290-300, :440-466).
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc


def _inputs(B, H, T, K, V, seed, w_lo=-6.0, w_hi=-0.5, h0=True):
    g = torch.Generator().manual_seed(seed)
    r = torch.randn(B, H, T, K, generator=g, dtype=torch.float64)
    k = torch.randn(B, H, T, K, generator=g, dtype=torch.float64)
    v = torch.randn(B, H, T, V, generator=g, dtype=torch.float64)
    x = torch.rand(B, H, T, K, generator=g, dtype=torch.float64) * (w_hi - w_lo) + w_lo
    w = -torch.exp(x)
    u = 0.1 * torch.randn(H, K, generator=g, dtype=torch.float64)
    hh = 0.5 * torch.randn(B, H, K, V, generator=g, dtype=torch.float64) if h0 else None
    # round to fp32 so the oracle (fp32 I/O) and the fp64 formulation see the same numbers
    f = lambda t: None if t is None else t.float().double()
    return f(r), f(k), f(v), f(w), f(u), f(hh)


def quadratic_wkv(r, k, v, w, u, h0, scale):
    """Attention form: o_t = s[(r_t e^{G_{t-1}}) h0 + sum_{tau<t} (r_t e^{G_{t-1}-G_tau} . k_tau) v_tau
    + (r_t u . k_t) v_t],  S_T = e^{G_T} h0 + sum_tau (k_tau e^{G_T-G_tau}) v_tau^T."""
    B, H, T, K = r.shape
    G = torch.cumsum(w, dim=2)                                  # inclusive
    Gm1 = torch.cat([torch.zeros_like(G[:, :, :1]), G[:, :, :-1]], dim=2)
    # pairwise decay D[t, tau, i] = exp(G_{t-1} - G_tau) for tau < t, else 0
    diff = Gm1[:, :, :, None, :] - G[:, :, None, :, :]           # [B,H,T,T,K]
    mask = torch.tril(torch.ones(T, T, dtype=torch.bool), diagonal=-1)
    D = torch.where(mask[None, None, :, :, None], torch.exp(torch.clamp(diff, max=0.0)), torch.zeros_like(diff))
    A = torch.einsum("bhti,bhsi,bhtsi->bhts", r, k, D)
    bonus = torch.einsum("bhti,hi,bhti->bht", r, u, k)
    o = torch.einsum("bhts,bhsv->bhtv", A, v) + bonus[..., None] * v
    GT = G[:, :, -1:, :]
    hT = torch.einsum("bhsi,bhsv->bhiv", k * torch.exp(GT - G), v)
    if h0 is not None:
        o = o + torch.einsum("bhti,bhiv->bhtv", r * torch.exp(Gm1), h0)
        hT = hT + torch.exp(GT[:, :, 0, :])[..., None] * h0
    return scale * o, hT


def _rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


@pytest.mark.parametrize("shape", [(2, 2, 37, 8, 6), (1, 3, 70, 16, 16), (1, 1, 1, 4, 4)])
@pytest.mark.parametrize("scale", [1.0, 0.7])
def test_fwd_equals_quadratic_closed_form(shape, scale):
    B, H, T, K, V = shape
    r, k, v, w, u, h0 = _inputs(B, H, T, K, V, seed=11)
    o, hT = orc.wkv6_fwd(r.numpy(), k.numpy(), v.numpy(), w.numpy(), u.numpy(), h0.numpy(), scale)
    o_ref, hT_ref = quadratic_wkv(r, k, v, w, u, h0, scale)
    assert _rel(o, o_ref) < 1e-5
    assert _rel(hT, hT_ref) < 1e-5


def test_fwd_zero_decay_is_causal_linear_attention():
    B, H, T, K, V = 1, 2, 25, 8, 8
    r, k, v, _, u, _ = _inputs(B, H, T, K, V, seed=3, h0=False)
    w = torch.zeros(B, H, T, K, dtype=torch.float64)
    o, hT = orc.wkv6_fwd(r.numpy(), k.numpy(), v.numpy(), w.numpy(), u.numpy())
    scores = torch.tril(r @ k.transpose(-1, -2), diagonal=-1)          # (r_t . k_tau), tau < t
    o_ref = scores @ v + ((r * u[None, :, None, :] * k).sum(-1, keepdim=True)) * v
    assert _rel(o, o_ref) < 1e-5
    assert _rel(hT, k.transpose(-1, -2) @ v) < 1e-5                     # S_T = sum_tau k v^T


def test_fwd_infinite_decay_keeps_only_previous_token():
    B, H, T, K, V = 1, 2, 9, 4, 5
    r, k, v, _, u, h0 = _inputs(B, H, T, K, V, seed=5)
    w = torch.full((B, H, T, K), -1e4, dtype=torch.float64)            # exp(w) == 0
    o, hT = orc.wkv6_fwd(r.numpy(), k.numpy(), v.numpy(), w.numpy(), u.numpy(), h0.numpy())
    bonus = (r * u[None, :, None, :] * k).sum(-1, keepdim=True) * v
    prev = torch.zeros_like(bonus)
    prev[:, :, 1:] = (r[:, :, 1:] * k[:, :, :-1]).sum(-1, keepdim=True) * v[:, :, :-1]
    prev[:, :, 0] = torch.einsum("bhi,bhiv->bhv", r[:, :, 0], h0)
    assert _rel(o, bonus + prev) < 1e-5
    assert _rel(hT, k[:, :, -1, :, None] * v[:, :, -1, None, :]) < 1e-5


def test_fwd_single_token():
    r, k, v, w, u, h0 = _inputs(2, 2, 1, 8, 8, seed=7)
    o, hT = orc.wkv6_fwd(r.numpy(), k.numpy(), v.numpy(), w.numpy(), u.numpy(), h0.numpy(), 0.5)
    o_ref = 0.5 * (torch.einsum("bhi,bhiv->bhv", r[:, :, 0], h0)
                   + (r[:, :, 0] * u * k[:, :, 0]).sum(-1, keepdim=True) * v[:, :, 0])
    hT_ref = torch.exp(w[:, :, 0])[..., None] * h0 + k[:, :, 0, :, None] * v[:, :, 0, None, :]
    assert _rel(o[:, :, 0], o_ref) < 1e-6
    assert _rel(hT, hT_ref) < 1e-6


def test_fwd_segment_split_carries_state():
    B, H, T, K, V = 2, 2, 50, 8, 8
    r, k, v, w, u, h0 = _inputs(B, H, T, K, V, seed=9)
    a = lambda t: t.numpy()
    o, hT = orc.wkv6_fwd(a(r), a(k), a(v), a(w), a(u), a(h0))
    cut = 23
    o1, h1 = orc.wkv6_fwd(a(r[:, :, :cut]), a(k[:, :, :cut]), a(v[:, :, :cut]), a(w[:, :, :cut]), a(u), a(h0))
    o2, h2 = orc.wkv6_fwd(a(r[:, :, cut:]), a(k[:, :, cut:]), a(v[:, :, cut:]), a(w[:, :, cut:]), a(u), h1)
    assert _rel(np.concatenate([o1, o2], axis=2), o) < 1e-6
    assert _rel(h2, hT) < 1e-6


def test_fwd_linear_in_v():
    r, k, v, w, u, _ = _inputs(1, 2, 30, 8, 8, seed=13, h0=False)
    v2 = torch.randn_like(v).float().double()
    a = lambda t: t.numpy()
    o1, _ = orc.wkv6_fwd(a(r), a(k), a(v), a(w), a(u))
    o2, _ = orc.wkv6_fwd(a(r), a(k), a(v2), a(w), a(u))
    o3, _ = orc.wkv6_fwd(a(r), a(k), (v + v2).float().numpy(), a(w), a(u))
    assert _rel(o3, o1 + o2) < 1e-5


@pytest.mark.parametrize("with_state", [False, True])
def test_bwd_equals_autograd_of_closed_form(with_state):
    B, H, T, K, V = 2, 2, 29, 8, 6
    scale = 0.8
    r, k, v, w, u, h0 = _inputs(B, H, T, K, V, seed=21, h0=with_state)
    g = torch.Generator().manual_seed(99)
    dO = torch.randn(B, H, T, V, generator=g, dtype=torch.float64).float().double()
    dhT = torch.randn(B, H, K, V, generator=g, dtype=torch.float64).float().double() if with_state else None
    leaves = [t.clone().requires_grad_(True) for t in (r, k, v, w, u)]
    h0l = h0.clone().requires_grad_(True) if with_state else None
    o, hT = quadratic_wkv(*leaves, h0l, scale)
    loss = (o * dO).sum()
    if with_state:
        loss = loss + (hT * dhT).sum()
    loss.backward()
    a = lambda t: None if t is None else t.detach().numpy()
    got = orc.wkv6_bwd(a(r), a(k), a(v), a(w), a(u), a(dO), a(h0), a(dhT), scale)
    for name, leaf in zip(("dr", "dk", "dv", "dw", "du"), leaves):
        assert _rel(got[name], leaf.grad) < 1e-5, name
    if with_state:
        assert _rel(got["dh0"], h0l.grad) < 1e-5


def test_bwd_dh0_without_state_is_gradient_at_zero():
    B, H, T, K, V = 1, 2, 17, 4, 4
    r, k, v, w, u, _ = _inputs(B, H, T, K, V, seed=23, h0=False)
    dO = torch.randn(B, H, T, V, dtype=torch.float64).float().double()
    z = torch.zeros(B, H, K, V, dtype=torch.float64, requires_grad=True)
    o, _ = quadratic_wkv(r, k, v, w, u, z, 1.0)
    (o * dO).sum().backward()
    a = lambda t: t.detach().numpy()
    got = orc.wkv6_bwd(a(r), a(k), a(v), a(w), a(u), a(dO))
    assert _rel(got["dh0"], z.grad) < 1e-5


# ---------------------------------------------------------------------------
# elementwise parts of the time-mix block
# ---------------------------------------------------------------------------

def _ref_torch_mix(x, maa, mexp, bias):
    """Torch code shaped like RWKV6TimeMix.forward :440-452 (non-SP token shift :294-300)."""
    shifted = torch.cat([torch.zeros_like(x.select(0, 0)).unsqueeze(0), x.narrow(0, 0, x.size(0) - 1)], 0)
    delta = shifted - x
    xxx = x + delta * maa
    m = mexp + bias
    mixed = x.unsqueeze(-2) + delta.unsqueeze(-2) * m
    return xxx, torch.stack(mixed.unbind(-2), 0)


def test_shift_lerp_and_ddlerp_forward_and_backward():
    T, B, C = 7, 3, 16
    g = torch.Generator().manual_seed(1)
    x = torch.randn(T, B, C, generator=g, dtype=torch.float64, requires_grad=True)
    maa = torch.rand(C, generator=g, dtype=torch.float64, requires_grad=True)
    mexp = torch.randn(T, B, 5, C, generator=g, dtype=torch.float64, requires_grad=True)
    bias = torch.randn(5, C, generator=g, dtype=torch.float64, requires_grad=True)
    xxx, mixed = _ref_torch_mix(x, maa, mexp, bias)
    d_xxx = torch.randn_like(xxx)
    d_mixed = torch.randn_like(mixed)
    ((xxx * d_xxx).sum() + (mixed * d_mixed).sum()).backward()
    n = lambda t: t.detach().numpy()
    assert _rel(orc.shift_lerp_fwd(n(x), n(maa)), n(xxx)) < 1e-12
    assert _rel(orc.ddlerp_fwd(n(x), n(mexp), n(bias)), n(mixed)) < 1e-12
    dx, dm, db, dmaa = orc.mix_bwd(n(x), n(maa), n(mexp), n(bias), n(d_mixed), n(d_xxx))
    assert _rel(dx, n(x.grad)) < 1e-12
    assert _rel(dm, n(mexp.grad)) < 1e-12
    assert _rel(db, n(bias.grad)) < 1e-12
    assert _rel(dmaa, n(maa.grad)) < 1e-12


def test_token_shift_first_row_zero():
    x = np.arange(24, dtype=np.float64).reshape(4, 2, 3)
    y = orc.token_shift(x)
    assert np.all(y[0] == 0) and np.all(y[1:] == x[:-1])


@pytest.mark.parametrize("groups,C", [(4, 64), (8, 512)])
def test_group_norm_matches_torch(groups, C):
    N = 33
    g = torch.Generator().manual_seed(2)
    x = torch.randn(N, C, generator=g, dtype=torch.float64) * 3 + 1
    gamma = torch.randn(C, generator=g, dtype=torch.float64)
    beta = torch.randn(C, generator=g, dtype=torch.float64)
    ref = torch.nn.functional.group_norm(x, groups, gamma, beta, eps=1e-5)
    y, _, _ = orc.group_norm_fwd(x.numpy(), groups, gamma.numpy(), beta.numpy(), 1e-5)
    assert _rel(y, ref) < 1e-12


def test_gn_gate_backward_matches_autograd():
    N, C, groups, eps = 21, 64, 4, 1e-5
    g = torch.Generator().manual_seed(4)
    o = torch.randn(N, C, generator=g, dtype=torch.float64, requires_grad=True)
    z = torch.randn(N, C, generator=g, dtype=torch.float64, requires_grad=True)
    gamma = torch.randn(C, generator=g, dtype=torch.float64, requires_grad=True)
    beta = torch.randn(C, generator=g, dtype=torch.float64, requires_grad=True)
    y = torch.nn.functional.group_norm(o, groups, gamma, beta, eps) * torch.nn.functional.silu(z)
    dy = torch.randn_like(y)
    (y * dy).sum().backward()
    n = lambda t: t.detach().numpy()
    y_o, _, _ = orc.gn_gate_fwd(n(o), n(z), groups, n(gamma), n(beta), eps)
    assert _rel(y_o, n(y)) < 1e-12
    do, dz, dgam, dbet = orc.gn_gate_bwd(n(o), n(z), groups, n(gamma), n(beta), eps, n(dy))
    assert _rel(do, n(o.grad)) < 1e-10
    assert _rel(dz, n(z.grad)) < 1e-12
    assert _rel(dgam, n(gamma.grad)) < 1e-12
    assert _rel(dbet, n(beta.grad)) < 1e-12


def test_bottleneck_matches_einops_pattern():
    T, B, C, E, R = 5, 2, 12, 5, 3
    g = torch.Generator().manual_seed(6)
    x = torch.randn(T, B, C, generator=g, dtype=torch.float64)
    wd = torch.randn(C, E, R, generator=g, dtype=torch.float64)
    wu = torch.randn(E, R, C, generator=g, dtype=torch.float64)
    b = torch.randn(E, C, generator=g, dtype=torch.float64)
    # the reference: einsum(x, W_down, "t b d, d e r -> t b e r").tanh(), then "t b e r, e r d -> t b e d"
    neck = torch.tanh((x.reshape(T * B, C) @ wd.reshape(C, E * R)).reshape(T, B, E, R))
    ref = torch.stack([neck[:, :, e] @ wu[e] for e in range(E)], dim=2) + b
    got = orc.bottleneck_fwd(x.numpy(), wd.numpy(), wu.numpy(), b.numpy())
    assert _rel(got, ref) < 1e-12


def test_bottleneck_backward_matches_autograd():
    T, B, C, E, R = 4, 3, 10, 5, 3
    g = torch.Generator().manual_seed(8)
    x = torch.randn(T, B, C, generator=g, dtype=torch.float64, requires_grad=True)
    wd = torch.randn(C, E, R, generator=g, dtype=torch.float64, requires_grad=True)
    wu = torch.randn(E, R, C, generator=g, dtype=torch.float64, requires_grad=True)
    b = torch.randn(E, C, generator=g, dtype=torch.float64, requires_grad=True)
    neck = torch.tanh(torch.einsum("tbd,der->tber", x, wd))
    m = torch.einsum("tber,erd->tbed", neck, wu) + b
    dm = torch.randn_like(m)
    (m * dm).sum().backward()
    n = lambda t: t.detach().numpy()
    dx, dwd, dwu, db = orc.bottleneck_bwd(n(x), n(wd), n(wu), n(dm))
    for got, ref in ((dx, x.grad), (dwd, wd.grad), (dwu, wu.grad), (db, b.grad)):
        assert _rel(got, ref) < 1e-12


def _ref_torch_channel_mix(x, mix, w_up, w_gate, w_down):
    """The reference's RWKV6ChannelMix.forward (rwkv6_layer_specs.py:512-536) in torch, TP=1."""
    shifted = torch.cat([torch.zeros_like(x[:1]), x[:-1]], 0)
    delta = shifted - x
    mixed = x.unsqueeze(-2) + delta.unsqueeze(-2) * mix
    mixed_up, mixed_gate = mixed.unbind(-2)
    h = torch.square(torch.relu(mixed_up @ w_up.T))
    out = h @ w_down.T
    return out * torch.sigmoid(mixed_gate @ w_gate.T)


def test_cmix_lerp_end_points():
    """mix = 0 passes x through, mix = 1 gives the token-shifted x (a sign or index slip in the
    delta fails one of the two)."""
    T, B, C = 5, 2, 8
    x = np.random.default_rng(0).standard_normal((T, B, C))
    mixed = orc.cmix_lerp_fwd(x, np.stack([np.zeros(C), np.ones(C)]))
    assert np.array_equal(mixed[0], x)
    assert np.allclose(mixed[1][1:], x[:-1]) and np.all(mixed[1][0] == 0)


def test_channel_mix_forward_and_backward_match_autograd():
    T, B, C, F = 6, 2, 16, 24
    g = torch.Generator().manual_seed(3)
    d = dict(dtype=torch.float64)
    x = torch.randn(T, B, C, generator=g, **d, requires_grad=True)
    mix = torch.rand(2, C, generator=g, **d, requires_grad=True)
    w_up = (0.3 * torch.randn(F, C, generator=g, **d)).requires_grad_(True)
    w_gate = (0.3 * torch.randn(C, C, generator=g, **d)).requires_grad_(True)
    w_down = (0.3 * torch.randn(C, F, generator=g, **d)).requires_grad_(True)
    y = _ref_torch_channel_mix(x, mix, w_up, w_gate, w_down)
    dy = torch.randn(y.shape, generator=g, **d)
    (y * dy).sum().backward()
    n = lambda t: t.detach().numpy()
    assert _rel(orc.channel_mix_fwd(n(x), n(mix), n(w_up), n(w_gate), n(w_down)), n(y)) < 1e-12
    got = orc.channel_mix_bwd(n(x), n(mix), n(w_up), n(w_gate), n(w_down), n(dy))
    for a, leaf in zip(got, (x, mix, w_up, w_gate, w_down)):
        assert _rel(a, n(leaf.grad)) < 1e-12


# ---------------------------------------------------------------------------------------
# oracle/lm.py: the whole-model restatement (checker for the layer / LM tests, config-1
# CPU baseline)
# ---------------------------------------------------------------------------------------

def test_lm_forward_matches_rwkv_lm_forward(pkg):
    """oracle.lm.model_forward (torch, the reference's module names and tensor shapes) equals
    the fp64 numpy forward written against RWKV-LM's own names (tests/rwkv_lm_reference.py,
    built from the numpy oracle pieces) on the same weights mapped by the checkpoint key map."""
    import rwkv_lm_reference as ref
    from oracle import lm

    C, H, F_, L, V = 128, 2, 448, 2, 200
    sd = ref.make_state_dict(C, H, F_, L, V, seed=5)
    p = lm.params_from_state_dict(pkg.modules.rwkv_lm_to_state_dict(sd, L), requires_grad=False)
    tokens = torch.randint(0, V, (2, 40), generator=torch.Generator().manual_seed(2))
    got = lm.model_forward(p, tokens, L, H).numpy()
    want = ref.forward(sd, tokens.numpy(), L, H)
    assert _rel(got, want) < 1e-6


def test_lm_wkv_wrapper_gradcheck():
    """The autograd wrapper around the C oracle against finite differences (the oracle's
    I/O is fp32, so the step is 1e-3 and the bars are loose; a dropped or swapped gradient
    fails by O(1))."""
    from oracle import lm

    g = torch.Generator().manual_seed(0)
    B, H, T, K = 1, 1, 5, 64
    r, k, v = (torch.randn(B, H, T, K, generator=g, dtype=torch.float64) for _ in range(3))
    w = -torch.exp(torch.rand(B, H, T, K, generator=g, dtype=torch.float64) * 3 - 3)
    u = 0.3 * torch.randn(H, K, generator=g, dtype=torch.float64)
    leaves = [t.requires_grad_(True) for t in (r, k, v, w, u)]
    assert torch.autograd.gradcheck(lm.OracleWKV.apply, leaves, eps=1e-3, atol=2e-3, rtol=2e-2)


def test_lm_loss_is_masked_mean_cross_entropy():
    from oracle import lm

    g = torch.Generator().manual_seed(1)
    T, B, V = 9, 3, 17
    logits = torch.randn(T, B, V, generator=g, dtype=torch.float64)
    tgt = torch.randint(0, V, (B, T), generator=g)
    mask = torch.ones(B, T)
    mask[:, -1] = 0
    got = lm.lm_loss(logits, tgt, mask)
    want = torch.nn.functional.cross_entropy(logits[:-1].transpose(0, 1).reshape(-1, V),
                                             tgt[:, :-1].reshape(-1))
    assert abs(float(got) - float(want)) < 1e-12


def test_lm_linear_with_and_without_bias_is_f_linear():
    """oracle/lm.py's linear (the TP = 1 Column/RowParallelLinear, bias when the layer has one)
    against torch.nn.functional.linear, the library routine."""
    from oracle import lm

    g = torch.Generator().manual_seed(0)
    x = torch.randn(5, 3, 16, generator=g, dtype=torch.float64)
    w = torch.randn(8, 16, generator=g, dtype=torch.float64)
    b = torch.randn(8, generator=g, dtype=torch.float64)
    assert torch.allclose(lm.linear({"l.weight": w}, "l", x), torch.nn.functional.linear(x, w))
    assert torch.allclose(lm.linear({"l.weight": w, "l.bias": b}, "l", x),
                          torch.nn.functional.linear(x, w, b))


def test_lm_bf16_storage_rounds_outputs_and_gradients():
    """lm.bf16_storage(): a storage point rounds its value and the gradient through it to bf16
    (torch's own bf16 conversion, round to nearest even) and is the identity outside; the
    channel mix run under it returns bf16-representable values, and it and its input gradient
    differ from the plain fp64 run by about bf16 rounding (2^-9 relative).  (The gradients of
    a tensor that several ops read are summed unrounded where they meet.)"""
    from oracle import lm

    g = torch.Generator().manual_seed(3)
    t = torch.randn(64, generator=g, dtype=torch.float64, requires_grad=True)
    gr = torch.randn(64, generator=g, dtype=torch.float64)
    assert lm.rb(t) is t
    with lm.bf16_storage():
        y = lm.rb(t)
    y.backward(gr)
    assert torch.equal(y.detach(), t.detach().to(torch.bfloat16).double())
    assert torch.equal(t.grad, gr.to(torch.bfloat16).double())
    assert lm.rb(t) is t                                   # the context is closed again

    C, F, T, B = 64, 128, 7, 2
    p = {"mix_coeffs": torch.rand(2, C, generator=g, dtype=torch.float64),
         "linear_up.weight": 0.1 * torch.randn(F, C, generator=g, dtype=torch.float64),
         "linear_down.weight": 0.1 * torch.randn(C, F, generator=g, dtype=torch.float64),
         "linear_gate.weight": 0.1 * torch.randn(C, C, generator=g, dtype=torch.float64)}
    x = torch.randn(T, B, C, generator=g, dtype=torch.float64)
    dy = torch.randn(T, B, C, generator=g, dtype=torch.float64)
    outs = []
    for storage in (False, True):
        xx = x.clone().requires_grad_(True)
        if storage:
            with lm.bf16_storage():
                y = lm.channel_mix(p, xx)
                y.backward(dy)
        else:
            y = lm.channel_mix(p, xx)
            y.backward(dy)
        outs.append((y.detach(), xx.grad))
    (y64, dx64), (yb, dxb) = outs
    assert torch.equal(yb, yb.to(torch.bfloat16).double())
    for a, b in ((yb, y64), (dxb, dx64)):
        rel = float(torch.linalg.norm(a - b) / torch.linalg.norm(b))
        assert 2.0 ** -12 < rel < 2.0 ** -5, rel
