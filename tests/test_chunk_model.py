"""The chunked algorithm of the HIP kernels, modelled in fp64 numpy
(tests/wkv_chunk_model.py), equals the naive recurrence of the oracle.

This pins the kernel algebra (sub-block reference points, the three-phase
state scan, the suffix-sum form of dw) on the CPU, so a GPU mismatch can only
be an indexing or precision problem of the HIP code.
"""
import numpy as np
import pytest

from oracle import oracle as orc
import wkv_chunk_model as cm


def _rel(a, b):
    return float(np.abs(np.asarray(a) - np.asarray(b)).max() / max(np.abs(np.asarray(b)).max(), 1e-30))


def _inputs(B, H, T, K, V, seed, w_lo=-6.0, w_hi=-0.5):
    rng = np.random.default_rng(seed)
    f = lambda a: a.astype(np.float32)
    r, k = f(rng.standard_normal((B, H, T, K))), f(rng.standard_normal((B, H, T, K)))
    v = f(rng.standard_normal((B, H, T, V)))
    w = f(-np.exp(rng.uniform(w_lo, w_hi, (B, H, T, K))))
    u = f(0.1 * rng.standard_normal((H, K)))
    h0 = f(0.5 * rng.standard_normal((B, H, K, V)))
    dO = f(rng.standard_normal((B, H, T, V)))
    dhT = f(rng.standard_normal((B, H, K, V)))
    return r, k, v, w, u, h0, dO, dhT


@pytest.mark.parametrize("T", [1, 17, 64, 130, 200])
@pytest.mark.parametrize("state", [False, True])
def test_chunk_model_matches_recurrence(T, state):
    B, H, K, V = 1, 2, 16, 8
    r, k, v, w, u, h0, dO, dhT = _inputs(B, H, T, K, V, seed=T)
    h0 = h0 if state else None
    dhT = dhT if state else None
    o, hT = orc.wkv6_fwd(r, k, v, w, u, h0, 0.9)
    o_m, hT_m, _ = cm.fwd(r, k, v, w, u, h0, 0.9)
    assert _rel(o_m, o) < 1e-5 and _rel(hT_m, hT) < 1e-5
    g = orc.wkv6_bwd(r, k, v, w, u, dO, h0, dhT, 0.9)
    gm = cm.bwd(r, k, v, w, u, dO, h0, dhT, 0.9)
    for name in ("dr", "dk", "dv", "dw", "du", "dh0"):
        assert _rel(gm[name], g[name]) < 1e-5, name


def test_chunk_model_strong_decay():
    """Per-token log-decay down to -exp(2.3) ~ -10: the 8-token half sub-block sums
    stay below the fp32 exponent range, so the factorised products stay finite."""
    r, k, v, w, u, h0, dO, dhT = _inputs(1, 1, 96, 8, 8, seed=5, w_lo=-3.0, w_hi=2.3)
    o, hT = orc.wkv6_fwd(r, k, v, w, u, h0)
    o_m, hT_m, _ = cm.fwd(r, k, v, w, u, h0)
    assert _rel(o_m, o) < 1e-5 and _rel(hT_m, hT) < 1e-5
    g = orc.wkv6_bwd(r, k, v, w, u, dO, h0, dhT)
    gm = cm.bwd(r, k, v, w, u, dO, h0, dhT)
    for name in ("dr", "dk", "dv", "dw", "du", "dh0"):
        assert _rel(gm[name], g[name]) < 1e-5, name


@pytest.mark.parametrize("T", [1, 64, 130])
@pytest.mark.parametrize("strong", [False, True])
def test_midpoint_form_matches_recurrence(T, strong):
    lo, hi = (-3.0, 2.3) if strong else (-6.0, -0.5)
    r, k, v, w, u, h0, dO, dhT = _inputs(1, 2, T, 16, 8, seed=T + 7, w_lo=lo, w_hi=hi)
    o, _ = orc.wkv6_fwd(r, k, v, w, u, h0, 0.8)
    assert _rel(cm.fwd_mid(r, k, v, w, u, h0, 0.8), o) < 1e-5
    g = orc.wkv6_bwd(r, k, v, w, u, dO, h0, dhT, 0.8)
    gm = cm.bwd_mid(r, k, v, w, u, dO, h0, dhT, 0.8)
    for name in ("dr", "dk", "dv", "dw", "du", "dh0"):
        assert _rel(gm[name], g[name]) < 1e-5, name


@pytest.mark.parametrize("T", [64, 130])
def test_midpoint_form_extreme_decay_needs_split_factors(T):
    """Per-token log-decay down to -exp(5) ~ -148, floored at -10 as the kernels do.  With
    fp32-range exponentials the midpoint form stays exact only if each cross-block factor
    e^{mu_I - mu_J} is split at the source block's end (p_IJ q_J): the single factor spans
    16+ tokens and underflows for pairs that still matter (the control below)."""
    r, k, v, w, u, h0, dO, dhT = _inputs(1, 2, T, 16, 8, seed=T + 11, w_lo=-3.0, w_hi=5.0)
    w = np.maximum(w, -10.0).astype(np.float32)
    o, _ = orc.wkv6_fwd(r, k, v, w, u, h0, 1.0)
    assert _rel(cm.fwd_mid(r, k, v, w, u, h0, 1.0), o) < 1e-5
    g = orc.wkv6_bwd(r, k, v, w, u, dO, h0, dhT, 1.0)
    gm = cm.bwd_mid(r, k, v, w, u, dO, h0, dhT, 1.0)
    for name in ("dr", "dk", "dv", "dw", "du", "dh0"):
        assert _rel(gm[name], g[name]) < 1e-5, name
    # control: the unsplit factor loses those pairs
    assert _rel(cm.fwd_mid(r, k, v, w, u, h0, 1.0, split=False), o) > 1e-2


@pytest.mark.parametrize("T", [64, 130])
@pytest.mark.parametrize("strong", [False, True])
def test_walk_form_matches_recurrence(T, strong):
    """The forward walk's form (cross-block operands referenced at the end of the block
    before the target, built from the midpoint values times fp32-range table factors)
    equals the recurrence, also with per-token decays down to the -10 floor."""
    lo, hi = (-3.0, 5.0) if strong else (-6.0, -0.5)
    r, k, v, w, u, h0, dO, dhT = _inputs(1, 2, T, 16, 8, seed=T + 23, w_lo=lo, w_hi=hi)
    w = np.maximum(w, -10.0).astype(np.float32)
    o, hT = orc.wkv6_fwd(r, k, v, w, u, h0, 0.7)
    o_m, hT_m = cm.fwd_walk(r, k, v, w, u, h0, 0.7)
    assert _rel(o_m, o) < 1e-5 and _rel(hT_m, hT) < 1e-5
