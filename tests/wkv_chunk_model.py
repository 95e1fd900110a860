"""fp64 numpy model of the chunked WKV6 algorithm the HIP kernels implement.

This is test infrastructure: it restates, step for step, the decomposition in
``rwkv-megatron_amd/csrc/wkv6.hip`` (64-token chunks, 16-token sub-blocks,
per-sub-block decay reference points, three-phase state scan, suffix-sum dw)
so that the algebra can be checked against the naive recurrence on the CPU,
independently of GPU indexing.

Chunk notation (per (b, h, chunk), tokens t = 0..63, channel i):
  G[t]   = sum_{s<=t} w[s]          inclusive cumulative log-decay in the chunk
  Gm1[t] = G[t-1], Gm1[0] = 0
  b_W    = G[16W-1] (0 for W=0)    reference at the start of sub-block W
  mu_W   = G[16W+7]                reference at the middle of sub-block W
  e_W    = G[16W+15]               reference at the end of sub-block W
Every exponent below is <= 0 except the diagonal-block factors around mu_W,
which are bounded by the decay of 8 tokens.
"""
import numpy as np

L = 64
SUB = 16


def _chunks(x, T, NT):
    """[..., T, D] -> [..., NT, 64, D] zero-padded."""
    pad = NT * L - T
    if pad:
        x = np.concatenate([x, np.zeros(x.shape[:-2] + (pad, x.shape[-1]))], axis=-2)
    return x.reshape(x.shape[:-2] + (NT, L, x.shape[-1]))


def _chunk_cumsum(wc):
    G = np.cumsum(wc, axis=-2)
    Gm1 = np.concatenate([np.zeros_like(G[..., :1, :]), G[..., :-1, :]], axis=-2)
    return G, Gm1


def fwd(r, k, v, w, u, h0=None, scale=1.0):
    r, k, v, w = (np.asarray(a, np.float64) for a in (r, k, v, w))
    u = np.asarray(u, np.float64)
    B, H, T, K = r.shape
    V = v.shape[-1]
    NT = (T + L - 1) // L
    rc, kc, vc, wc = (_chunks(a, T, NT) for a in (r, k, v, w))
    G, Gm1 = _chunk_cumsum(wc)
    GL = G[..., -1, :]                                        # [B,H,NT,K]
    # phase A: chunk-local state
    Sloc = np.einsum("bhcti,bhctj->bhcij", kc * np.exp(GL[..., None, :] - G), vc)
    # phase B: scan
    S = np.zeros((B, H, K, V)) if h0 is None else np.asarray(h0, np.float64).copy()
    S_in = np.empty((B, H, NT + 1, K, V))
    for c in range(NT):
        S_in[:, :, c] = S
        S = np.exp(GL[:, :, c])[..., None] * S + Sloc[:, :, c]
    S_in[:, :, NT] = S
    # phase C: output
    O = np.zeros((B, H, NT, L, V))
    bonus = np.einsum("bhcti,hi,bhcti->bhct", rc, u, kc)
    for W in range(L // SUB):
        tw = slice(SUB * W, SUB * W + SUB)
        bW = G[..., SUB * W - 1, :] if W > 0 else np.zeros_like(GL)
        muW = G[..., SUB * W + 7, :]
        rW, GW = rc[..., tw, :], Gm1[..., tw, :]
        # inter-chunk: (r e^{Gm1}) S_in
        O[..., tw, :] += np.einsum("bhcti,bhcij->bhctj", rW * np.exp(GW), S_in[:, :, :NT])
        # off-diagonal sub-blocks J < W, reference b_W
        if W > 0:
            ts = slice(0, SUB * W)
            Rb = rW * np.exp(GW - bW[..., None, :])
            Kb = kc[..., ts, :] * np.exp(bW[..., None, :] - G[..., ts, :])
            A = np.einsum("bhcti,bhcsi->bhcts", Rb, Kb)
            O[..., tw, :] += np.einsum("bhcts,bhcsj->bhctj", A, vc[..., ts, :])
        # diagonal sub-block, reference mu_W, strictly causal + u-bonus on the diagonal
        Rd = rW * np.exp(GW - muW[..., None, :])
        Kd = kc[..., tw, :] * np.exp(muW[..., None, :] - G[..., tw, :])
        A = np.einsum("bhcti,bhcsi->bhcts", Rd, Kd) * np.tril(np.ones((SUB, SUB)), -1)
        A += np.einsum("bhct,ts->bhcts", bonus[..., tw], np.eye(SUB))
        O[..., tw, :] += np.einsum("bhcts,bhcsj->bhctj", A, vc[..., tw, :])
    o = scale * O.reshape(B, H, NT * L, V)[:, :, :T]
    return o, S_in[:, :, NT], S_in


def bwd(r, k, v, w, u, dO, h0=None, dhT=None, scale=1.0):
    r, k, v, w, dO = (np.asarray(a, np.float64) for a in (r, k, v, w, dO))
    u = np.asarray(u, np.float64)
    B, H, T, K = r.shape
    V = v.shape[-1]
    NT = (T + L - 1) // L
    _, _, S_in = fwd(r, k, v, w, u, h0, scale)
    rc, kc, vc, wc, dc = (_chunks(a, T, NT) for a in (r, k, v, w, dO))
    dc = scale * dc
    G, Gm1 = _chunk_cumsum(wc)
    GL = G[..., -1, :]
    # phase A: chunk-local dstate: contribution of the chunk's outputs to dS at its start
    dSloc = np.einsum("bhcti,bhctj->bhcij", rc * np.exp(Gm1), dc)
    # phase B: reverse scan -> dS_out[c] = gradient of the state after chunk c
    dS = np.zeros((B, H, K, V)) if dhT is None else np.asarray(dhT, np.float64).copy()
    dS_out = np.empty((B, H, NT, K, V))
    for c in range(NT - 1, -1, -1):
        dS_out[:, :, c] = dS
        dS = np.exp(GL[:, :, c])[..., None] * dS + dSloc[:, :, c]
    dh0 = dS
    # phase C: gradients
    dA = np.einsum("bhctj,bhcsj->bhcts", dc, vc)               # dO_t . v_tau
    dd = np.einsum("bhctt->bhct", dA)
    bonus = np.einsum("bhcti,hi,bhcti->bhct", rc, u, kc)
    dr_h = np.zeros_like(rc)
    dk_h = np.zeros_like(kc)
    dv = np.einsum("bhcti,bhcij->bhctj", kc * np.exp(GL[..., None, :] - G), dS_out)
    S_out = S_in[:, :, 1:]
    D = np.einsum("bhcij,bhcij->bhci", S_out, dS_out)
    tril = np.tril(np.ones((SUB, SUB)), -1)
    for W in range(L // SUB):
        tw = slice(SUB * W, SUB * W + SUB)
        bW = G[..., SUB * W - 1, :] if W > 0 else np.zeros_like(GL)
        muW = G[..., SUB * W + 7, :]
        eW = G[..., SUB * W + 15, :]
        # dr for targets t in W
        acc = np.einsum("bhctj,bhcij->bhcti", dc[..., tw, :], S_in[:, :, :NT] * np.exp(bW)[..., None])
        if W > 0:
            ts = slice(0, SUB * W)
            acc += np.einsum("bhcts,bhcsi->bhcti", dA[..., tw, ts],
                             kc[..., ts, :] * np.exp(bW[..., None, :] - G[..., ts, :]))
        dr_h[..., tw, :] = np.exp(Gm1[..., tw, :] - bW[..., None, :]) * acc
        accd = np.einsum("bhcts,bhcsi->bhcti", dA[..., tw, tw] * tril,
                         kc[..., tw, :] * np.exp(muW[..., None, :] - G[..., tw, :]))
        dr_h[..., tw, :] += np.exp(Gm1[..., tw, :] - muW[..., None, :]) * accd
        # dk for sources tau in W
        acc = np.einsum("bhcsj,bhcij->bhcsi", vc[..., tw, :], dS_out * np.exp(GL - eW)[..., None])
        if W < L // SUB - 1:
            tt = slice(SUB * W + SUB, L)
            acc += np.einsum("bhcts,bhcti->bhcsi", dA[..., tt, tw],
                             rc[..., tt, :] * np.exp(Gm1[..., tt, :] - eW[..., None, :]))
        dk_h[..., tw, :] = np.exp(eW[..., None, :] - G[..., tw, :]) * acc
        accd = np.einsum("bhcts,bhcti->bhcsi", dA[..., tw, tw] * tril,
                         rc[..., tw, :] * np.exp(Gm1[..., tw, :] - muW[..., None, :]))
        dk_h[..., tw, :] += np.exp(muW[..., None, :] - G[..., tw, :]) * accd
        # dv intra: sum_{t >= tau} A[t, tau] dO_t
        for I in range(W, L // SUB):
            ti = slice(SUB * I, SUB * I + SUB)
            if I > W:
                Rb = rc[..., ti, :] * np.exp(Gm1[..., ti, :] - eW[..., None, :])
                Ke = kc[..., tw, :] * np.exp(eW[..., None, :] - G[..., tw, :])
                A = np.einsum("bhcti,bhcsi->bhcts", Rb, Ke)
            else:
                Rd = rc[..., ti, :] * np.exp(Gm1[..., ti, :] - muW[..., None, :])
                Kd = kc[..., tw, :] * np.exp(muW[..., None, :] - G[..., tw, :])
                A = np.einsum("bhcti,bhcsi->bhcts", Rd, Kd) * tril
                A += np.einsum("bhct,ts->bhcts", bonus[..., tw], np.eye(SUB))
            dv[..., tw, :] += np.einsum("bhcts,bhctj->bhcsj", A, dc[..., ti, :])
    dr = dr_h + u[None, :, None, None, :] * kc * dd[..., None]
    dk = dk_h + u[None, :, None, None, :] * rc * dd[..., None]
    x = rc * dr_h - kc * dk_h
    suffix = np.cumsum(x[..., ::-1, :], axis=-2)[..., ::-1, :] - x   # sum_{m > t}
    dw = suffix - kc * dk_h + D[..., None, :]
    du = np.einsum("bhcti,bhcti,bhct->hi", rc, kc, dd)
    cut = lambda a: a.reshape(B, H, NT * L, -1)[:, :, :T]
    return dict(dr=cut(dr), dk=cut(dk), dv=cut(dv), dw=cut(dw), du=du, dh0=dh0)


# ---------------------------------------------------------------------------
# Midpoint-referenced form (the form of the current kernels).  Per sub-block I,
# mu_I = G[16I+7]; stored operand tiles
#   Rm[t] = r_t e^{G_{t-1} - mu_I(t)},   Km[tau] = k_tau e^{mu_J(tau) - G_tau}
# are bounded by the decay of 8 tokens either way.  A cross-block pair (I > J) uses
# f_IJ = e^{mu_I - mu_J} split at the end b_J = G[16J+15] of the source block into
# p_IJ = e^{mu_I - b_J} and q_J = e^{b_J - mu_J}, one on each side of the contraction.
# Every exponential is evaluated with fp32's range (_ex: underflow below ~e^-103,
# overflow above e^88.7), as in the kernels, so split=False reproduces the single-factor
# form that loses pairs whose f underflows while their own decay is still O(1).
# ---------------------------------------------------------------------------

def _ex(x):
    with np.errstate(over="ignore", under="ignore"):
        return np.exp(np.asarray(x, np.float32)).astype(np.float64)


def _pq(G, mu, I, J, split):
    """(operand factor on the target side, factor on the source side) of block pair I > J."""
    if not split:
        return _ex(mu[..., I, :] - mu[..., J, :]), np.ones_like(mu[..., J, :])
    b = G[..., SUB * J + SUB - 1, :]
    return _ex(mu[..., I, :] - b), _ex(b - mu[..., J, :])

def _mid(G, Gm1):
    NB = L // SUB
    mu = np.stack([G[..., SUB * I + 7, :] for I in range(NB)], axis=-2)      # [...,4,K]
    blk = np.arange(L) // SUB
    mu_t = mu[..., blk, :]                                                      # [...,64,K]
    return mu, mu_t


def fwd_mid(r, k, v, w, u, h0=None, scale=1.0, split=True):
    r, k, v, w = (np.asarray(a, np.float64) for a in (r, k, v, w))
    u = np.asarray(u, np.float64)
    B, H, T, K = r.shape
    V = v.shape[-1]
    NT = (T + L - 1) // L
    _, _, S_in = fwd(r, k, v, w, u, h0, scale)          # scan phases are unchanged
    rc, kc, vc, wc = (_chunks(a, T, NT) for a in (r, k, v, w))
    G, Gm1 = _chunk_cumsum(wc)
    mu, mu_t = _mid(G, Gm1)
    Rm = rc * _ex(Gm1 - mu_t)
    Km = kc * _ex(mu_t - G)
    bonus = np.einsum("bhcti,hi,bhcti->bhct", rc, u, kc)
    O = np.zeros((B, H, NT, L, V))
    tril = np.tril(np.ones((SUB, SUB)), -1)
    for I in range(L // SUB):
        ti = slice(SUB * I, SUB * I + SUB)
        O[..., ti, :] += np.einsum("bhcti,bhcij->bhctj", Rm[..., ti, :] * _ex(mu[..., I, None, :]),
                                   S_in[:, :, :NT])
        for J in range(I + 1):
            tj = slice(SUB * J, SUB * J + SUB)
            if I == J:
                A = np.einsum("bhcti,bhcsi->bhcts", Rm[..., ti, :], Km[..., tj, :])
                A = A * tril + np.einsum("bhct,ts->bhcts", bonus[..., ti], np.eye(SUB))
            else:
                pf, qf = _pq(G, mu, I, J, split)
                A = np.einsum("bhcti,bhcsi->bhcts", Rm[..., ti, :] * pf[..., None, :],
                              Km[..., tj, :] * qf[..., None, :])
            O[..., ti, :] += np.einsum("bhcts,bhcsj->bhctj", A, vc[..., tj, :])
    return scale * O.reshape(B, H, NT * L, V)[:, :, :T]


def bwd_mid(r, k, v, w, u, dO, h0=None, dhT=None, scale=1.0, split=True):
    r, k, v, w, dO = (np.asarray(a, np.float64) for a in (r, k, v, w, dO))
    u = np.asarray(u, np.float64)
    B, H, T, K = r.shape
    V = v.shape[-1]
    NT = (T + L - 1) // L
    _, _, S_in = fwd(r, k, v, w, u, h0, scale)
    rc, kc, vc, wc, dc = (_chunks(a, T, NT) for a in (r, k, v, w, dO))
    dc = scale * dc
    G, Gm1 = _chunk_cumsum(wc)
    GL = G[..., -1, :]
    mu, mu_t = _mid(G, Gm1)
    dSloc = np.einsum("bhcti,bhctj->bhcij", rc * np.exp(Gm1), dc)
    dS = np.zeros((B, H, K, V)) if dhT is None else np.asarray(dhT, np.float64).copy()
    dS_out = np.empty((B, H, NT, K, V))
    for c in range(NT - 1, -1, -1):
        dS_out[:, :, c] = dS
        dS = np.exp(GL[:, :, c])[..., None] * dS + dSloc[:, :, c]
    dh0 = dS
    Rm = rc * _ex(Gm1 - mu_t)
    Km = kc * _ex(mu_t - G)
    Fm = _ex(Gm1 - mu_t)
    Fk = _ex(mu_t - G)
    dA = np.einsum("bhctj,bhcsj->bhcts", dc, vc)
    dd = np.einsum("bhctt->bhct", dA)
    bonus = np.einsum("bhcti,hi,bhcti->bhct", rc, u, kc)
    # D = rowsum(S_out dS) as the kernel forms it: e^{G_63} rowsum(S_in dS) plus the sum of
    # Km times the dS part of the dk accumulator (S_out = e^{G_63} S_in + S_loc, exactly)
    D = _ex(GL) * np.einsum("bhcij,bhcij->bhci", S_in[:, :, :NT], dS_out)
    tril = np.tril(np.ones((SUB, SUB)), -1)
    acc_r = np.zeros_like(rc)
    acc_k = np.zeros_like(kc)
    dv = np.zeros_like(vc)
    NB = L // SUB
    for W in range(NB):
        tw = slice(SUB * W, SUB * W + SUB)
        # dr accumulator (columns i): inter, off-diagonal, diagonal
        a = _ex(mu[..., W, :])[..., None, :] * np.einsum("bhctj,bhcij->bhcti", dc[..., tw, :], S_in[:, :, :NT])
        for J in range(W):
            tj = slice(SUB * J, SUB * J + SUB)
            pf, qf = _pq(G, mu, W, J, split)
            a += pf[..., None, :] * np.einsum("bhcts,bhcsi->bhcti", dA[..., tw, tj],
                                              Km[..., tj, :] * qf[..., None, :])
        a += np.einsum("bhcts,bhcsi->bhcti", dA[..., tw, tw] * tril, Km[..., tw, :])
        acc_r[..., tw, :] = a
        # dk accumulator
        a = _ex(GL - mu[..., W, :])[..., None, :] * np.einsum("bhcsj,bhcij->bhcsi", vc[..., tw, :], dS_out)
        D = D + (Km[..., tw, :] * a).sum(-2)
        for I in range(W + 1, NB):
            ti = slice(SUB * I, SUB * I + SUB)
            pf, qf = _pq(G, mu, I, W, split)
            a += qf[..., None, :] * np.einsum("bhcts,bhcti->bhcsi", dA[..., ti, tw],
                                              Rm[..., ti, :] * pf[..., None, :])
        a += np.einsum("bhcts,bhcti->bhcsi", dA[..., tw, tw] * tril, Rm[..., tw, :])
        acc_k[..., tw, :] = a
        # dv
        dv[..., tw, :] = np.einsum("bhcsi,bhcij->bhcsj", Km[..., tw, :] * _ex(GL - mu[..., W, :])[..., None, :],
                                   dS_out)
        for I in range(W, NB):
            ti = slice(SUB * I, SUB * I + SUB)
            if I == W:
                A = np.einsum("bhcti,bhcsi->bhcts", Rm[..., ti, :], Km[..., tw, :])
                A = A * tril + np.einsum("bhct,ts->bhcts", bonus[..., ti], np.eye(SUB))
            else:
                pf, qf = _pq(G, mu, I, W, split)
                A = np.einsum("bhcti,bhcsi->bhcts", Rm[..., ti, :] * pf[..., None, :],
                              Km[..., tw, :] * qf[..., None, :])
            dv[..., tw, :] += np.einsum("bhcts,bhctj->bhcsj", A, dc[..., ti, :])
    dr = Fm * acc_r + u[None, :, None, None, :] * kc * dd[..., None]
    dk = Fk * acc_k + u[None, :, None, None, :] * rc * dd[..., None]
    x = Rm * acc_r - Km * acc_k
    suffix = np.cumsum(x[..., ::-1, :], axis=-2)[..., ::-1, :] - x
    dw = suffix - Km * acc_k + D[..., None, :]
    du = np.einsum("bhcti,bhcti,bhct->hi", rc, kc, dd)
    cut = lambda a: a.reshape(B, H, NT * L, -1)[:, :, :T]
    return dict(dr=cut(dr), dk=cut(dk), dv=cut(dv), dw=cut(dw), du=du, dh0=dh0)


# ---------------------------------------------------------------------------
# Forward walk form (wkv6_fwd_walk).  Diagonal blocks use the midpoint tiles Rm, Km; the
# inter-chunk term Ri = Rm e^{mu_I} = r e^{G_{t-1}}; cross-block pairs (I > J) reference
# both operands at b_{I-1} = G[16I-1], the end of the block before the target block:
#   Rp[t]      = Rm[t] e^{mu_I - b_{I-1}}          = r_t e^{G_{t-1} - b_{I-1}}
#   Kc_I[tau]  = Km[tau] e^{b_{I-1} - mu_J}        = k_tau e^{b_{I-1} - G_tau}
# with every table factor evaluated in fp32 range (_ex), as the kernel forms them from the
# fp32 midpoint-referenced values.
# ---------------------------------------------------------------------------

def fwd_walk(r, k, v, w, u, h0=None, scale=1.0):
    r, k, v, w = (np.asarray(a, np.float64) for a in (r, k, v, w))
    u = np.asarray(u, np.float64)
    B, H, T, K = r.shape
    V = v.shape[-1]
    NT = (T + L - 1) // L
    _, hT, S_in = fwd(r, k, v, w, u, h0, scale)
    rc, kc, vc, wc = (_chunks(a, T, NT) for a in (r, k, v, w))
    G, Gm1 = _chunk_cumsum(wc)
    mu, mu_t = _mid(G, Gm1)
    Rm = rc * _ex(Gm1 - mu_t)
    Km = kc * _ex(mu_t - G)
    bonus = np.einsum("bhcti,hi,bhcti->bhct", rc, u, kc)
    O = np.zeros((B, H, NT, L, V))
    tril = np.tril(np.ones((SUB, SUB)), -1)
    for I in range(L // SUB):
        ti = slice(SUB * I, SUB * I + SUB)
        O[..., ti, :] += np.einsum("bhcti,bhcij->bhctj", Rm[..., ti, :] * _ex(mu[..., I, None, :]),
                                   S_in[:, :, :NT])
        A = np.einsum("bhcti,bhcsi->bhcts", Rm[..., ti, :], Km[..., ti, :])
        A = A * tril + np.einsum("bhct,ts->bhcts", bonus[..., ti], np.eye(SUB))
        O[..., ti, :] += np.einsum("bhcts,bhcsj->bhctj", A, vc[..., ti, :])
        if I > 0:
            bp = G[..., SUB * I - 1, :]
            Rp = Rm[..., ti, :] * _ex(mu[..., I, :] - bp)[..., None, :]
            for J in range(I):
                tj = slice(SUB * J, SUB * J + SUB)
                Kc = Km[..., tj, :] * _ex(bp - mu[..., J, :])[..., None, :]
                A = np.einsum("bhcti,bhcsi->bhcts", Rp, Kc)
                O[..., ti, :] += np.einsum("bhcts,bhcsj->bhctj", A, vc[..., tj, :])
    return scale * O.reshape(B, H, NT * L, V)[:, :, :T], hT
