"""GPU parity of the HIP WKV6 path (through the C ABI via the autograd drop-in)
against the CPU oracle on identical bf16 inputs.

Tolerance (bf16 I/O, fp32 accumulate): for every output tensor,
    max|gpu - oracle| / max|oracle|  <= 1e-2  and
    ||gpu - oracle||_2 / ||oracle||_2 <= 1e-2,
and the mean of the reference's elementwise metric |gpu - oracle| / (|oracle| + 1e-4)
(rwkv6_model.py:161-163) within parity.ELEM_MEAN_WKV, the same for every tensor, dw
included; its max is printed (tests/parity.py).
The oracle runs in fp64 on the same bf16-rounded inputs, so the error is the
kernels' own (bf16 MFMA operands, bf16 outputs).
"""
import numpy as np
import pytest
import torch

import parity
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def _inputs(B, H, T, seed, w_lo=-6.0, w_hi=-0.5, u_bf16=False):
    g = torch.Generator().manual_seed(seed)
    bf = lambda t: t.to(torch.bfloat16)
    K = V = 64
    r = bf(torch.randn(B, H, T, K, generator=g))
    k = bf(torch.randn(B, H, T, K, generator=g))
    v = bf(torch.randn(B, H, T, V, generator=g))
    w = bf(-torch.exp(torch.rand(B, H, T, K, generator=g) * (w_hi - w_lo) + w_lo))
    u = 0.1 * torch.randn(H, K, generator=g)
    if u_bf16:
        u = bf(u)
    h0 = 0.5 * torch.randn(B, H, K, V, generator=g)
    do = bf(torch.randn(B, H, T, V, generator=g))
    dht = torch.randn(B, H, K, V, generator=g)
    return dict(r=r, k=k, v=v, w=w, u=u, h0=h0, do=do, dht=dht)


def _n(t):
    return None if t is None else t.detach().float().cpu().numpy()


def run_gpu(pkg, x, scale, with_h0, with_dht, fn="chunk_rwkv6"):
    dev = torch.device("cuda:0")
    leaves = {n: x[n].to(dev).requires_grad_(True) for n in ("r", "k", "v", "w", "u")}
    h0 = x["h0"].to(dev).requires_grad_(True) if with_h0 else None
    op = getattr(pkg, fn)
    o, hT = op(leaves["r"], leaves["k"], leaves["v"], leaves["w"], leaves["u"], scale=scale,
               initial_state=h0, output_final_state=True)
    loss = (o.float() * x["do"].to(dev).float()).sum()
    if with_dht:
        loss = loss + (hT * x["dht"].to(dev)).sum()
    loss.backward()
    torch.cuda.synchronize()
    out = dict(o=_n(o), hT=_n(hT))
    for n in ("r", "k", "v", "w", "u"):
        out["d" + n] = _n(leaves[n].grad)
    if with_h0:
        out["dh0"] = _n(h0.grad)
    return out


def run_oracle(x, scale, with_h0, with_dht):
    a = {n: _n(t) for n, t in x.items()}
    h0 = a["h0"] if with_h0 else None
    dht = a["dht"] if with_dht else None
    o, hT = orc.wkv6_fwd(a["r"], a["k"], a["v"], a["w"], a["u"], h0, scale)
    g = orc.wkv6_bwd(a["r"], a["k"], a["v"], a["w"], a["u"], a["do"], h0, dht, scale)
    out = dict(o=o, hT=hT)
    out.update(g)
    return out


def _compare(got, ref, names, **bars):
    parity.check_all(got, ref, names, elem_mean=parity.ELEM_MEAN_WKV, **bars)


SHAPES = [(1, 1, 1), (2, 2, 63), (2, 2, 64), (2, 3, 130), (1, 2, 257)]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("state", [False, True])
def test_wkv_parity_small(pkg, shape, state):
    B, H, T = shape
    x = _inputs(B, H, T, seed=B * 1000 + H * 100 + T)
    scale = 1.0 if not state else 0.5
    got = run_gpu(pkg, x, scale, state, state)
    ref = run_oracle(x, scale, state, state)
    names = ["o", "hT", "dr", "dk", "dv", "dw", "du"] + (["dh0"] if state else [])
    _compare(got, ref, names)


def test_wkv_parity_bf16_u_and_fused_recurrent_name(pkg):
    x = _inputs(2, 2, 96, seed=7, u_bf16=True)
    got = run_gpu(pkg, x, 1.0, False, False, fn="fused_recurrent_rwkv6")
    assert got["du"] is not None
    ref = run_oracle(x, 1.0, False, False)
    _compare(got, ref, ["o", "dr", "dk", "dv", "dw", "du"])


def test_wkv_strong_decay(pkg):
    """Log-decay down to -exp(2.3) per token (much faster forgetting than the default init)."""
    x = _inputs(1, 2, 192, seed=9, w_lo=-3.0, w_hi=2.3)
    got = run_gpu(pkg, x, 1.0, True, True)
    ref = run_oracle(x, 1.0, True, True)
    _compare(got, ref, ["o", "hT", "dr", "dk", "dv", "dw", "du", "dh0"])


def test_wkv_extreme_decay_is_floored(pkg):
    """Log-decay down to -exp(5) ~ -148 per token: the kernels floor w at -10 (decay factor
    4.5e-5; the exact factor is below that, so outputs and states move by less than that
    relative amount); a floored token's dw is taken at the floor (scaled by the same
    factor, as the exact one is).  Outputs, states and gradients stay finite and match
    the exact fp64 oracle."""
    x = _inputs(1, 2, 130, seed=11, w_lo=-3.0, w_hi=5.0)
    got = run_gpu(pkg, x, 1.0, True, True)
    assert all(np.isfinite(v).all() for v in got.values())
    ref = run_oracle(x, 1.0, True, True)
    _compare(got, ref, ["o", "hT", "dr", "dk", "dv", "dw", "du", "dh0"])


@pytest.mark.parametrize("shape", [(2, 2, 200), (4, 6, 64 * 24 + 3), (2, 64, 64 * 17 + 5)])
def test_wkv_deterministic(pkg, shape):
    """Bit-identical reruns: the chunk-parallel backward (B*H = 4 and 24) and, at B*H = 128,
    the segmented forward and reverse walks (their pieces and folds sum in a fixed order)."""
    x = _inputs(*shape, seed=3)
    a = run_gpu(pkg, x, 1.0, True, True)
    b = run_gpu(pkg, x, 1.0, True, True)
    for n in a:
        assert np.array_equal(a[n], b[n]), n


def test_wkv_empty_sequence(pkg):
    dev = torch.device("cuda:0")
    B, H, K = 2, 2, 64
    r = torch.zeros(B, H, 0, K, dtype=torch.bfloat16, device=dev)
    u = torch.zeros(H, K, device=dev)
    h0 = torch.randn(B, H, K, K, device=dev)
    o, hT = pkg.chunk_rwkv6(r, r, r, r, u, scale=1.0, initial_state=h0, output_final_state=True)
    torch.cuda.synchronize()
    assert o.shape == (B, H, 0, K)
    assert torch.equal(hT, h0)


@pytest.mark.parametrize("shape", [(1, 2, 1100), (1, 1, 64 * 40 + 17), (2, 24, 64 * 32 + 11),
                                   (3, 32, 64 * 20), (2, 8, 64 * 64), (1, 32, 64 * 15 + 40),
                                   (2, 64, 64 * 17 + 5), (1, 128, 64 * 30 + 9),
                                   (1, 1, 64 * 72 + 10), (1, 1, 64 * 64 + 30)])
def test_wkv_parity_segmented(pkg, shape):
    """Few sequences of many chunks: the forward cuts each sequence into segments (pre-pass
    pieces folded into each segment's start state, then output walks), here 2 segments of 9
    chunks, 5 of 9 with a ragged last chunk, 4 of 9 (48 sequences), 2 of 10 (96 sequences),
    8 of 8 (16 sequences) and 2 of 8 with a ragged last chunk (32 sequences).  The backward
    runs chunk-parallel for those six (the (b,h, segment) walks would fill less than 7/8 of the
    device: 2, 5, 192, 192, 128 and 64 of 256) and as a segmented reverse walk (backward pieces
    folded into each segment's starting state gradient) for the 128-sequence shapes: 2
    segments of 9 chunks, and of 16 + 15 chunks with a ragged last one.  The pieces step two
    chunks at a time, so segments of an odd chunk count (9, 15) end on a one-chunk step.
    The last two shapes end the forward on a one-chunk (ragged, 10 tokens) and a two-chunk
    segment (9 and 8 segments of 9 chunks): the walk's decay scan runs two chunks ahead, so
    there its look-ahead stays on the segment's last chunk from the start."""
    B, H, T = shape
    x = _inputs(B, H, T, seed=T)
    got = run_gpu(pkg, x, 0.5, True, True)
    ref = run_oracle(x, 0.5, True, True)
    _compare(got, ref, ["o", "hT", "dr", "dk", "dv", "dw", "du", "dh0"])


# (B, H, T, with h0 / dhT) of the BASELINE.json WKV shapes: config 2 (isolated op), config 5
# (long context with carried state), and the per-layer WKV of config 3 (1.6B shape:
# B=4, C=2048 -> H=32, T=4096) and config 4 (7B shape: B=2, C=4096 -> H=64, T=8192), the
# last two with an initial state and a final-state gradient so every state path runs at
# the size the segmented forward and the chunk-parallel state gradients take
BASELINE_WKV = {"config2": (8, 32, 4096, False), "config5": (1, 32, 32768, True),
                "config3": (4, 32, 4096, True), "config4": (2, 64, 8192, True)}


@pytest.mark.parametrize("cfg", list(BASELINE_WKV))
def test_wkv_baseline_configs(pkg, cfg):
    """BASELINE.json WKV shapes at full size through chunk_rwkv6, against the fp64 oracle."""
    B, H, T, state = BASELINE_WKV[cfg]
    x = _inputs(B, H, T, seed=int(cfg[-1]))
    args = (1.0, state, state)
    print(f"{cfg}: B={B} H={H} T={T} h0/dhT={state}", flush=True)
    got = run_gpu(pkg, x, *args)
    ref = run_oracle(x, *args)
    names = ["o", "hT", "dr", "dk", "dv", "dw", "du"] + (["dh0"] if state else [])
    _compare(got, ref, names)


@pytest.mark.parametrize("cfg", ["config3", "config4"])
def test_wkv_seqfirst_baseline_configs(pkg, cfg):
    """The time-mix module's WKV entry (r, k, v, decay [T,B,H*64], w = -exp(decay) inside)
    at the per-layer shapes of configs 3 and 4, with h0, hT and a final-state gradient;
    d_decay = dw * w against the oracle."""
    B, H, T, _ = BASELINE_WKV[cfg]
    K = 64
    print(f"{cfg} seq-first: B={B} H={H} T={T}", flush=True)
    g = torch.Generator().manual_seed(30 + int(cfg[-1]))
    bf = lambda t: t.to(torch.bfloat16)
    r, k, v = (bf(torch.randn(T, B, H * K, generator=g)) for _ in range(3))
    decay = bf(torch.rand(T, B, H * K, generator=g) * 5.5 - 6.0)
    u = 0.1 * torch.randn(H, K, generator=g)
    h0 = 0.5 * torch.randn(B, H, K, K, generator=g)
    do = bf(torch.randn(B, H, T, K, generator=g))
    dht = torch.randn(B, H, K, K, generator=g)
    dev = torch.device("cuda:0")
    leaves = [t.to(dev).requires_grad_(True) for t in (r, k, v, decay, u, h0)]
    o, hT = pkg.wkv6_seqfirst(*leaves[:5], H, scale=1.0, initial_state=leaves[5], output_final_state=True)
    ((o.float() * do.to(dev).float()).sum() + (hT * dht.to(dev)).sum()).backward()
    torch.cuda.synchronize()
    got = dict(o=_n(o), hT=_n(hT), du=_n(leaves[4].grad), dh0=_n(leaves[5].grad))
    hf = lambda t: t.float().view(T, B, H, K).permute(1, 2, 0, 3).numpy()
    a = lambda t: t.detach().float().cpu()
    for name, leaf in zip(("dr", "dk", "dv", "dw"), leaves[:4]):
        got[name] = hf(a(leaf.grad))
    del leaves, o, hT
    w_hf = -np.exp(hf(decay).astype(np.float64))
    o_ref, hT_ref = orc.wkv6_fwd(hf(r), hf(k), hf(v), w_hf, u.numpy(), h0.numpy(), 1.0)
    gr = orc.wkv6_bwd(hf(r), hf(k), hf(v), w_hf, u.numpy(), _n(do), h0.numpy(), dht.numpy(), 1.0)
    ref = dict(o=o_ref, hT=hT_ref, dr=gr["dr"], dk=gr["dk"], dv=gr["dv"], du=gr["du"],
               dw=gr["dw"] * w_hf, dh0=gr["dh0"])
    _compare(got, ref, ["o", "hT", "dr", "dk", "dv", "dw", "du", "dh0"])


def test_wkv_decay_gradient_through_exp_past_the_floor(pkg):
    """The reference forms w = -exp(decay) in torch and hands it to the op (:336, :339), so
    autograd gives d decay = dw * w.  Decays up to 8 (w down to -2981, far below the kernels'
    -10 floor): a floored token's dw must be 0 (the derivative of the floored forward, within
    e^-10 of the exact one), or dw * w would grow like exp(decay).  d decay, and every other
    gradient, against the oracle's exact dw * w."""
    B, H, T, K = 2, 2, 150, 64
    g = torch.Generator().manual_seed(41)
    bf = lambda t: t.to(torch.bfloat16)
    r, k, v = (bf(torch.randn(B, H, T, K, generator=g)) for _ in range(3))
    decay = torch.rand(B, H, T, K, generator=g) * 11.0 - 3.0          # U(-3, 8)
    u = 0.1 * torch.randn(H, K, generator=g)
    do = bf(torch.randn(B, H, T, K, generator=g))
    dev = torch.device("cuda:0")
    leaves = [t.to(dev).requires_grad_(True) for t in (r, k, v, decay, u)]
    w = (-torch.exp(leaves[3])).to(torch.bfloat16)                      # as :336 under bf16
    o, _ = pkg.chunk_rwkv6(leaves[0], leaves[1], leaves[2], w, leaves[4], scale=1.0)
    (o.float() * do.to(dev).float()).sum().backward()
    torch.cuda.synchronize()
    wb = _n(w)
    o_ref, _ = orc.wkv6_fwd(_n(r), _n(k), _n(v), wb, u.numpy(), None, 1.0)
    gr = orc.wkv6_bwd(_n(r), _n(k), _n(v), wb, u.numpy(), _n(do), None, None, 1.0)
    got = dict(o=_n(o), dr=_n(leaves[0].grad), dk=_n(leaves[1].grad), dv=_n(leaves[2].grad),
               d_decay=_n(leaves[3].grad), du=_n(leaves[4].grad))
    ref = dict(o=o_ref, dr=gr["dr"], dk=gr["dk"], dv=gr["dv"], d_decay=gr["dw"] * wb, du=gr["du"])
    floored = wb < -10.0
    assert floored.mean() > 0.2
    assert np.all(got["d_decay"][floored] == 0.0)
    _compare(got, ref, ["o", "dr", "dk", "dv", "d_decay", "du"])


@pytest.mark.parametrize("shape", [(2, 2, 63), (3, 2, 130), (1, 3, 64), (2, 1, 1300), (2, 24, 2059),
                                   (2, 64, 1093)])
def test_wkv_seqfirst_entry(pkg, shape):
    """The time-mix module's entry: r, k, v, decay in [T,B,H*64], w = -exp(decay) inside,
    o head-first; d_decay = dw * w.  Checked against the oracle on the rearranged inputs.
    (2, 24, 2059): B*H = 48, 4 forward segments of 9 chunks and the chunk-parallel backward;
    (2, 64, 1093): B*H = 128, the segmented walks (2 segments of 9 chunks, ragged end), with
    scale 0.5 (the other shapes take RWKV-6's unit scale)."""
    B, H, T = shape
    K = 64
    scale = 0.5 if H == 64 else 1.0
    g = torch.Generator().manual_seed(T + B)
    bf = lambda t: t.to(torch.bfloat16)
    r, k, v = (bf(torch.randn(T, B, H * K, generator=g)) for _ in range(3))
    decay = bf(torch.rand(T, B, H * K, generator=g) * 5.5 - 6.0)
    u = 0.1 * torch.randn(H, K, generator=g)
    do = bf(torch.randn(B, H, T, K, generator=g))
    dev = torch.device("cuda:0")
    leaves = [t.to(dev).requires_grad_(True) for t in (r, k, v, decay, u)]
    o, _ = pkg.wkv6_seqfirst(*leaves, H, scale=scale)
    (o.float() * do.to(dev).float()).sum().backward()
    torch.cuda.synchronize()
    hf = lambda t: t.float().view(T, B, H, K).permute(1, 2, 0, 3).numpy()
    w_hf = -np.exp(hf(decay).astype(np.float64))
    a = lambda t: t.detach().float().cpu()
    o_ref, _ = orc.wkv6_fwd(hf(r), hf(k), hf(v), w_hf, u.numpy(), None, scale)
    gr = orc.wkv6_bwd(hf(r), hf(k), hf(v), w_hf, u.numpy(), _n(do), None, None, scale)
    got = dict(o=_n(o), du=_n(leaves[4].grad))
    for name, leaf in zip(("dr", "dk", "dv"), leaves[:3]):
        got[name] = hf(a(leaf.grad))
    got["dw"] = hf(a(leaves[3].grad))
    ref = dict(o=o_ref, dr=gr["dr"], dk=gr["dk"], dv=gr["dv"], du=gr["du"], dw=gr["dw"] * w_hf)
    _compare(got, ref, ["o", "dr", "dk", "dv", "dw", "du"])


def test_wkv_seqfirst_with_state(pkg):
    """Sequence-first entry with initial_state (grad), final state (with a loss on it) and
    decays from exp(-4) to exp(3) (w down to -20, past the -10 floor): h0, hT, dh0 and
    d_decay = dw * w against the oracle.  d_decay scales dw by |w|, so it shows any absolute
    error of dw under strong decay (a dw formed from a rounded chunk-end state that cancels
    against the chunk's own terms reaches 2.7e-2 of max here; the kernel stays near 3e-3)."""
    B, H, T, K = 2, 2, 100, 64
    g = torch.Generator().manual_seed(21)
    bf = lambda t: t.to(torch.bfloat16)
    r, k, v = (bf(torch.randn(T, B, H * K, generator=g)) for _ in range(3))
    decay = bf(torch.rand(T, B, H * K, generator=g) * 7.0 - 4.0)
    u = 0.1 * torch.randn(H, K, generator=g)
    h0 = 0.5 * torch.randn(B, H, K, K, generator=g)
    do = bf(torch.randn(B, H, T, K, generator=g))
    dht = torch.randn(B, H, K, K, generator=g)
    dev = torch.device("cuda:0")
    leaves = [t.to(dev).requires_grad_(True) for t in (r, k, v, decay, u, h0)]
    o, hT = pkg.wkv6_seqfirst(*leaves[:5], H, scale=1.0, initial_state=leaves[5], output_final_state=True)
    ((o.float() * do.to(dev).float()).sum() + (hT * dht.to(dev)).sum()).backward()
    torch.cuda.synchronize()
    hf = lambda t: t.float().view(T, B, H, K).permute(1, 2, 0, 3).numpy()
    w_hf = -np.exp(hf(decay).astype(np.float64))
    a = lambda t: t.detach().float().cpu()
    o_ref, hT_ref = orc.wkv6_fwd(hf(r), hf(k), hf(v), w_hf, u.numpy(), h0.numpy(), 1.0)
    gr = orc.wkv6_bwd(hf(r), hf(k), hf(v), w_hf, u.numpy(), _n(do), h0.numpy(), dht.numpy(), 1.0)
    got = dict(o=_n(o), hT=_n(hT), du=_n(leaves[4].grad), dh0=_n(leaves[5].grad))
    for name, leaf in zip(("dr", "dk", "dv", "dw"), leaves[:4]):
        got[name] = hf(a(leaf.grad))
    ref = dict(o=o_ref, hT=hT_ref, dr=gr["dr"], dk=gr["dk"], dv=gr["dv"], du=gr["du"],
               dw=gr["dw"] * w_hf, dh0=gr["dh0"])
    _compare(got, ref, ["o", "hT", "dr", "dk", "dv", "dw", "du", "dh0"])
