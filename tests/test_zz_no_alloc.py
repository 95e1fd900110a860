"""rwkv6_wkv_fwd_noalloc, the forward entry point without a workspace argument, against
rwkv6_wkv_fwd on the same inputs through the C ABI: o, the final state and the saved chunk
states must be bit-identical (same kernels; only where the pre-pass keeps its segment states
differs).  Two calls in a row, the second with a smaller input, both on shapes whose forward
runs the segment pre-pass (B*H < 256), so the library's scratch array carries data; the second
call finds the first call's contents there.  The outputs are also checked against the CPU
oracle (max_rel / l2_rel 1e-2)."""
import ctypes

import pytest
import torch

import parity
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

# (B, H, T, with h0): 32 chunks in 4 segments x 16 sequences (48 segment states in the
# scratch array), then 18 chunks in 2 segments x 4 sequences (4 segment states)
CALLS = [(2, 8, 2000, True), (1, 4, 1100, False)]


def _inputs(B, H, T, seed):
    g = torch.Generator().manual_seed(seed)
    bf = lambda t: t.to(torch.bfloat16)
    r, k, v = (bf(torch.randn(B, H, T, 64, generator=g)) for _ in range(3))
    w = bf(-torch.exp(torch.rand(B, H, T, 64, generator=g) * 5.5 - 6.0))
    u = 0.1 * torch.randn(H, 64, generator=g)
    h0 = 0.5 * torch.randn(B, H, 64, 64, generator=g)
    return r, k, v, w, u, h0


def _forward(pkg, noalloc, r, k, v, w, u, h0):
    L = pkg._lib.load()
    B, H, T, K = r.shape
    P = lambda t: ctypes.c_void_p(0 if t is None else t.data_ptr())
    o = torch.empty_like(v)
    hT = torch.empty(B, H, K, K, dtype=torch.float32, device=DEV)
    saved = torch.empty(L.rwkv6_wkv_saved_bytes(B, H, T, K, K), dtype=torch.uint8, device=DEV)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    head = (P(r), P(k), P(v), P(w), P(u), pkg._lib.RWKV6_F32, P(h0), P(o), P(hT), P(saved))
    tail = (B, H, T, K, K, 1.0, stream)
    if noalloc:
        st = L.rwkv6_wkv_fwd_noalloc(*head, *tail)
    else:
        ws = torch.empty(L.rwkv6_wkv_workspace_bytes(B, H, T, K, K, 0), dtype=torch.uint8, device=DEV)
        st = L.rwkv6_wkv_fwd(*head, P(ws), *tail)
    pkg._lib.check(st, "wkv forward")
    torch.cuda.synchronize()
    return o.cpu(), hT.cpu(), saved.cpu()


def test_noalloc_forward_matches_workspace_forward(pkg):
    for i, (B, H, T, with_h0) in enumerate(CALLS):
        print(f"call {i}: B={B} H={H} T={T} h0={with_h0}", flush=True)
        r, k, v, w, u, h0 = _inputs(B, H, T, seed=i)
        dev = [t.to(DEV) for t in (r, k, v, w, u)]
        h0d = h0.to(DEV) if with_h0 else None
        want = _forward(pkg, False, *dev, h0d)
        got = _forward(pkg, True, *dev, h0d)
        for name, a, b in zip(("o", "hT", "saved"), got, want):
            assert torch.equal(a, b), f"call {i}: {name} differs from rwkv6_wkv_fwd"
        n = lambda t: t.float().numpy()
        o_ref, hT_ref = orc.wkv6_fwd(n(r), n(k), n(v), n(w), n(u), n(h0) if with_h0 else None, 1.0)
        parity.check(f"call {i} o", n(got[0]), o_ref, elem_mean=parity.ELEM_MEAN_WKV)
        parity.check(f"call {i} hT", n(got[1]), hT_ref, elem_mean=parity.ELEM_MEAN_WKV)


def _noalloc_args(pkg, r, k, v, w, u, h0, o, hT, saved):
    B, H, T, K = r.shape
    P = lambda t: ctypes.c_void_p(0 if t is None else t.data_ptr())
    return (P(r), P(k), P(v), P(w), P(u), pkg._lib.RWKV6_F32, P(h0), P(o), P(hT), P(saved),
            B, H, T, K, K, 1.0, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))


def test_noalloc_forward_replays_from_a_hip_graph(pkg):
    """The no-alloc forward captured in a HIP graph (torch.cuda.CUDAGraph) after one eager call
    on the device, replayed three times with eager no-alloc calls of another shape in between
    (they overwrite the shared scratch array): every replay is bit-identical to rwkv6_wkv_fwd."""
    L = pkg._lib.load()
    (B, H, T, _), (B2, H2, T2, _) = CALLS
    print(f"graph: B={B} H={H} T={T}, between replays B={B2} H={H2} T={T2}", flush=True)
    r, k, v, w, u, h0 = (t.to(DEV) for t in _inputs(B, H, T, seed=7))
    want = _forward(pkg, False, r, k, v, w, u, h0)
    o = torch.empty_like(v)
    hT = torch.empty(B, H, 64, 64, dtype=torch.float32, device=DEV)
    saved = torch.empty(L.rwkv6_wkv_saved_bytes(B, H, T, 64, 64), dtype=torch.uint8, device=DEV)
    other = [t.to(DEV) for t in _inputs(B2, H2, T2, seed=8)]
    o2 = torch.empty_like(other[2])
    hT2 = torch.empty(B2, H2, 64, 64, dtype=torch.float32, device=DEV)
    saved2 = torch.empty(L.rwkv6_wkv_saved_bytes(B2, H2, T2, 64, 64), dtype=torch.uint8, device=DEV)
    # the eager first call on the device (documented: set-up must not run under capture)
    pkg._lib.check(L.rwkv6_wkv_fwd_noalloc(*_noalloc_args(pkg, r, k, v, w, u, h0, o, hT, saved)),
                   "eager no-alloc forward")
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            st = L.rwkv6_wkv_fwd_noalloc(*_noalloc_args(pkg, r, k, v, w, u, h0, o, hT, saved))
    torch.cuda.current_stream().wait_stream(side)
    pkg._lib.check(st, "captured no-alloc forward")
    for rep in range(3):
        o.zero_()
        hT.zero_()
        saved.zero_()
        pkg._lib.check(L.rwkv6_wkv_fwd_noalloc(*_noalloc_args(pkg, *other[:5], None, o2, hT2, saved2)),
                       "eager no-alloc forward, other shape")
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, a, b in zip(("o", "hT", "saved"), (o.cpu(), hT.cpu(), saved.cpu()), want):
            assert torch.equal(a, b), f"replay {rep}: {name} differs from rwkv6_wkv_fwd"
        print(f"replay {rep}: bit-identical", flush=True)
    del graph


def test_noalloc_rejects_bad_shapes_before_launch(pkg):
    L = pkg._lib.load()
    p = ctypes.c_void_p(0x100000)
    assert L.rwkv6_wkv_fwd_noalloc(p, p, p, p, p, 1, None, p, None, p, 2, 2, 64, 32, 64, 1.0,
                                   None) == pkg._lib.RWKV6_ERR_UNSUPPORTED
