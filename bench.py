"""Benchmark of the RWKV-6 WKV6 hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

Workload ("config 2"): WKV6 forward + backward at
B=8, H=32, T=4096, K=V=64, bf16 r/k/v/w, fp32 u, h0 = 0, final state returned,
dO ~ N(0,1).  One step = one forward and one backward of chunk_rwkv6 through
the C ABI, inputs already resident in HBM.  value = tokens (B*T) per second.

Also reported:
  * per-phase kernel times, measured live with HIP events recorded by the
    library on the stream the kernels run on (rwkv6_wkv_*_ex);
  * roofline of the dominant kernel (the backward's gradient kernel, HBM-bound):
    algorithmic bytes per launch (reads r,k,v,w,dO + writes dr,dk,dv,dw = 1152 B per
    token-head) over its
    average event-timed duration, against 8 TB/s;
  * TFLOP/s of the whole op (fwd 32768 + bwd 65536 FLOP per token-head) and the
    fraction of the 2.5 PFLOP/s dense bf16 MFMA peak;
  * cpu_baseline: the CPU oracle (fp64 naive recurrence, C + OpenMP, a port of
    fla's naive recurrent RWKV-6) timed on this host on the same workload;
  * config5 (WKV6 long context with carried state), slice_7b (config 4: four 7B-shape
    layers fwd+bwd), train_step (config 3: the 1.6B-shape training step) and config1 (the
    tiny LM's fwd+bwd step on the GPU, eager and replayed from a HIP graph, and, as its CPU
    baseline, the reference model restated in torch fp32 on this host); the CPU baselines
    also give forward-only times, and
    cpu_host names the CPU model and thread counts.
"""
from __future__ import annotations

import argparse
import ctypes
import importlib
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "WKV6 fwd+bwd ms & % MFMA peak; RWKV6-1.6B-shape train tokens/s, 1 GPU"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FLOP_FWD = 32768          # per token-head, chunk 64, full tiles (2*64*(K+V) + 4*K*V)
FLOP_BWD = 65536
BYTES_BWD_GRADS = 1152    # per token-head: read r,k,v,w,dO, write dr,dk,dv,dw (bf16, K=V=64)
BYTES_FWD = 640           # per token-head: read r,k,v,w, write o


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=5, help="untimed steps first")
    ap.add_argument("--settle-s", type=float, default=0.3,
                    help="then untimed steps for this many seconds right before each timed WKV "
                         "region: the GPU raises its clocks only after ~30 ms of sustained load "
                         "and lowers them within milliseconds of idling (reported as settle_s)")
    ap.add_argument("--B", type=int, default=8)
    ap.add_argument("--H", type=int, default=32)
    ap.add_argument("--T", type=int, default=4096)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample-heads", type=int, default=0,
                    help="(b,h) sequences in the CPU sample (0 = the whole workload)")
    ap.add_argument("--no-train", action="store_true",
                    help="skip the config-3 training step (RWKV6 1.6B shape) measurement")
    ap.add_argument("--no-extra-configs", action="store_true",
                    help="skip the config-5 WKV and config-4 7B-slice measurements")
    ap.add_argument("--train-only", action="store_true",
                    help="run only the config-3 training step (for kernel profiles)")
    ap.add_argument("--config5-only", action="store_true",
                    help="run only the config-5 WKV measurement (for kernel profiles)")
    ap.add_argument("--train-steps", type=int, default=3)
    ap.add_argument("--train-warmup", type=int, default=2)
    ap.add_argument("--copy-calibration-mb", type=int, default=0,
                    help="after timing, run an elementwise copy kernel (dst = -src, plain vector loads "
                         "and stores) over this many MiB 3 times: the reference kernel of known size "
                         "for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE counters")
    return ap.parse_args()


def cpu_info():
    """The host the CPU baselines ran on: CPU model, logical CPUs, and the threads used."""
    import torch
    from oracle import oracle as orc

    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "os_cpu_count": os.cpu_count(),
            "torch_threads": torch.get_num_threads(), "oracle_omp_threads": orc.max_threads()}


def cpu_baseline(B, H, T, sample_heads, with_state=False):
    """Time the CPU oracle on this host: forward + backward (the reported value) and forward
    alone; returns the reported dict."""
    import numpy as np
    from oracle import oracle as orc

    n = B * H if sample_heads <= 0 else min(sample_heads, B * H)
    Hs = min(H, n)
    Bs = max(1, n // Hs)
    rng = np.random.default_rng(0)
    K = 64
    f = lambda *s: rng.standard_normal(s).astype(np.float32)
    r, k, v, dO = f(Bs, Hs, T, K), f(Bs, Hs, T, K), f(Bs, Hs, T, K), f(Bs, Hs, T, K)
    w = -np.exp(rng.uniform(-6, -0.5, (Bs, Hs, T, K))).astype(np.float32)
    u = (0.1 * f(Hs, K)).astype(np.float32)
    h0 = (0.5 * f(Bs, Hs, K, K)).astype(np.float32) if with_state else None
    dhT = f(Bs, Hs, K, K) if with_state else None
    threads = orc.max_threads()
    # one warm-up on a short prefix, then the median of 3 timed runs
    orc.wkv6_fwd(r[:, :, :64], k[:, :, :64], v[:, :, :64], w[:, :, :64], u)
    runs, fwd_runs = [], []
    for _ in range(3):
        t0 = time.perf_counter()
        orc.wkv6_fwd(r, k, v, w, u, h0)
        t1 = time.perf_counter()
        orc.wkv6_bwd(r, k, v, w, u, dO, h0, dhT)
        runs.append(time.perf_counter() - t0)
        fwd_runs.append(t1 - t0)
    dt = sorted(runs)[1]
    dt_f = sorted(fwd_runs)[1]
    frac = (Bs * Hs) / (B * H)
    tokens_per_s = (B * T) * frac / dt
    return {
        "value": tokens_per_s, "unit": "tokens/s", "cores": threads, "kind": "port",
        "sample": f"oracle fp64 naive recurrence fwd+bwd over {Bs*Hs} of {B*H} (b,h) sequences "
                  f"at T={T}{' with h0, dhT' if with_state else ''} (median of 3 runs, {dt:.2f} s), "
                  f"scaled to the whole B={B},H={H} job",
        "fwd_bwd_ms": dt / frac * 1e3, "fwd_ms": dt_f / frac * 1e3,
        "fwd_tokens_per_s": (B * T) * frac / dt_f,
    }


def config1_bench(pkg, gpu_steps, with_cpu):
    """the tiny RWKV-6 LM (2 layers, d_model 512, 8 heads, ffn 1792, vocab
    65536, fp32 weights with RWKV-LM's decay ramp), batch 2 x 512 random token ids, one
    forward + backward with next-token cross entropy (the last position masked).  GPU: the
    package's model (fp32 parameters, bf16 activations).  CPU: the reference's forward restated
    in torch fp32 with the C oracle's WKV (oracle/lm.py), 1 warm-up and the median of 3."""
    import torch
    import torch.nn.functional as F

    M = pkg.modules
    cfg = M.TransformerConfig(hidden_size=512, num_attention_heads=8, ffn_hidden_size=1792,
                              num_layers=2, params_dtype=torch.float32, rwkv_lm_decay_init=True)
    V, B, T = 65536, 2, 512
    torch.manual_seed(0)
    model = M.RWKV6Model(cfg, V, device="cuda:0")
    g = torch.Generator().manual_seed(0)
    tokens = torch.randint(0, V, (B, T), generator=g)
    targets = torch.cat([tokens[:, 1:], torch.zeros(B, 1, dtype=tokens.dtype)], 1)
    mask = torch.ones(B, T)
    mask[:, -1] = 0
    tok_d, tgt_d, mask_d = tokens.cuda(), targets.cuda().reshape(-1), mask.cuda().reshape(-1)

    def gpu_step():
        logits = model(tok_d)
        losses = F.cross_entropy(logits.float().transpose(0, 1).reshape(-1, V), tgt_d, reduction="none")
        loss = (losses * mask_d).sum() / mask_d.sum()
        loss.backward()
        model.zero_grad(set_to_none=True)
        return loss

    for _ in range(3):
        gpu_step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(gpu_steps):
        gpu_step()
    e1.record()
    torch.cuda.synchronize()
    gpu_ms = e0.elapsed_time(e1) / gpu_steps

    # The same step captured once in a HIP graph and replayed: the step is launch-bound
    # (~270 small kernels), which the graph's single submission removes.  Gradients land in
    # the graph's own .grad tensors, overwritten by every replay.
    def fwd_bwd():
        logits = model(tok_d)
        losses = F.cross_entropy(logits.float().transpose(0, 1).reshape(-1, V), tgt_d, reduction="none")
        loss = (losses * mask_d).sum() / mask_d.sum()
        loss.backward()
        return loss

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            model.zero_grad(set_to_none=True)
            fwd_bwd()
    torch.cuda.current_stream().wait_stream(side)
    model.zero_grad(set_to_none=True)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fwd_bwd()
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    e0.record()
    for _ in range(gpu_steps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    graph_ms = e0.elapsed_time(e1) / gpu_steps
    del graph
    model.zero_grad(set_to_none=True)
    out = {"workload": "BASELINE config 1: tiny RWKV-6 LM (2 layers, d_model 512, 8 heads, ffn 1792, "
                       "vocab 65536, fp32 weights), batch 2 x 512, fwd+bwd with next-token CE",
           "gpu_ms_per_step": gpu_ms, "gpu_tokens_per_s": B * T / (gpu_ms * 1e-3),
           "gpu_graph_ms_per_step": graph_ms, "gpu_graph_tokens_per_s": B * T / (graph_ms * 1e-3),
           "gpu_steps": gpu_steps,
           "gpu_precision": "fp32 parameters, bf16 activations: the GPU figures are a "
                            "bf16-activation step (the HIP kernels take bf16 r/k/v/w and "
                            "activations; the CPU baseline runs fp32 throughout)"}
    if with_cpu:
        from oracle import lm

        p = lm.params_from_state_dict(model.state_dict(), dtype=torch.float32)

        def cpu_step():
            loss = lm.lm_loss(lm.model_forward(p, tokens, cfg.num_layers, cfg.num_attention_heads,
                                               cfg.layernorm_epsilon), targets, mask)
            loss.backward()
            for t in p.values():
                t.grad = None

        cpu_step()
        runs = []
        for _ in range(3):
            t0 = time.perf_counter()
            cpu_step()
            runs.append(time.perf_counter() - t0)
        dt = sorted(runs)[1]
        out["cpu_baseline"] = {"value": B * T / dt, "unit": "tokens/s", "ms_per_step": dt * 1e3,
                               "cores": torch.get_num_threads(), "kind": "port",
                               "sample": "the whole config-1 step (torch fp32 restatement of the "
                                         "reference model, oracle/lm.py, with the C oracle's WKV), "
                                         "median of 3 runs after 1 warm-up"}
    del model
    torch.cuda.empty_cache()
    return out


def bwd_walk_segments(BH, T):
    """Segments per sequence of the library's reverse walk (wkv6_bwd_loop), 0 when the backward
    runs chunk-parallel: the rule of bwd_walk_segments() in csrc/wkv6.hip (walk_segments() with
    a 256-workgroup target; the walk when it is one segment or the segments fill 7/8 of it)."""
    NT = -(-T // 64)
    if NT <= 0:
        return 1
    P = min(max(1, 256 // BH), max(1, NT // 8))
    NC = -(-NT // P)
    P = -(-NT // NC)
    return P if P == 1 or 8 * BH * P >= 7 * 256 else 0


def bwd_kernel(BH, T):
    return "wkv6_bwd_loop" if bwd_walk_segments(BH, T) else "wkv6_bwd_chunk_grads"


def bwd_path(BH, T):
    P = bwd_walk_segments(BH, T)
    if P == 1:
        return "reverse walk (wkv6_bwd_loop)"
    if P > 1:
        return (f"segmented reverse walk ({P} segments: wkv6_bwd_pieces, wkv6_bwd_fold, "
                "wkv6_bwd_loop)")
    return "chunk-parallel (wkv6_bwd_chunk_dstate, wkv6_state_scan_bwd, wkv6_bwd_chunk_grads)"


def measured_traffic(B, H, T):
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3 counter runs
    (FETCH_SIZE and WRITE_SIZE, each scaled by the same counter on a copy of known size)."""
    path = os.path.join(ROOT, "profiles", bwd_kernel(B * H, T) + "_traffic.json")
    try:
        with open(path) as f:
            d = json.load(f)
    except (OSError, ValueError):
        return None
    if (d.get("B"), d.get("H"), d.get("T")) != (B, H, T):
        return None
    return d.get("traffic_bytes")


def settle(step, seconds):
    """Runs untimed steps for `seconds` of wall clock (checked every 10 steps, synchronised):
    the clocks of an idle GPU are low and rise under ~30 ms of sustained load.  Returns the
    seconds actually spent and the steps run."""
    import torch

    if seconds <= 0:
        return 0.0, 0
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    n = 0
    while time.perf_counter() - t0 < seconds:
        for _ in range(10):
            step()
        n += 10
        torch.cuda.synchronize()
    return time.perf_counter() - t0, n


def time_wkv(pkg, L, B, H, T, steps, warmup, with_state=False, settle_s=0.0):
    """WKV6 fwd+bwd through the C ABI (the _ex entries) on synthetic inputs resident in HBM.
    with_state: h0 ~ N(0, 0.5^2), dhT ~ N(0,1), dh0 returned (config 5).
    Three loops of `steps` steps after the warm-up: the timed region proper (ms_per_step) with
    no event inside it; the same steps with HIP events around the backward's gradient kernel,
    the roofline kernel, recorded by the library on the kernels' stream (its live average
    becomes bwd_phases[2]); and the same steps with an event around every phase for the rest
    of the breakdown.  Each event recorded between two kernels adds a gap to the stream (a
    few to tens of microseconds per step), which is why the step time comes from a loop
    without them.
    The warm-up steps and then `settle_s` seconds of steps (settle()) run right before the
    timed region, untimed.
    Returns (ms_per_step, fwd_ms, bwd_ms, fwd_phases, bwd_phases, ms_per_step_with_events,
    settle seconds, settle steps)."""
    import torch

    dev = torch.device("cuda:0")
    K = 64
    g = torch.Generator().manual_seed(0)
    bf = lambda t: t.to(torch.bfloat16).to(dev)
    r, k, v = (bf(torch.randn(B, H, T, K, generator=g)) for _ in range(3))
    w = bf(-torch.exp(torch.rand(B, H, T, K, generator=g) * 5.5 - 6.0))
    u = (0.1 * torch.randn(H, K, generator=g)).to(dev)
    do = bf(torch.randn(B, H, T, K, generator=g))
    h0 = (0.5 * torch.randn(B, H, K, K, generator=g)).to(dev) if with_state else None
    dhT = torch.randn(B, H, K, K, generator=g).to(dev) if with_state else None
    dh0 = torch.empty(B, H, K, K, dtype=torch.float32, device=dev) if with_state else None

    saved = torch.empty(L.rwkv6_wkv_saved_bytes(B, H, T, K, K), dtype=torch.uint8, device=dev)
    ws_f = torch.empty(L.rwkv6_wkv_workspace_bytes(B, H, T, K, K, 0), dtype=torch.uint8, device=dev)
    ws_b = torch.empty(L.rwkv6_wkv_workspace_bytes(B, H, T, K, K, 1), dtype=torch.uint8, device=dev)
    o = torch.empty_like(v)
    hT = torch.empty(B, H, K, K, dtype=torch.float32, device=dev)
    dr, dk, dv, dw = (torch.empty_like(r) for _ in range(4))
    du = torch.empty(H, K, dtype=torch.float32, device=dev)
    P = lambda t: ctypes.c_void_p(0 if t is None else t.data_ptr())
    stream = torch.cuda.current_stream(dev)
    sp = ctypes.c_void_p(stream.cuda_stream)
    ev = lambda: torch.cuda.Event(enable_timing=True)

    def step(fev=None, bev=None):
        fa = (ctypes.c_void_p * 6)(*[e.cuda_event for e in fev]) if fev else None
        ba = (ctypes.c_void_p * 8)(*[e.cuda_event if e else None for e in bev]) if bev else None
        pkg._lib.check(L.rwkv6_wkv_fwd_ex(P(r), P(k), P(v), P(w), P(u), pkg._lib.RWKV6_F32, P(h0), P(o),
                                          P(hT), P(saved), P(ws_f), B, H, T, K, K, 1.0, sp, fa), "fwd")
        pkg._lib.check(L.rwkv6_wkv_bwd_ex(P(r), P(k), P(v), P(w), P(u), pkg._lib.RWKV6_F32, P(do), P(dhT),
                                          P(saved), P(dr), P(dk), P(dv), P(dw), P(du), P(dh0), P(ws_b),
                                          B, H, T, K, K, 1.0, sp, ba), "bwd")

    fevs = [[ev() for _ in range(6)] for _ in range(steps)]
    bevs = [[ev() for _ in range(8)] for _ in range(steps)]
    gevs = [[ev() for _ in range(8)] for _ in range(steps)]   # only [4], [5] recorded
    t0, t1, t2, t3 = ev(), ev(), ev(), ev()
    for e in [x for evs in fevs + bevs + gevs for x in evs] + [t0, t1, t2, t3]:
        e.record(stream)               # torch creates the hipEvent_t on first record
    torch.cuda.synchronize()
    # the warm-up and the settle phase run right before the timed region: an idle GPU lowers
    # its clocks within milliseconds and takes ~30 ms of load to raise them again
    for _ in range(warmup):
        step()
    settled_s, settled_n = settle(step, settle_s)
    torch.cuda.synchronize()
    t0.record(stream)
    for i in range(steps):
        step()
    t1.record(stream)
    torch.cuda.synchronize()
    ms_step = t0.elapsed_time(t1) / steps
    t2.record(stream)
    for i in range(steps):
        step(None, [None, None, None, None, gevs[i][4], gevs[i][5], None, None])
    t3.record(stream)
    torch.cuda.synchronize()
    ms_step_ev = t2.elapsed_time(t3) / steps
    for i in range(steps):
        step(fevs[i], bevs[i])
    torch.cuda.synchronize()
    avg = lambda evs, a, b: sum(e[a].elapsed_time(e[b]) for e in evs) / len(evs)
    fwd_ph = [avg(fevs, 2 * p, 2 * p + 1) for p in range(3)]
    bwd_ph = [avg(bevs, 2 * p, 2 * p + 1) for p in range(4)]
    bwd_ph[2] = avg(gevs, 4, 5)        # the roofline kernel, from its own timed loop
    return ms_step, avg(fevs, 0, 5), avg(bevs, 0, 7), fwd_ph, bwd_ph, ms_step_ev, settled_s, settled_n


def config5_bench(pkg, L, args):
    """the long-context one-GPU share with carried state (h0, dhT, dh0):
    WKV6 fwd+bwd at B=1, H=32, T=32768 through the C ABI, timed as config 2 (time_wkv)."""
    B5, H5, T5 = 1, 32, 32768
    c5 = time_wkv(pkg, L, B5, H5, T5, args.steps, args.warmup, with_state=True,
                  settle_s=args.settle_s)
    return {"workload": "BASELINE config 5: WKV6 B=1, H=32, T=32768, h0 ~ N(0,0.5^2), "
                        "dhT ~ N(0,1), final state and dh0 returned",
            "ms_per_step": c5[0], "tokens_per_s": B5 * T5 / (c5[0] * 1e-3),
            "steps": args.steps, "warmup": args.warmup, "settle_s": c5[6],
            "settle_steps": c5[7], "fwd_ms": c5[1], "bwd_ms": c5[2],
            "phase_ms": {"fwd_segment_states": c5[3][0], "fwd_segment_fold": c5[3][1],
                         "fwd_walk": c5[3][2], "bwd_state_pre_pass": c5[4][0],
                         "bwd_state_fold_or_scan": c5[4][1], "bwd_grads": c5[4][2],
                         "bwd_du_reduce": c5[4][3]},
            "bwd_path": bwd_path(B5 * H5, T5),
            "tflops": B5 * H5 * T5 * (FLOP_FWD + FLOP_BWD) / (c5[0] * 1e-3) / 1e12}


def train_step_bench(pkg, steps, warmup):
    """RWKV-6 1.6B shape (24 layers, C=2048, 32 heads, ffn 7168, vocab 65536),
    batch 4 x 4096 random tokens, bf16 weights, full forward + backward + grad clip + AdamW.
    Returns tokens/s and the model-FLOP utilisation against 2.5 PFLOP/s dense bf16."""
    import torch

    M = pkg.modules
    cfg = M.TransformerConfig(hidden_size=2048, num_attention_heads=32, ffn_hidden_size=7168,
                              num_layers=24, params_dtype=torch.bfloat16)
    B, T, V = 4, 4096, 65536
    torch.manual_seed(0)
    model = M.RWKV6Model(cfg, V, device="cuda:0")
    n_params = sum(p.numel() for p in model.parameters())
    opt = torch.optim.AdamW(model.parameters(), lr=2.5e-4, betas=(0.9, 0.995), eps=1e-8,
                            weight_decay=0.1, fused=True)
    g = torch.Generator(device="cuda:0").manual_seed(1)
    tokens = torch.randint(0, V, (B, T + 1), device="cuda:0", generator=g)
    inp, tgt = tokens[:, :-1], tokens[:, 1:]

    def step():
        logits = model(inp)                                      # [T, B, V]
        loss = torch.nn.functional.cross_entropy(logits.float().view(-1, V), tgt.t().reshape(-1))
        loss.backward()
        torch.nn.utils.clip_grad_norm_(model.parameters(), 1.0)
        opt.step()
        opt.zero_grad(set_to_none=True)
        return loss

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        loss = step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    # 6 * (matmul parameters incl. the output head) per token, + the WKV op (fwd+bwd per token-head)
    emb = model.embedding.weight.numel()
    flop_tok = 6 * (n_params - emb) + cfg.num_layers * cfg.num_attention_heads * (FLOP_FWD + FLOP_BWD)
    tps = B * T / (ms * 1e-3)
    out = {"workload": "RWKV-6 1.6B-shape train step (BASELINE config 3): 24 layers, d_model 2048, "
                       "32 heads, ffn 7168, vocab 65536, batch 4 x 4096, bf16, fwd+bwd+clip+AdamW",
           "tokens_per_s": tps, "ms_per_step": ms, "params": n_params, "steps": steps, "warmup": warmup,
           "model_tflops": flop_tok * tps / 1e12, "mfu": flop_tok * tps / 1e12 / BF16_PEAK_TFLOPS,
           "final_loss": float(loss.item())}
    del model, opt
    torch.cuda.empty_cache()
    return out


def slice_7b_bench(pkg, steps, warmup):
    """4 RWKV-6 layers of the 7B shape (d_model 4096, 64 heads, ffn 14336),
    bf16 random-init weights, activations [8192, 2, 4096] ~ N(0,1) (sequence-first, as the
    reference), fwd + bwd through LN + time mix + channel mix + residual with dY ~ N(0,1)."""
    import torch

    M = pkg.modules
    cfg = M.TransformerConfig(hidden_size=4096, num_attention_heads=64, ffn_hidden_size=14336,
                              num_layers=4, params_dtype=torch.bfloat16)
    T, B, C = 8192, 2, 4096
    torch.manual_seed(0)
    layers = torch.nn.ModuleList(M.RWKV6Layer(cfg, i + 1, device="cuda:0") for i in range(4))
    g = torch.Generator(device="cuda:0").manual_seed(2)
    x = torch.randn(T, B, C, device="cuda:0", dtype=torch.bfloat16, generator=g).requires_grad_(True)
    dy = torch.randn(T, B, C, device="cuda:0", dtype=torch.bfloat16, generator=g)

    def step():
        y = x
        for layer in layers:
            y = layer(y)
        y.backward(dy)
        x.grad = None
        for p in layers.parameters():
            p.grad = None

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    # 6 * matmul parameters per token (2-D weights and the LoRA factors) + WKV fwd+bwd per token-head
    mm = sum(p.numel() for n, p in layers.named_parameters() if p.dim() >= 2)
    flop = 6 * mm * T * B + 4 * cfg.num_attention_heads * T * B * (FLOP_FWD + FLOP_BWD)
    out = {"workload": "BASELINE config 4: 4 RWKV-6 layers, d_model 4096, 64 heads, ffn 14336, "
                       "bf16, activations [8192, 2, 4096], fwd+bwd",
           "ms_per_step": ms, "tokens_per_s": T * B / (ms * 1e-3), "flop_per_step": flop,
           "tflops": flop / (ms * 1e-3) / 1e12, "mfu": flop / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
           "steps": steps, "warmup": warmup}
    del layers, x, dy
    torch.cuda.empty_cache()
    return out


def _extra(fn, *a):
    """One of the extra configurations; an exception there is recorded in its own field
    instead of costing the run its JSON line."""
    try:
        return fn(*a)
    except Exception as e:  # noqa: BLE001 -- reported, the headline line still prints
        return {"error": f"{type(e).__name__}: {e}"}


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the WKV6 path shards over B and H "
              "with no exchange; multi-GPU runs are out of scope).", file=sys.stderr)
        sys.exit(2)
    import torch

    pkg = importlib.import_module("rwkv-megatron_amd")
    L = pkg._lib.load()
    if args.train_only:
        print(json.dumps({"train_step": train_step_bench(pkg, args.train_steps, args.train_warmup)}),
              flush=True)
        return
    if args.config5_only:
        print(json.dumps({"config5": config5_bench(pkg, L, args)}), flush=True)
        return
    dev = torch.device("cuda:0")
    B, H, T, K = args.B, args.H, args.T, 64
    N_th = B * H * T

    ms_step, fwd_ms, bwd_ms, fwd_ph, bwd_ph, ms_step_ev, settle_s, settle_n = time_wkv(
        pkg, L, B, H, T, args.steps, args.warmup, settle_s=args.settle_s)

    grads_ms = bwd_ph[2]
    achieved = N_th * BYTES_BWD_GRADS / (grads_ms * 1e-3) / 1e9
    flops = N_th * (FLOP_FWD + FLOP_BWD)
    tflops = flops / (ms_step * 1e-3) / 1e12
    alg_bytes = N_th * (BYTES_FWD + BYTES_BWD_GRADS)
    out = {
        "metric": METRIC,
        "value": B * T / (ms_step * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "WKV6 fwd+bwd, BASELINE config 2 (chunk_rwkv6 via C ABI)",
                   "B": B, "H": H, "T": T, "K": K, "V": K, "h0": None, "output_final_state": True,
                   "parallelism": "single GPU"},
        "settle_s": settle_s,
        "settle_steps": settle_n,
        "ms_per_step_with_roofline_events": ms_step_ev,
        "wkv6_fwd_ms": fwd_ms,
        "wkv6_bwd_ms": bwd_ms,
        "wkv6_tflops": tflops,
        "wkv6_pct_bf16_mfma_peak": 100.0 * tflops / BF16_PEAK_TFLOPS,
        "wkv6_alg_hbm_frac": alg_bytes / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS,
        # bwd phases: state pre-pass (backward pieces, or chunk dS_loc), then their fold (or
        # the chunk scan), then the gradients (the walk, or the chunk gradient kernel), du
        "phase_ms": {"fwd_segment_states": fwd_ph[0], "fwd_walk": fwd_ph[2],
                     "bwd_state_pre_pass": bwd_ph[0], "bwd_state_fold_or_scan": bwd_ph[1],
                     "bwd_grads": bwd_ph[2], "bwd_du_reduce": bwd_ph[3]},
        "bwd_path": bwd_path(B * H, T),
        "roofline": {"kernel": bwd_kernel(B * H, T), "bound": "hbm", "achieved": achieved,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "traffic": measured_traffic(B, H, T)},
    }
    if not args.no_extra_configs:
        out["config5"] = _extra(config5_bench, pkg, L, args)
        if not args.no_cpu_baseline and "error" not in out["config5"]:
            out["config5"]["cpu_baseline"] = _extra(cpu_baseline, 1, 32, 32768, 0, True)
        out["slice_7b"] = _extra(slice_7b_bench, pkg, args.train_steps, args.train_warmup)
    if args.copy_calibration_mb > 0:
        n = args.copy_calibration_mb * (1 << 20) // 2
        src = torch.empty(n, dtype=torch.bfloat16, device=dev).normal_()
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(3):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        out["copy_calibration_bytes"] = 2 * n
    if not args.no_train:
        out["train_step"] = _extra(train_step_bench, pkg, args.train_steps, args.train_warmup)
    if not args.no_extra_configs:
        out["config1"] = _extra(config1_bench, pkg, max(5, args.steps // 2), not args.no_cpu_baseline)
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = _extra(cpu_baseline, B, H, T, args.cpu_sample_heads)
        out["cpu_host"] = _extra(cpu_info)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
