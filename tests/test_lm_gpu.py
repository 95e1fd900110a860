"""BASELINE config 1 on the GPU: the tiny RWKV-6 language model (2 layers, d_model 512,
8 heads of 64, ffn 1792, vocab 65536, fp32 weights with normal(0, 0.02) init and RWKV-LM's
decay ramp), batch 2 x 512 uniform random token ids, one forward + backward with cross
entropy on next-token targets (the last position masked; pretrain_rwkv6.py:144-160).

The package runs it with fp32 parameters and bf16 activations (the kernels' dtype); the
checker is oracle/lm.py in fp64 on the same fp32 weights (rwkv6_model.py:28-37, :108-112;
rwkv6_layer_specs.py:431-550) with the C oracle's WKV.  Bars: the loss to 1e-3 relative;
logits and every parameter gradient parity.BLOCK_BARS (max_rel 1e-1, l2_rel 3e-2,
reference-metric mean 3e-1: bf16 activations through two layers), and a relative L2 error at
most 1.5x that of the same model run in bf16 storage (lm.bf16_storage()) plus 2e-3.
"""
import pytest
import torch
import torch.nn.functional as F

import parity
from oracle import lm

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
BARS = parity.BLOCK_BARS


def config1_batch(V=65536, B=2, T=512, seed=0):
    g = torch.Generator().manual_seed(seed)
    tokens = torch.randint(0, V, (B, T), generator=g)
    targets = torch.cat([tokens[:, 1:], torch.zeros(B, 1, dtype=tokens.dtype)], 1)
    mask = torch.ones(B, T)
    mask[:, -1] = 0
    return tokens, targets, mask


def test_config1_tiny_lm_forward_backward(pkg):
    M = pkg.modules
    cfg = M.TransformerConfig(hidden_size=512, num_attention_heads=8, ffn_hidden_size=1792,
                              num_layers=2, params_dtype=torch.float32, rwkv_lm_decay_init=True)
    V = 65536
    torch.manual_seed(0)
    model = M.RWKV6Model(cfg, V, device=DEV)
    tokens, targets, mask = config1_batch(V)

    logits = model(tokens.to(DEV))
    assert logits.shape == (512, 2, V) and logits.dtype == torch.bfloat16
    flat = logits.float().transpose(0, 1).reshape(-1, V)
    losses = F.cross_entropy(flat, targets.to(DEV).reshape(-1), reduction="none")
    m = mask.to(DEV).reshape(-1)
    loss = (losses * m).sum() / m.sum()
    loss.backward()
    torch.cuda.synchronize()

    def reference():
        p = lm.params_from_state_dict(model.state_dict())
        lg = lm.model_forward(p, tokens, cfg.num_layers, cfg.num_attention_heads,
                              cfg.layernorm_epsilon)
        ls = lm.lm_loss(lg, targets, mask)
        ls.backward()
        return lg, ls, p

    ref_logits, ref_loss, p = reference()
    with lm.bf16_storage():
        emu_logits, emu_loss, pe = reference()

    print(f"loss gpu {loss.item():.6f} ref {ref_loss.item():.6f} "
          f"bf16-storage ref {emu_loss.item():.6f}", flush=True)
    assert abs(loss.item() - ref_loss.item()) <= 1e-3 * abs(ref_loss.item())
    n = lambda t: t.detach().double().cpu().numpy()
    parity.check_block("logits", n(logits), n(ref_logits), n(emu_logits), **BARS)
    got = {name: n(prm.grad) for name, prm in model.named_parameters()}
    parity.check_all_block(got, {k: n(p[k].grad) for k in got}, {k: n(pe[k].grad) for k in got},
                           sorted(got), **BARS)


def test_config1_graph_replay_matches_eager(pkg):
    """The config-1 forward + backward captured once in a HIP graph (torch.cuda.CUDAGraph, the
    package's kernels launched on the capturing stream) and replayed: every replay, with eager
    GPU work and synchronizations between replays, gives the eager step's loss and parameter
    gradients (1e-6 relative bar; the kernels are deterministic)."""
    M = pkg.modules
    cfg = M.TransformerConfig(hidden_size=512, num_attention_heads=8, ffn_hidden_size=1792,
                              num_layers=2, params_dtype=torch.float32, rwkv_lm_decay_init=True)
    V = 65536
    torch.manual_seed(0)
    model = M.RWKV6Model(cfg, V, device=DEV)
    tokens, targets, mask = config1_batch(V)
    tok, tgt, m = tokens.to(DEV), targets.to(DEV).reshape(-1), mask.to(DEV).reshape(-1)

    def step():
        logits = model(tok)
        losses = F.cross_entropy(logits.float().transpose(0, 1).reshape(-1, V), tgt, reduction="none")
        loss = (losses * m).sum() / m.sum()
        loss.backward()
        return loss

    model.zero_grad(set_to_none=True)
    ref_loss = step().detach().clone()
    ref_grads = {n: p.grad.detach().clone() for n, p in model.named_parameters()}

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            model.zero_grad(set_to_none=True)
            step()
    torch.cuda.current_stream().wait_stream(side)
    model.zero_grad(set_to_none=True)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_loss = step()
    other = torch.randn(1024, 1024, device=DEV)
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        rel = abs(static_loss.item() - ref_loss.item()) / abs(ref_loss.item())
        worst = 0.0
        for n, p in model.named_parameters():
            d = (p.grad - ref_grads[n]).abs().max().item()
            s = ref_grads[n].abs().max().item()
            worst = max(worst, d / s if s > 0 else d)
        print(f"replay {rep}: loss rel diff {rel:.2e}, worst grad max-rel diff {worst:.2e}", flush=True)
        assert rel <= 1e-6 and worst <= 1e-6
        # eager work between replays (its own kernels, outside the model's gradients)
        with torch.no_grad():
            model(tok)
            other = other @ other.T / 1024
        torch.cuda.synchronize()
