"""Error metrics that every GPU parity test computes and prints for each tensor.

* ``max_rel`` = max|got - ref| / max|ref| and ``l2_rel`` = ||got - ref||_2 / ||ref||_2: the
  bars the tests assert (bf16 I/O with fp32 accumulation against an fp64 oracle on the same
  bf16-rounded inputs);
* the reference's own comparison, ``diff = |got - ref| / (|ref| + 1e-4)`` reduced to its max
  and mean (/root/reference/rwkv_megatron/rwkv6_model.py:161-163, where RWKV-Megatron
  compares its hidden states with the HF model's).  Its max is dominated by entries whose
  reference value is near zero (a bf16 output rounds to 2^-9 of its own magnitude, and an
  entry of 1e-3 next to entries of 1 gets an absolute error of ~1e-3 from the accumulation),
  so the tests bound its mean (budgets below, per kind of tensor) and print the max.
"""
from __future__ import annotations

import numpy as np

TOL_MAX = 1e-2
TOL_L2 = 1e-2
# Budgets for the mean of the reference's elementwise metric, per kind of tensor (about twice
# the largest value measured on MI355X across the GPU tests).  The mean is not asserted for
# tensors of fewer than MIN_ELEMS entries, where one near-zero reference entry decides it.
ELEM_MEAN = 5e-3         # elementwise kernels: one bf16 rounding of an fp32 result (<= 2.1e-3)
ELEM_MEAN_LORA = 8e-2    # kernels around bf16 hipBLASLt GEMMs (LoRA, channel-mix block; <= 3.8e-2)
# WKV o, final state and every gradient, dw and d_decay included (largest measured on MI355X:
# dw / d_decay 4.3e-2 in a sequence-first test, dv 3.6e-2, o 2.1e-2; at BASELINE config 2 dw is
# at 1.7e-2).  Its relative L2 error (<= 3.3e-3) is the same as every other WKV tensor's.
ELEM_MEAN_WKV = 6e-2
ELEM_MEAN_BLOCK = 3e-1   # whole blocks / layers / models, bf16 activations (<= 1.6e-1)
MIN_ELEMS = 4096
# Whole blocks / layers / models keep bf16 activations between the bf16 hipBLASLt GEMMs (as
# bf16 training does); each kernel on the way is pinned on its own at 1e-2.  The relative L2
# error is the bar that matters there; the max-normalised error of a tensor of millions of
# entries sits in the tail of the bf16 storage errors (up to 5.6e-2 measured on the 16.8 M
# entries of a 4096 x 4096 weight gradient whose l2_rel is 1.8e-2).
BLOCK_TOL_MAX = 1e-1
BLOCK_TOL_L2 = 3e-2
BLOCK_BARS = dict(tol_max=BLOCK_TOL_MAX, tol_l2=BLOCK_TOL_L2, elem_mean=ELEM_MEAN_BLOCK)
# A second bar for blocks, set by the reference rather than by measurement: the same block
# restated in oracle/lm.py and run under lm.bf16_storage() (fp64 compute, every op's output
# and every activation gradient rounded to bf16 once: the reference as it runs in bf16) has
# an error against the plain fp64 run; the GPU path's relative L2 error may be at most
# BF16_RATIO times that, plus BF16_L2_FLOOR for tensors the emulation happens to get almost
# exactly (a sum over many tokens whose roundings cancel).
BF16_RATIO = 1.5
BF16_L2_FLOOR = 2e-3


def metrics(got, ref) -> dict:
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    if ref.size == 0:
        return dict(max_rel=0.0, l2_rel=0.0, elem_max=0.0, elem_mean=0.0)
    d = np.abs(got - ref)
    diff = d / (np.abs(ref) + 1e-4)
    return dict(max_rel=float(d.max() / max(np.abs(ref).max(), 1e-30)),
                l2_rel=float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)),
                elem_max=float(diff.max()), elem_mean=float(diff.mean()))


def fmt(name: str, m: dict) -> str:
    return (f"{name}: max_rel {m['max_rel']:.1e} l2_rel {m['l2_rel']:.1e} | "
            f"ref-diff max {m['elem_max']:.1e} mean {m['elem_mean']:.1e}")


def check(name, got, ref, tol_max=TOL_MAX, tol_l2=TOL_L2, elem_mean=ELEM_MEAN) -> dict:
    """Prints all four metrics of one tensor and asserts the bars (elem_mean None: printed only)."""
    m = metrics(got, ref)
    print(fmt(name, m), flush=True)
    ok = m["max_rel"] <= tol_max and m["l2_rel"] <= tol_l2
    if elem_mean is not None and np.size(ref) >= MIN_ELEMS:
        ok = ok and m["elem_mean"] <= elem_mean
    assert ok, f"{name}: parity failed {m} (bars max_rel {tol_max}, l2_rel {tol_l2}, " \
               f"ref-diff mean {elem_mean})"
    return m


def check_all(got: dict, ref: dict, names, elem_mean_of=None, **bars) -> dict:
    """check() over several tensors; reports every one before failing.  elem_mean_of(name), if
    given, picks the reference-metric budget per tensor."""
    out, bad = {}, []
    for n in names:
        b = dict(bars)
        if elem_mean_of is not None:
            b["elem_mean"] = elem_mean_of(n)
        try:
            out[n] = check(n, got[n], ref[n], **b)
        except AssertionError as e:
            bad.append(str(e))
    assert not bad, "\n".join(bad)
    return out


def check_block(name, got, ref, emu, **bars) -> dict:
    """check() at the block bars, then the bar relative to the reference in bf16 storage:
    l2_rel(got, ref) <= BF16_RATIO * l2_rel(emu, ref) + BF16_L2_FLOOR."""
    m = check(name, got, ref, **bars)
    me = metrics(emu, ref)
    bound = BF16_RATIO * me["l2_rel"] + BF16_L2_FLOOR
    print(f"    {name}: reference in bf16 storage l2_rel {me['l2_rel']:.1e} -> bound {bound:.1e} "
          f"(ratio {m['l2_rel'] / max(me['l2_rel'], 1e-30):.2f})", flush=True)
    assert m["l2_rel"] <= bound, f"{name}: l2_rel {m['l2_rel']:.2e} above {bound:.2e} " \
                                 f"({BF16_RATIO} x the bf16-storage reference's {me['l2_rel']:.2e})"
    return m


def check_all_block(got: dict, ref: dict, emu: dict, names, **bars) -> dict:
    """check_block() over several tensors; reports every one before failing."""
    out, bad = {}, []
    for n in names:
        try:
            out[n] = check_block(n, got[n], ref[n], emu[n], **bars)
        except AssertionError as e:
            bad.append(str(e))
    assert not bad, "\n".join(bad)
    return out
