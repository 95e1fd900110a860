"""CPU checks of the C-ABI library: it loads, exports every symbol the header
declares, and its argument validation rejects bad calls before touching the GPU."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "rwkv6_amd.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(rwkv6_\w+)\s*\(", text)))


def test_header_declares_entry_points():
    names = _declared()
    for must in ("rwkv6_wkv_fwd", "rwkv6_wkv_bwd", "rwkv6_shift_lerp_fwd", "rwkv6_ddlerp_lora_fwd",
                 "rwkv6_ddlerp_lora_bwd", "rwkv6_lora_bias_fwd", "rwkv6_gn_gate_fwd",
                 "rwkv6_gn_gate_bwd", "rwkv6_strerror"):
        assert must in names


def test_library_exports_every_declared_symbol(pkg):
    lib = ctypes.CDLL(pkg._lib.LIB_PATH)
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, missing
    # and the ctypes signature table covers exactly the header
    assert sorted(pkg._lib.SIGNATURES) == _declared()


def test_version_and_strerror(pkg):
    L = pkg._lib.load()
    assert L.rwkv6_abi_version() == pkg._lib.ABI_VERSION == 3
    assert L.rwkv6_strerror(0) == b"ok"
    assert b"64" in L.rwkv6_strerror(2)
    assert L.rwkv6_strerror(12345) == b"unknown rwkv6 status code"


def test_workspace_sizes(pkg):
    L = pkg._lib.load()
    B, H, T = 8, 32, 4096
    NT = T // 64
    saved = L.rwkv6_wkv_saved_bytes(B, H, T, 64, 64)
    assert saved >= B * H * (NT + 1) * 64 * 64 * 2                  # bf16 state per chunk + final
    # forward: no per-chunk state (the walk carries it); per-segment states only when B*H
    # is far below the device's workgroup count (config 5: 32 sequences of 512 chunks)
    assert 0 < L.rwkv6_wkv_workspace_bytes(B, H, T, 64, 64, 0) < 16 << 20
    assert L.rwkv6_wkv_workspace_bytes(1, 32, 32768, 64, 64, 0) >= 32 * 64 * 64 * 4
    # backward, one reverse walk per sequence (B*H fills the device): only the fp32 du
    # partials of each (b,h); config 5 (B*H = 32, 8 segments of 64 chunks): du partials per
    # (b,h, segment), the 7 later segments' piece states (fp32 dS and decay) and the 7
    # segment-start state gradients, all far below a per-chunk state
    assert 0 < L.rwkv6_wkv_workspace_bytes(B, H, T, 64, 64, 1) < 1 << 20
    assert L.rwkv6_wkv_workspace_bytes(B, H, T, 64, 64, 1) >= B * H * 64 * 4
    c5 = L.rwkv6_wkv_workspace_bytes(1, 32, 32768, 64, 64, 1)
    assert 32 * (8 * 64 * 4 + 7 * (64 * 64 * 4 + 64 * 4) + 7 * 64 * 64 * 4) <= c5 < 16 << 20
    assert L.rwkv6_wkv_saved_bytes(B, H, T, 32, 64) == 0          # unsupported head size


def _fake(addr):
    return ctypes.c_void_p(addr)


def test_validation_rejects_before_launch(pkg):
    """Bad calls return an error code without dereferencing anything (the pointers are fake)."""
    L = pkg._lib.load()
    p = _fake(0x100000)
    args = lambda K=64, u_dt=1, r=p, saved=p: (r, p, p, p, p, u_dt, None, p, None, saved, p,
                                               2, 2, 64, K, 64, 1.0, None)
    assert L.rwkv6_wkv_fwd(*args(K=32)) == pkg._lib.RWKV6_ERR_UNSUPPORTED
    assert L.rwkv6_wkv_fwd(*args(u_dt=7)) == pkg._lib.RWKV6_ERR_INVALID_ARG
    assert L.rwkv6_wkv_fwd(*args(r=None)) == pkg._lib.RWKV6_ERR_INVALID_ARG
    assert L.rwkv6_wkv_fwd(*args(saved=None)) == pkg._lib.RWKV6_ERR_INVALID_ARG
    assert L.rwkv6_wkv_fwd(*args(r=_fake(0x100002))) == pkg._lib.RWKV6_ERR_ALIGNMENT
    assert L.rwkv6_shift_lerp_fwd(p, p, 1, p, 4, 2, 12, None) == pkg._lib.RWKV6_ERR_UNSUPPORTED
    assert L.rwkv6_lora_bias_fwd(p, p, p, 3, p, 4, 1, 64, 32, None) == pkg._lib.RWKV6_ERR_INVALID_ARG
    assert L.rwkv6_lora_bias_fwd(p, p, p, 1, p, 4, 3, 64, 32, None) == pkg._lib.RWKV6_ERR_UNSUPPORTED
    assert L.rwkv6_lora_bias_fwd(p, p, p, 1, p, 4, 0, 64, 32, None) == pkg._lib.RWKV6_ERR_INVALID_ARG
    assert L.rwkv6_gn_gate_fwd(p, 1, p, p, p, 0, 1e-5, p, p, p, 4, 2, 2, 32, None) == \
        pkg._lib.RWKV6_ERR_UNSUPPORTED
    assert L.rwkv6_gn_gate_fwd(None, 1, p, p, p, 0, 1e-5, p, p, p, 4, 2, 2, 64, None) == \
        pkg._lib.RWKV6_ERR_INVALID_ARG
    E = pkg._lib
    assert L.rwkv6_cmix_lerp_fwd(p, p, 1, p, 4, 2, 12, None) == E.RWKV6_ERR_UNSUPPORTED
    assert L.rwkv6_cmix_lerp_fwd(p, None, 1, p, 4, 2, 16, None) == E.RWKV6_ERR_INVALID_ARG
    assert L.rwkv6_cmix_lerp_bwd(p, p, 1, p, p, p, None, 4, 2, 16, None) == E.RWKV6_ERR_INVALID_ARG
    assert L.rwkv6_relu_sq_fwd(p, p, 12, None) == E.RWKV6_ERR_UNSUPPORTED
    assert L.rwkv6_relu_sq_fwd(p, p, -8, None) == E.RWKV6_ERR_INVALID_ARG
    assert L.rwkv6_relu_sq_bwd(p, None, p, 16, None) == E.RWKV6_ERR_INVALID_ARG
    assert L.rwkv6_sigmoid_gate_fwd(p, _fake(0x100008), p, 16, None) == E.RWKV6_ERR_ALIGNMENT
    assert L.rwkv6_sigmoid_gate_bwd(p, p, p, p, None, 16, None) == E.RWKV6_ERR_INVALID_ARG
    assert L.rwkv6_relu_sq_fwd(None, None, 0, None) == E.RWKV6_OK       # empty: nothing to do


def test_overlapping_outputs_are_rejected(pkg):
    """An output that overlaps an input (or another output) is refused before any launch:
    several kernels re-load a clamped last piece after other threads stored theirs, and the
    walks read chunk c + 1 before storing chunk c (the pointers are fake; nothing is read)."""
    L = pkg._lib.load()
    E = pkg._lib
    a, b, c, d = (_fake(0x100000 * i) for i in (1, 2, 3, 4))
    inside = _fake(0x100000 + 16)                                   # 16 bytes into a
    assert L.rwkv6_relu_sq_fwd(a, a, 16, None) == E.RWKV6_ERR_INVALID_ARG
    assert L.rwkv6_relu_sq_fwd(a, inside, 16, None) == E.RWKV6_ERR_INVALID_ARG
    assert L.rwkv6_sigmoid_gate_bwd(a, b, c, d, d, 16, None) == E.RWKV6_ERR_INVALID_ARG
    assert L.rwkv6_sigmoid_gate_fwd(a, b, inside, 16, None) == E.RWKV6_ERR_INVALID_ARG
    assert L.rwkv6_shift_lerp_fwd(a, b, 1, a, 4, 2, 16, None) == E.RWKV6_ERR_INVALID_ARG
    # WKV forward: o on top of v
    assert L.rwkv6_wkv_fwd(a, b, c, d, _fake(0x500000), 1, None, c, None, _fake(0x600000),
                           _fake(0x700000), 1, 1, 64, 64, 64, 1.0, None) == E.RWKV6_ERR_INVALID_ARG
    # GroupNorm backward: a gate gradient without a gate input
    assert L.rwkv6_gn_gate_bwd(a, 1, None, b, b, 0, p_ := _fake(0x500000), p_, c, d, _fake(0x600000),
                               _fake(0x700000), _fake(0x800000), _fake(0x900000), 4, 2, 2, 64,
                               None) == E.RWKV6_ERR_INVALID_ARG


def test_python_checker_maps_codes(pkg):
    with pytest.raises(NotImplementedError):
        pkg._lib.check(2, "x")
    with pytest.raises(ValueError):
        pkg._lib.check(1, "x")
    with pytest.raises(pkg._lib.Rwkv6Error):
        pkg._lib.check(3, "x")
    pkg._lib.check(0, "x")


def test_wrapper_rejects_cpu_tensors(pkg):
    import torch
    x = torch.zeros(1, 1, 4, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        pkg.chunk_rwkv6(x, x, x, x, torch.zeros(1, 64))
    with pytest.raises(NotImplementedError):
        pkg.chunk_rwkv6(x, x, x, x, torch.zeros(1, 64), cu_seqlens=torch.tensor([0, 4]))


@pytest.mark.parametrize("version,msg", [(2, "ABI version 2"), (None, "lacks")])
def test_stale_library_gets_the_rebuild_message(pkg, tmp_path, version, msg):
    """A stub library built here with gcc: an older ABI version, or the current version with
    symbols missing, must fail with the rebuild hint, not a ctypes AttributeError."""
    import shutil
    import subprocess

    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    v = pkg._lib.ABI_VERSION if version is None else version
    src = tmp_path / "stub.c"
    src.write_text(f"int rwkv6_abi_version(void) {{ return {v}; }}\n"
                   "const char* rwkv6_strerror(int c) { (void)c; return \"ok\"; }\n")
    so = tmp_path / "libstub.so"
    subprocess.run(["gcc", "-shared", "-fPIC", "-o", str(so), str(src)], check=True)
    with pytest.raises(RuntimeError, match="rebuild") as e:
        pkg._lib.bind(ctypes.CDLL(str(so)), str(so))
    assert msg in str(e.value)
