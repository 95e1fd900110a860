"""ctypes binding of librwkv6_amd.so (C ABI declared in include/rwkv6_amd.h).

The library is the only compute path: if it is missing this module raises, it
never falls back to another implementation.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "librwkv6_amd.so")

RWKV6_OK = 0
RWKV6_ERR_INVALID_ARG = 1
RWKV6_ERR_UNSUPPORTED = 2
RWKV6_ERR_LAUNCH = 3
RWKV6_ERR_ALIGNMENT = 4
RWKV6_F32 = 0
RWKV6_BF16 = 1
ABI_VERSION = 3                # RWKV6_ABI_VERSION of the header these signatures mirror

_vp = ctypes.c_void_p
_fp = ctypes.c_void_p          # float* passed as an address
_i64 = ctypes.c_int64
_int = ctypes.c_int
_f32 = ctypes.c_float

# name -> (restype, argtypes); mirrors include/rwkv6_amd.h
SIGNATURES = {
    "rwkv6_abi_version": (_int, []),
    "rwkv6_strerror": (ctypes.c_char_p, [_int]),
    "rwkv6_wkv_saved_bytes": (ctypes.c_size_t, [_i64] * 5),
    "rwkv6_wkv_workspace_bytes": (ctypes.c_size_t, [_i64] * 5 + [_int]),
    "rwkv6_wkv_fwd": (_int, [_vp] * 5 + [_int] + [_fp, _vp, _fp, _vp, _vp] + [_i64] * 5 + [_f32, _vp]),
    "rwkv6_wkv_bwd": (_int, [_vp] * 5 + [_int] + [_vp, _fp, _vp] + [_vp] * 5 + [_fp, _vp]
                      + [_i64] * 5 + [_f32, _vp]),
    "rwkv6_wkv_fwd_ex": (_int, [_vp] * 5 + [_int] + [_fp, _vp, _fp, _vp, _vp] + [_i64] * 5
                         + [_f32, _vp, _vp]),
    "rwkv6_wkv_bwd_ex": (_int, [_vp] * 5 + [_int] + [_vp, _fp, _vp] + [_vp] * 5 + [_fp, _vp]
                         + [_i64] * 5 + [_f32, _vp, _vp]),
    "rwkv6_wkv_fwd_noalloc": (_int, [_vp] * 5 + [_int] + [_fp, _vp, _fp, _vp] + [_i64] * 5
                              + [_f32, _vp]),
    "rwkv6_wkv_fwd_seqfirst": (_int, [_vp] * 5 + [_int] + [_fp, _vp, _fp, _vp, _vp] + [_i64] * 5
                               + [_f32, _vp]),
    "rwkv6_wkv_bwd_seqfirst": (_int, [_vp] * 5 + [_int] + [_vp, _fp, _vp] + [_vp] * 5 + [_fp, _vp]
                               + [_i64] * 5 + [_f32, _vp]),
    "rwkv6_shift_lerp_fwd": (_int, [_vp, _vp, _int, _vp] + [_i64] * 3 + [_vp]),
    "rwkv6_ddlerp_lora_fwd": (_int, [_vp] * 4 + [_int, _vp] + [_i64] * 4 + [_vp]),
    "rwkv6_lora_bias_fwd": (_int, [_vp] * 3 + [_int, _vp] + [_i64] * 4 + [_vp]),
    "rwkv6_ddlerp_lora_bwd_workspace_bytes": (ctypes.c_size_t, [_i64] * 3),
    "rwkv6_lora_tanh_bwd": (_int, [_vp, _i64, _i64, _vp, _vp] + [_i64] * 3 + [_vp]),
    "rwkv6_col_sum_workspace_bytes": (ctypes.c_size_t, [_i64] * 2),
    "rwkv6_col_sum": (_int, [_vp, _i64, _i64, _int, _vp, _vp, _vp]),
    "rwkv6_ddlerp_lora_bwd": (_int, [_vp] * 4 + [_int] + [_vp] * 6 + [_i64] * 4 + [_vp]),
    "rwkv6_shift_lerp_bwd_workspace_bytes": (ctypes.c_size_t, [_i64] * 3),
    "rwkv6_shift_lerp_bwd": (_int, [_vp, _vp, _int] + [_vp] * 6 + [_i64] * 3 + [_vp]),
    "rwkv6_cmix_lerp_fwd": (_int, [_vp, _vp, _int, _vp] + [_i64] * 3 + [_vp]),
    "rwkv6_cmix_lerp_bwd_workspace_bytes": (ctypes.c_size_t, [_i64] * 3),
    "rwkv6_cmix_lerp_bwd": (_int, [_vp, _vp, _int] + [_vp] * 4 + [_i64] * 3 + [_vp]),
    "rwkv6_relu_sq_fwd": (_int, [_vp, _vp, _i64, _vp]),
    "rwkv6_relu_sq_bwd": (_int, [_vp, _vp, _vp, _i64, _vp]),
    "rwkv6_sigmoid_gate_fwd": (_int, [_vp, _vp, _vp, _i64, _vp]),
    "rwkv6_sigmoid_gate_bwd": (_int, [_vp] * 5 + [_i64, _vp]),
    "rwkv6_sum_partials": (_int, [_fp, _i64, _i64, _int, _vp, _vp]),
    "rwkv6_gn_gate_fwd": (_int, [_vp, _int, _vp, _vp, _vp, _int, _f32, _vp, _fp, _fp] + [_i64] * 4 + [_vp]),
    "rwkv6_gn_gate_bwd_workspace_bytes": (ctypes.c_size_t, [_i64] * 4),
    "rwkv6_gn_gate_bwd": (_int, [_vp, _int, _vp, _vp, _vp, _int, _fp, _fp] + [_vp] * 5 + [_vp]
                          + [_i64] * 4 + [_vp]),
}

_lib = None


class Rwkv6Error(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    """Load the HIP library once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} not found: build it with `python rwkv-megatron_amd/build.py` "
                "(or __graft_entry__.build()); there is no fallback implementation")
        _lib = bind(ctypes.CDLL(LIB_PATH), LIB_PATH)
    return _lib


def bind(L: ctypes.CDLL, path: str) -> ctypes.CDLL:
    """Checks the library's ABI version first (a stale build lacks newer symbols, and
    binding them would fail with a bare AttributeError), then sets every signature."""
    ver = getattr(L, "rwkv6_abi_version", None)
    if ver is None:
        raise RuntimeError(f"{path} exports no rwkv6_abi_version: not this library, or a "
                           "broken build; rebuild it with `python rwkv-megatron_amd/build.py`")
    ver.restype, ver.argtypes = SIGNATURES["rwkv6_abi_version"]
    if ver() != ABI_VERSION:
        raise RuntimeError(
            f"{path} has ABI version {ver()}, these bindings expect {ABI_VERSION}: "
            "rebuild it with `python rwkv-megatron_amd/build.py`")
    missing = [n for n in SIGNATURES if not hasattr(L, n)]
    if missing:
        raise RuntimeError(f"{path} (ABI version {ABI_VERSION}) lacks {missing}: rebuild it "
                           "with `python rwkv-megatron_amd/build.py`")
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    return L


def check(status: int, what: str) -> None:
    if status == RWKV6_OK:
        return
    msg = load().rwkv6_strerror(status).decode()
    if status == RWKV6_ERR_UNSUPPORTED:
        raise NotImplementedError(f"{what}: {msg}")
    if status in (RWKV6_ERR_INVALID_ARG, RWKV6_ERR_ALIGNMENT):
        raise ValueError(f"{what}: {msg}")
    raise Rwkv6Error(f"{what}: {msg} (status {status})")
