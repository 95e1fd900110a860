"""Builds librwkv6_amd.so (all HIP sources in csrc/) for gfx950 with hipcc.

Usage: python rwkv-megatron_amd/build.py   (also called by __graft_entry__.build()).
The library lands next to this file so it travels with the source tree.
"""
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "librwkv6_amd.so")
ARCH = os.environ.get("RWKV6_OFFLOAD_ARCH", "gfx950")

# Packed-FP32 instructions are disabled for all device code; hipcc's host pass
# warns that it does not know the feature, which is harmless.
FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "-shared", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-command-line-argument",
]


def sources():
    return sorted(glob.glob(os.path.join(HERE, "csrc", "*.hip")))


def build(verbose: bool = False) -> str:
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    tmp = LIB + ".tmp"
    cmd = [hipcc, *FLAGS, *sources(), "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("hipcc failed building librwkv6_amd.so")
    if verbose:
        msgs = [l for l in (res.stdout + res.stderr).splitlines() if "packed-fp32-ops" not in l]
        if msgs:
            print("\n".join(msgs))
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
