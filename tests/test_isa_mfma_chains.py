"""No MFMA of one shape accumulates onto the result of an MFMA of another shape.

On MI355X a v_mfma_f32_16x16x16_bf16 that takes as its accumulator (SrcC) the registers a
v_mfma_f32_16x16x32_bf16 has just written gave wrong sums now and then: with no instruction
between the two, the dv of the reverse-walk backward lost part of its inter-chunk term in
multi-chunk sequences, in a pattern that changed from run to run, while the compiler placed no
wait states there.  Every kernel therefore keeps the two shapes in separate accumulators (or
hands the 16x16x32 result through a VALU instruction first).  This test compiles each HIP
source to gfx950 assembly with the library's own flags and checks, in code order, that no
MFMA reads as SrcC registers last written by an MFMA of a different opcode.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "rwkv-megatron_amd", "csrc")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def _regs(tok):
    m = re.match(r"[va]\[(\d+):(\d+)\]$", tok)
    if m:
        return range(int(m.group(1)), int(m.group(2)) + 1)
    m = re.match(r"[va](\d+)$", tok)
    return range(int(m.group(1)), int(m.group(1)) + 1) if m else range(0)


def mixed_chains(asm: str):
    """(kernel, earlier opcode, MFMA line) for every MFMA whose SrcC registers were last
    written, in code order within the kernel, by an MFMA of another opcode."""
    out = []
    kernel, writer = None, {}
    for raw in asm.splitlines():
        line = raw.strip()
        m = re.match(r"^(_Z\w+):", line)
        if m:
            kernel, writer = m.group(1), {}
            continue
        if kernel is None or not line or line[0] in ";." or line.endswith(":"):
            continue
        parts = line.split(None, 1)
        op = parts[0]
        ops = [x.strip() for x in parts[1].split(",")] if len(parts) > 1 else []
        if not (op.startswith("v_") or op.startswith("ds_read") or op.startswith("global_load")
                or op.startswith("buffer_load")) or not ops:
            continue
        if op.startswith("v_mfma") and len(ops) > 3:
            for r in _regs(ops[3]):
                w = writer.get(r)
                if w is not None and w.startswith("v_mfma") and w != op:
                    out.append((kernel, w, line))
                    break
        for r in _regs(ops[0]):
            writer[r] = op
    return out


def test_scanner_flags_a_mixed_chain():
    asm = "\n".join([
        "_Z1kv:",
        "v_mfma_f32_16x16x32_bf16 v[18:21], v[94:97], v[90:93], 0",
        "v_mfma_f32_16x16x32_bf16 v[18:21], v[98:101], v[102:105], v[18:21]",
        "v_mfma_f32_16x16x16_bf16 v[18:21], v[106:107], v[108:109], v[18:21]",
        "_Z1jv:",
        "v_mfma_f32_16x16x32_bf16 v[18:21], v[94:97], v[90:93], 0",
        "v_mul_f32_e32 v18, v1, v18",
        "v_mfma_f32_16x16x16_bf16 v[18:21], v[106:107], v[108:109], v[18:21]",
        "v_mfma_f32_16x16x16_bf16 v[22:25], v[106:107], v[108:109], 0",
        "v_mfma_f32_16x16x16_bf16 v[22:25], v[106:107], v[108:109], v[22:25]",
    ])
    hits = mixed_chains(asm)
    assert [h[0] for h in hits] == ["_Z1kv", "_Z1jv"]   # jv: v[19:21] still come from the x32


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
@pytest.mark.parametrize("src", sorted(f for f in os.listdir(CSRC) if f.endswith(".hip")))
def test_no_mixed_shape_mfma_accumulation(src, tmp_path):
    asm = tmp_path / (src + ".s")
    cmd = [HIPCC, "-O3", "-std=c++17", "--offload-arch=gfx950", "--offload-device-only", "-S",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-Wno-unused-command-line-argument", os.path.join(CSRC, src), "-o", str(asm)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    hits = mixed_chains(asm.read_text())
    assert not hits, "\n".join(f"{k}: {w} -> {l}" for k, w, l in hits[:10])
