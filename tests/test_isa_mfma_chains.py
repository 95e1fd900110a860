"""No MFMA of one shape accumulates onto the result of an MFMA of another shape.

On MI355X a v_mfma_f32_16x16x16_bf16 that takes as its accumulator (SrcC) the registers a
v_mfma_f32_16x16x32_bf16 has just written gave wrong sums now and then: with no instruction
between the two, the dv of the reverse-walk backward lost part of its inter-chunk term in
multi-chunk sequences, in a pattern that changed from run to run, while the compiler placed no
wait states there.  Every kernel therefore keeps the two shapes in separate accumulators (or
hands the 16x16x32 result through a VALU instruction first).  This test compiles each HIP
source to gfx950 assembly with the library's own flags and checks that no MFMA reads as SrcC
registers last written by an MFMA of a different opcode: in code order, and across every loop
back-edge (a branch to an earlier label), whose loop body is scanned once more with the
writers the first pass left, so an MFMA at the top of a loop that accumulates onto what an
MFMA at its bottom wrote is caught too.
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


def _parse(line):
    parts = line.split(None, 1)
    op = parts[0]
    ops = [x.strip() for x in parts[1].split(",")] if len(parts) > 1 else []
    return op, ops


def _scan(lines, labels, writer, kernel, out, depth):
    """Scans lines in order, updating writer (register -> set of opcodes that may have last
    written it).  At a back-edge to an earlier label the loop body is scanned once more from
    the current writers (nested loops up to two levels), and the writers of both paths merge."""
    for pos, line in enumerate(lines):
        op, ops = _parse(line)
        if op.startswith("s_branch") or op.startswith("s_cbranch"):
            tgt = ops[0] if ops else None
            a = labels.get(tgt)
            if a is not None and a <= pos and depth < 2:
                again = {r: set(w) for r, w in writer.items()}
                _scan(lines[a:pos + 1], {k: v - a for k, v in labels.items() if a <= v <= pos},
                      again, kernel, out, depth + 1)
                for r, w in again.items():
                    writer.setdefault(r, set()).update(w)
            continue
        if not (op.startswith("v_") or op.startswith("ds_read") or op.startswith("global_load")
                or op.startswith("buffer_load")) or not ops:
            continue
        if op.startswith("v_mfma") and len(ops) > 3:
            hit = next((w for r in _regs(ops[3]) for w in sorted(writer.get(r, ()))
                        if w.startswith("v_mfma") and w != op), None)
            if hit is not None and (kernel, hit, line) not in out:
                out.append((kernel, hit, line))
        for r in _regs(ops[0]):
            writer[r] = {op}


def mixed_chains(asm: str):
    """(kernel, earlier opcode, MFMA line) for every MFMA whose SrcC registers may have been
    last written by an MFMA of another opcode, in code order or around a loop."""
    out = []
    kernels, cur = [], None
    for raw in asm.splitlines():
        line = raw.split(";")[0].strip()
        m = re.match(r"^(_Z\w+):", line)
        if m:
            cur = (m.group(1), [])
            kernels.append(cur)
            continue
        if cur is None or not line or (line[0] == "." and not line.endswith(":")):
            continue
        cur[1].append(line)
    for kernel, body in kernels:
        lines, labels = [], {}
        for line in body:
            if line.endswith(":"):
                labels[line[:-1]] = len(lines)
            elif line:
                lines.append(line)
        _scan(lines, labels, {}, kernel, out, 0)
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


def test_scanner_follows_a_loop_back_edge():
    asm = "\n".join([
        "_Z1lv:",
        "v_mov_b32_e32 v18, 0",
        ".LBB0_1:                                ; %loop",
        "v_mfma_f32_16x16x16_bf16 v[18:21], v[106:107], v[108:109], v[18:21]",
        "v_mul_f32_e32 v1, v2, v3",
        "v_mfma_f32_16x16x32_bf16 v[18:21], v[94:97], v[90:93], v[22:25]",
        "s_cbranch_scc1 .LBB0_1",
        "s_endpgm",
        "_Z1mv:",
        ".LBB1_1:",
        "v_mfma_f32_16x16x16_bf16 v[18:21], v[106:107], v[108:109], v[18:21]",
        "v_mfma_f32_16x16x32_bf16 v[18:21], v[94:97], v[90:93], v[22:25]",
        "v_mul_f32_e32 v18, v1, v18",
        "v_mul_f32_e32 v19, v1, v19",
        "v_mul_f32_e32 v20, v1, v20",
        "v_mul_f32_e32 v21, v1, v21",
        "s_cbranch_scc1 .LBB1_1",
    ])
    hits = mixed_chains(asm)
    # lv: the top MFMA reads what the bottom x32 wrote on the next trip; mv: a VALU op sits between
    assert [(h[0], h[1]) for h in hits] == [("_Z1lv", "v_mfma_f32_16x16x32_bf16")]


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
