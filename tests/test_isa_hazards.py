"""Static check of the built gfx950 code object (CPU only).

The kernels issue their global-to-LDS copies (``global_load_lds_dwordx4``) as
inline assembly, with a wave-uniform 64-bit base in SGPRs. A VALU instruction
that writes an SGPR (for example ``v_readlane_b32`` restoring an SGPR the
register allocator spilled to a VGPR lane) needs five wait states before a
VMEM instruction reads that SGPR; the hardware does not interlock it, and the
compiler inserts the wait states for the instructions it generates but not for
inline assembly. A copy that read a stale base would address the wrong memory.

This test disassembles every gfx950 code object in ``libquant_ops_hip.so``
(one offload bundle per source file, concatenated in the ``.hip_fatbin``
section) and fails if any LDS-DMA instruction reads an SGPR that a VALU
instruction wrote fewer than five wait states before it.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "quant_ops_amd", "libquant_ops_hip.so")
LLVM = "/opt/rocm/llvm/bin"
TOOLS = ("llvm-objcopy", "clang-offload-bundler", "llvm-objdump")


def _sgprs(text):
    out = set()
    for m in re.finditer(r"s\[(\d+):(\d+)\]|\bs(\d+)\b", text):
        if m.group(3):
            out.add(int(m.group(3)))
        else:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    return out


def scan_lds_dma_hazards(lines):
    """Instructions (strings, one per line, comments stripped) -> list of
    (valu, dma) pairs where a VALU write of an SGPR the DMA reads precedes it
    by fewer than five wait states."""
    found = []
    for i, line in enumerate(lines):
        if not line.startswith("global_load_lds"):
            continue
        ops = line.split(None, 1)[1] if " " in line else ""
        read = _sgprs(ops.split(",", 1)[1]) if "," in ops else set()
        waits = 0
        for j in range(i - 1, max(-1, i - 8), -1):
            prev = lines[j]
            if prev.startswith("s_nop"):
                waits += int(prev.split()[1], 0) + 1
            else:
                if prev.startswith("v_") and " " in prev:
                    dst = prev.split(None, 1)[1].split(",")[0]
                    if _sgprs(dst) & read and waits < 5:
                        found.append((prev, line))
                waits += 1
            if waits >= 5:
                break
    return found


def test_scanner_finds_the_pattern():
    # a restored base immediately before the copy is a hazard; with an s_nop 4
    # between them (five wait states) it is not
    bad = ["v_readlane_b32 s0, v253, 62", "v_readlane_b32 s1, v253, 63",
           "global_load_lds_dwordx4 v156, s[0:1]"]
    assert len(scan_lds_dma_hazards(bad)) == 2
    ok = bad[:2] + ["s_nop 4", bad[2]]
    assert scan_lds_dma_hazards(ok) == []
    far = ["v_readlane_b32 s0, v253, 62", "s_mov_b32 m0, s3", "s_add_u32 s4, s4, 1", "s_nop 2",
           "global_load_lds_dwordx4 v156, s[0:1]"]
    assert scan_lds_dma_hazards(far) == []


BUNDLE_MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def gfx950_disassembly(lib, tmp_path):
    """Disassembly text of every gfx950 code object in ``lib``'s .hip_fatbin
    section (the section holds one offload bundle per source file)."""
    fatbin = tmp_path / "fatbin.bin"
    subprocess.run([os.path.join(LLVM, "llvm-objcopy"), f"--dump-section=.hip_fatbin={fatbin}", lib,
                    str(tmp_path / "lib.copy")], check=True)
    data = fatbin.read_bytes()
    starts = []
    i = data.find(BUNDLE_MAGIC)
    while i >= 0:
        starts.append(i)
        i = data.find(BUNDLE_MAGIC, i + 1)
    texts = []
    for k, (lo, hi) in enumerate(zip(starts, starts[1:] + [len(data)])):
        part, co = tmp_path / f"bundle{k}.bin", tmp_path / f"bundle{k}.co"
        part.write_bytes(data[lo:hi])
        subprocess.run([os.path.join(LLVM, "clang-offload-bundler"), "--unbundle", "--type=o", f"--input={part}",
                        "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--output={co}"], check=True)
        texts.append(subprocess.run([os.path.join(LLVM, "llvm-objdump"), "-d", "--mcpu=gfx950", str(co)],
                                    check=True, stdout=subprocess.PIPE, text=True).stdout)
    return texts


def _instructions(dis):
    lines = []
    for raw in dis.splitlines():
        ins = raw.split("//")[0].strip()
        if ins and not ins.startswith(";") and not ins.endswith(":"):
            lines.append(ins)
    return lines


@pytest.mark.skipif(not os.path.exists(LIB), reason="library not built")
@pytest.mark.skipif(not all(os.path.exists(os.path.join(LLVM, t)) for t in TOOLS), reason="ROCm LLVM tools absent")
def test_no_valu_sgpr_hazard_before_lds_dma(tmp_path):
    texts = gfx950_disassembly(LIB, tmp_path)
    assert len(texts) >= 2
    # the quantize and both GEMM sources copy through LDS-DMA
    with_dma = [t for t in texts if "global_load_lds" in t]
    for kernel in ("fq_few2_kernel", "gemm_i4_pp2", "gemm_f6_pp2"):
        assert any(kernel in t for t in with_dma), kernel
    for dis in with_dma:
        lines = _instructions(dis)
        n_dma = sum(1 for x in lines if x.startswith("global_load_lds"))
        found = scan_lds_dma_hazards(lines)
        assert not found, f"{len(found)} of {n_dma} LDS-DMA instructions read a VALU-written SGPR: {found[:3]}"
