"""Build recipe for the native parts of quant_ops_amd (run on the CPU host).

Produces, in-tree next to this file:

* ``libquant_ops_hip.so`` — the gfx950 HIP kernels behind the C ABI declared in
  ``include/quant_ops_hip.h`` (no torch dependency);
* ``_quant_ops_torch.so`` — the torch operator registration (``quant_ops::*``)
  that calls that C ABI, linked against it with an ``$ORIGIN`` rpath;
* ``libquant_ops_probes.so`` — microbenchmarks of the hardware ceilings
  (``bench.py --ceilings``), kept out of the product library.

``hipcc`` cross-compiles for gfx950 without a GPU. Every HIP file is built
with packed fp32 instructions disabled.

Usage: ``python -m quant_ops_amd._build`` (or ``build()`` from ``__graft_entry__``).
"""
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
OBJ = os.path.join(HERE, "_obj")

HIP_SOURCES = ["capi.hip", "flatquant_quant.hip", "int4_gemm.hip", "int4_gemm_f6.hip", "dequant.hip", "layout.hip", "w4a4_linear.hip"]
LIB_NAME = "libquant_ops_hip.so"
TORCH_LIB_NAME = "_quant_ops_torch.so"
# microbenchmarks of the hardware ceilings (bench.py --ceilings), a library of its own
PROBE_SOURCE = "probes.hip"
PROBE_LIB_NAME = "libquant_ops_probes.so"

ARCH = os.environ.get("QUANT_OPS_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # no implicit contraction: the reference rounds every float32 product before
    # rounding to half, and a fused mul-convert (v_fma_mixlo_f16) rounds once
    "-ffp-contract=off",
    # packed fp32 VALU forms are kept out of every kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}",
]
# Per-file additions. The quantize kernels keep MFMA results in VGPRs (the AGPR
# form costs a v_accvgpr_read per result element their epilogues consume); the
# GEMM lets the compiler place its accumulators, which measured faster. The
# quantize kernels also take their first 16 argument dwords preloaded into
# SGPRs (no scalar load before the first DMA issue: 1-2% on launches of a few
# microseconds); the GEMM measured no gain from it.
FILE_FLAGS = {
    "flatquant_quant.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1",
                            "-mllvm", "-amdgpu-kernarg-preload-count=16"],
}


def _run(cmd):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines()
        if "packed-fp32-ops" not in line and "is not a recognized feature" not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    return out


def _compile_hip(src):
    obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    _run([HIPCC, *HIP_FLAGS, *FILE_FLAGS.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj])
    return obj


def build_hip_library(verbose=True):
    os.makedirs(OBJ, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(8, len(HIP_SOURCES))) as ex:
        objs = list(ex.map(_compile_hip, HIP_SOURCES))
    out = os.path.join(HERE, LIB_NAME)
    tmp = out + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp])
    os.replace(tmp, out)
    if verbose:
        print(f"[quant_ops_amd] built {out}")
    return out


def build_torch_binding(verbose=True):
    import torch
    from torch.utils import cpp_extension

    torch_dir = os.path.dirname(torch.__file__)
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    incs = [f"-I{p}" for p in cpp_extension.include_paths()] + [f"-I{INCLUDE}", "-I/opt/rocm/include"]
    libdir = os.path.join(torch_dir, "lib")
    out = os.path.join(HERE, TORCH_LIB_NAME)
    tmp = out + ".tmp"
    cmd = [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        *incs, os.path.join(CSRC, "torch_ops.cpp"),
        f"-L{libdir}", "-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch_hip", "-ltorch",
        f"-L{HERE}", "-l:" + LIB_NAME,
        "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{libdir}",
        "-o", tmp,
    ]
    _run(cmd)
    os.replace(tmp, out)
    if verbose:
        print(f"[quant_ops_amd] built {out}")
    return out


def build_probe_library(verbose=True):
    os.makedirs(OBJ, exist_ok=True)
    out = os.path.join(HERE, PROBE_LIB_NAME)
    tmp = out + ".tmp"
    _run([HIPCC, *HIP_FLAGS, "-shared", os.path.join(CSRC, PROBE_SOURCE), "-o", tmp])
    os.replace(tmp, out)
    if verbose:
        print(f"[quant_ops_amd] built {out}")
    return out


def build(verbose=True):
    """Compile every native part (always recompiles)."""
    build_hip_library(verbose)
    build_torch_binding(verbose)
    build_probe_library(verbose)


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
