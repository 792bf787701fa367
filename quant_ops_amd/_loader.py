"""Loads the in-tree native libraries.

* ``_quant_ops_torch.so`` registers the ``quant_ops::*`` torch operators
  (``torch.ops.quant_ops``) on the GPU dispatch key; it pulls in
  ``libquant_ops_hip.so`` through its ``$ORIGIN`` rpath.

Mirrors the reference's loaders (``flatquant/kernels/__init__.py:7-34``,
``int4_matmul/kernels/__init__.py:5-44``) with two differences: the file name
does not encode the Python version, and a missing library does not make
``import`` fail — ``KERNELS_AVAILABLE`` is then False and every GPU entry point
raises instead of computing anything elsewhere. ``QUANT_OPS_DEBUG=1`` prints
what was loaded, as in the reference.
"""
import os

import torch

LIB_DIR = os.path.dirname(os.path.abspath(__file__))
HIP_LIB_PATH = os.path.join(LIB_DIR, "libquant_ops_hip.so")
TORCH_LIB_PATH = os.path.join(LIB_DIR, "_quant_ops_torch.so")

KERNELS_AVAILABLE = False
LOAD_ERROR = None


def _debug(msg):
    if os.environ.get("QUANT_OPS_DEBUG", "0") == "1":
        print(f"[quant_ops_amd] {msg}")


def _load():
    global KERNELS_AVAILABLE, LOAD_ERROR
    if not os.path.exists(TORCH_LIB_PATH):
        LOAD_ERROR = f"native library not built: {TORCH_LIB_PATH} (run python -m quant_ops_amd._build)"
        _debug(LOAD_ERROR)
        return
    try:
        torch.ops.load_library(TORCH_LIB_PATH)
    except Exception as exc:  # a broken build must not hide behind a fallback
        LOAD_ERROR = f"failed to load {TORCH_LIB_PATH}: {exc}"
        _debug(LOAD_ERROR)
        return
    KERNELS_AVAILABLE = True
    _debug(f"loaded {TORCH_LIB_PATH}; ops: {sorted(n for n in dir(torch.ops.quant_ops) if not n.startswith('_'))}")


def require_kernels(what: str):
    """Raise if the HIP library is not loaded (GPU tensors never fall back)."""
    if not KERNELS_AVAILABLE:
        raise RuntimeError(f"{what}: the quant_ops_amd HIP library is not available ({LOAD_ERROR})")


_load()
