"""Equivalents of the reference's two pybind extension modules.

The reference exposes one function per compiled extension besides its torch
operators:

* ``cuda_quant_ops.cuda_kronecker_quant_int8`` (``cuda_quant_kernel.cu:316-390``,
  bound at ``:419-421``), loaded by ``flatquant/kernels/__init__.py``;
* ``cuda_int4_matmul_ops.cuda_int4_matmul`` (``cuda_int4_matmul_kernel.cu:130-189``,
  bound at ``:222-224``), loaded by ``int4_matmul/kernels/__init__.py``.

Here both run the HIP operators (``torch.ops.quant_ops``) with the argument
handling of the reference's host functions, and ``torch.compiler.allow_in_graph``
is applied to them as ``flatquant/ops.py:11-22`` and ``int4_matmul/ops.py:11-20``
do. When the HIP library is not loaded the module objects are ``None`` and the
flags False; unlike the reference's flatquant loader, that does not make
``import`` fail.
"""
import types

import torch

from . import _loader


def cuda_kronecker_quant_int8(input, left_trans, right_trans, clip_ratio, pack_int32=False):
    """Fused Kronecker transform + int4 quantization of GPU tensors.

    Moves the inputs to the GPU and makes them contiguous as the reference's
    host function does (``cuda_quant_kernel.cu:331-334``); returns
    ``(codes, scales)`` with float32 scales. Unlike the reference it does not
    synchronise the stream.
    """
    _loader.require_kernels("cuda_kronecker_quant_int8")
    input = input.contiguous().cuda()
    left_trans = left_trans.contiguous().to(input.device)
    right_trans = right_trans.contiguous().to(input.device)
    return torch.ops.quant_ops.flatquant_dynamic_quantize(input, left_trans, right_trans, float(clip_ratio),
                                                         bool(pack_int32))


def cuda_int4_matmul(a_packed, b_packed, scale_a, scale_b):
    """int4 x int4 GEMM of GPU tensors with float32 scales, fp16 output.

    The argument checks and their messages are those of the reference's host
    function (``cuda_int4_matmul_kernel.cu:136-150``); the shape checks are the
    operator's.
    """
    _loader.require_kernels("cuda_int4_matmul")
    for name, t in (("a_packed", a_packed), ("b_packed", b_packed), ("scale_a", scale_a), ("scale_b", scale_b)):
        if not t.is_cuda:
            raise RuntimeError(f"{name} must be on CUDA")
    if a_packed.dtype != torch.int32:
        raise RuntimeError("a_packed must be int32")
    if b_packed.dtype != torch.int32:
        raise RuntimeError("b_packed must be int32")
    if scale_a.dtype != torch.float32:
        raise RuntimeError("scale_a must be float32")
    if scale_b.dtype != torch.float32:
        raise RuntimeError("scale_b must be float32")
    return torch.ops.quant_ops.int4_matmul(a_packed, b_packed, scale_a, scale_b)


def _module(name, **fns):
    mod = types.ModuleType(name)
    for key, fn in fns.items():
        setattr(mod, key, fn)
    return mod


CUDA_KERNELS_AVAILABLE = _loader.KERNELS_AVAILABLE
if CUDA_KERNELS_AVAILABLE:
    cuda_quant_ops = _module("cuda_quant_ops", cuda_kronecker_quant_int8=cuda_kronecker_quant_int8)
    cuda_int4_matmul_ops = _module("cuda_int4_matmul_ops", cuda_int4_matmul=cuda_int4_matmul)
else:
    cuda_quant_ops = None
    cuda_int4_matmul_ops = None

try:  # one graph node each under torch.compile (flatquant/ops.py:11-22, int4_matmul/ops.py:11-20)
    torch.compiler.allow_in_graph(cuda_kronecker_quant_int8)
    torch.compiler.allow_in_graph(cuda_int4_matmul)
except Exception:  # pragma: no cover - older torch
    pass
