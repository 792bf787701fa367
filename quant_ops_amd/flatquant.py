"""FlatQuant dynamic int4 quantization — drop-in for the reference's
``quant_ops.ops.quantization.flatquant`` (``flatquant/ops.py:1-178``).

GPU tensors go to the fused HIP kernel through ``torch.ops.quant_ops``. If the
HIP library is not loaded, GPU calls raise (they are never computed by the
PyTorch fallback behind the caller's back). CPU tensors, or ``use_cuda=False``,
run ``flatquant_pytorch``, the reference's PyTorch fallback, which is part of
the public API (``examples/basic_usage.py:13`` imports it).

Returned scales: the GPU op returns float32 [T] (the reference's op schema and
fake kernel, ``meta_ops.py:36``) holding exactly the value the fallback computes
in the input dtype; the fallback returns the input dtype, as the reference's does.
"""
from typing import Tuple

import torch
from torch.autograd import Function

from . import _loader


class _FlatQuantCUDA(Function):
    """Autograd wrapper around the operator; inference only (backward returns None).

    Reference: ``flatquant/ops.py:25-41``.
    """

    @staticmethod
    def forward(ctx, input_tensor, left_trans, right_trans, clip_ratio, pack_int32):
        return torch.ops.quant_ops.flatquant_dynamic_quantize(
            input_tensor, left_trans, right_trans, float(clip_ratio), bool(pack_int32)
        )

    @staticmethod
    def backward(ctx, grad_output, grad_scales):
        return None, None, None, None, None


try:  # let torch.compile keep the call as one node (flatquant/ops.py:43-51)
    torch.compiler.allow_in_graph(_FlatQuantCUDA.apply)
except Exception:  # pragma: no cover - older torch
    pass


def flatquant_cuda(
    input_tensor: torch.Tensor,
    left_trans: torch.Tensor,
    right_trans: torch.Tensor,
    clip_ratio: float = 1.0,
    pack_int32: bool = False,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Run the HIP kernel, moving host tensors to the current GPU first.

    Reference: ``flatquant/ops.py:54-75``.
    """
    _loader.require_kernels("flatquant_cuda")
    input_tensor = input_tensor.cuda()
    left_trans = left_trans.to(input_tensor.device)
    right_trans = right_trans.to(input_tensor.device)
    return _FlatQuantCUDA.apply(input_tensor, left_trans, right_trans, clip_ratio, pack_int32)


def flatquant_pytorch(
    input_tensor: torch.Tensor,
    left_trans: torch.Tensor,
    right_trans: torch.Tensor,
    clip_ratio: float = 1.0,
    pack_int32: bool = False,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """The PyTorch fallback (``flatquant/ops.py:78-130``), on any device.

    Per token, X = row viewed as [M, N]: ``Y = L^T (X R)`` with results in the
    input dtype after each product; scale = max(|min Y * c|, max Y * c) / 7
    (floored at 1e-8, in the input dtype); codes = clamp(round(Y / scale), -8, 7)
    as int8, or eight 4-bit offset codes (q + 8) per int32 word.
    """
    tokens, feats = input_tensor.shape
    m, n = left_trans.shape[0], right_trans.shape[0]
    y = torch.matmul(left_trans.T, torch.matmul(input_tensor.reshape(-1, m, n), right_trans))
    y = y.reshape(tokens, feats)
    top = y.amax(1, keepdim=True)
    bottom = y.amin(1, keepdim=True)
    scale = (torch.maximum((bottom * clip_ratio).abs(), top * clip_ratio) / 7.0).clamp(min=1e-8).squeeze(1)
    q = torch.round(y / scale.view(-1, 1).expand_as(y)).clamp(-8, 7)
    if not pack_int32:
        return q.to(torch.int8), scale
    nib = (q + 8).to(torch.uint8).view(tokens, feats // 8, 8).to(torch.int32)
    shifts = torch.arange(0, 32, 4, dtype=torch.int32, device=input_tensor.device)
    words = (nib << shifts).sum(dim=2, dtype=torch.int64)
    words = torch.where(words >= 2**31, words - 2**32, words).to(torch.int32)
    return words, scale


def flatquant_dynamic_quantize(
    input_tensor: torch.Tensor,
    left_trans: torch.Tensor,
    right_trans: torch.Tensor,
    clip_ratio: float = 1.0,
    pack_int32: bool = False,
    use_cuda: bool = True,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Main entry (``flatquant/ops.py:133-153``).

    ``use_cuda`` is accepted because the reference's tests and README pass it
    (``tests/test_accuracy.py:46,58``, ``README.md:78``): False selects the
    PyTorch fallback. GPU tensors otherwise always use the HIP kernel.
    """
    if not use_cuda or not input_tensor.is_cuda:
        return flatquant_pytorch(input_tensor, left_trans, right_trans, clip_ratio, pack_int32)
    _loader.require_kernels("flatquant_dynamic_quantize")
    return torch.ops.quant_ops.flatquant_dynamic_quantize(
        input_tensor, left_trans, right_trans, float(clip_ratio), bool(pack_int32)
    )


def dequantize_int4(quantized: torch.Tensor, scales: torch.Tensor, packed_int32: bool = False) -> torch.Tensor:
    """float32 ``q * scale[token]`` (``flatquant/ops.py:156-178``).

    GPU tensors use the HIP kernel; host tensors use torch element-wise ops.
    """
    if quantized.is_cuda:
        _loader.require_kernels("dequantize_int4")
        return torch.ops.quant_ops.dequantize_int4(quantized, scales, bool(packed_int32))
    if packed_int32:
        rows, words = quantized.shape
        shifts = torch.arange(0, 32, 4, dtype=torch.int32, device=quantized.device)
        nib = (quantized.unsqueeze(-1) >> shifts) & 0xF
        quantized = (nib - 8).to(torch.int8).reshape(rows, words * 8)
    return quantized.float() * scales.view(-1, 1).expand_as(quantized)
