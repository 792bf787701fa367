"""W4A4 int4 GEMM — drop-in for the reference's
``quant_ops.ops.quantization.int4_matmul`` (``int4_matmul/ops.py:1-158``).

Packed layout (shared with the quantizer): word ``p`` of a row holds columns
``8p .. 8p+7``, column ``8p + i`` in bits ``4i .. 4i+3`` as the offset code
``q + 8``. A is int32 [M, K/8]; B is int32 [K/8, N] where word ``(p, n)`` holds
``k = 8p .. 8p+7`` of column ``n`` — either row-major or the transposed view
``W.t()`` of a [N, K/8] weight (both are read in place on the GPU).

GPU tensors use the HIP i8-MFMA kernel; if the HIP library is not loaded they
raise. Host tensors use ``int4_matmul_pytorch``, the reference fallback.
"""
from typing import Optional

import torch

from . import _loader


def _shifts(device):
    return torch.arange(0, 32, 4, dtype=torch.int32, device=device)


def pack_int4_to_int32(tensor: torch.Tensor) -> torch.Tensor:
    """int8 codes in [-8, 7] [rows, F] -> int32 [rows, F/8] (``int4_matmul/ops.py:23-45``)."""
    rows, feats = tensor.shape
    assert feats % 8 == 0, f"features ({feats}) must be divisible by 8"
    nib = (tensor + 8).to(torch.uint8).view(rows, feats // 8, 8).to(torch.int32)
    words = (nib << _shifts(tensor.device)).sum(dim=2, dtype=torch.int64)
    return torch.where(words >= 2**31, words - 2**32, words).to(torch.int32)


def unpack_int32_to_int4(packed: torch.Tensor) -> torch.Tensor:
    """int32 [rows, W] -> int8 codes [rows, 8W] (``int4_matmul/ops.py:48-66``)."""
    rows, words = packed.shape
    nib = (packed.unsqueeze(-1) >> _shifts(packed.device)) & 0xF
    return (nib - 8).to(torch.int8).reshape(rows, words * 8)


def int4_matmul_pytorch(
    a_packed: torch.Tensor,
    b_packed: torch.Tensor,
    scale_a: torch.Tensor,
    scale_b: torch.Tensor,
    out_dtype: Optional[torch.dtype] = None,
) -> torch.Tensor:
    """Reference fallback (``int4_matmul/ops.py:69-103``).

    float32 matmul of the unpacked codes (exact for |sum| < 2**24), then
    ``* scale_a[m]``, then ``* scale_b[n]`` (float32), then one rounding to
    ``out_dtype`` (float16 unless given; the reference always returns float16).
    """
    m, kp = a_packed.shape
    n = b_packed.shape[1]
    qa = unpack_int32_to_int4(a_packed.reshape(-1, kp)).view(m, kp * 8)
    qb = unpack_int32_to_int4(b_packed.T).T.reshape(kp * 8, n)
    acc = torch.matmul(qa.float(), qb.float())
    out = acc * scale_a.view(m, 1) * scale_b.view(1, n)
    return out.to(out_dtype or torch.float16)


def int4_matmul_cuda(
    a_packed: torch.Tensor,
    b_packed: torch.Tensor,
    scale_a: torch.Tensor,
    scale_b: torch.Tensor,
    out_dtype: Optional[torch.dtype] = None,
) -> torch.Tensor:
    """HIP kernel, moving host tensors to the current GPU first (``int4_matmul/ops.py:106-137``).

    Unlike the reference, non-contiguous operands are not copied: A may have any
    row stride and B may be row-major or ``W.t()``; other B layouts are copied
    by the operator.
    """
    _loader.require_kernels("int4_matmul_cuda")
    dev = a_packed.device if a_packed.is_cuda else torch.device("cuda", torch.cuda.current_device())
    a_packed, b_packed = a_packed.to(dev), b_packed.to(dev)
    scale_a, scale_b = scale_a.to(dev), scale_b.to(dev)
    if out_dtype is None or out_dtype == torch.float16:
        return torch.ops.quant_ops.int4_matmul(a_packed, b_packed, scale_a, scale_b)
    return torch.ops.quant_ops.int4_matmul_ex(a_packed, b_packed, scale_a, scale_b, out_dtype)


def int4_matmul(
    a_packed: torch.Tensor,
    b_packed: torch.Tensor,
    scale_a: torch.Tensor,
    scale_b: torch.Tensor,
    out_dtype: Optional[torch.dtype] = None,
) -> torch.Tensor:
    """Main entry (``int4_matmul/ops.py:140-157``); ``out_dtype`` is an addition (default float16)."""
    if a_packed.is_cuda:
        _loader.require_kernels("int4_matmul")
        if out_dtype is None or out_dtype == torch.float16:
            return torch.ops.quant_ops.int4_matmul(a_packed, b_packed, scale_a, scale_b)
        return torch.ops.quant_ops.int4_matmul_ex(a_packed, b_packed, scale_a, scale_b, out_dtype)
    return int4_matmul_pytorch(a_packed, b_packed, scale_a, scale_b, out_dtype)
