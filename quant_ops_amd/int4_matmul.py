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
    """int8 codes in [-8, 7] [rows, F] -> int32 [rows, F/8] (``int4_matmul/ops.py:23-45``).

    GPU int8 tensors use the HIP kernel ``qo_pack_int4_to_int32``; other inputs
    run the reference's torch formula.
    """
    rows, feats = tensor.shape
    assert feats % 8 == 0, f"features ({feats}) must be divisible by 8"
    if tensor.is_cuda and tensor.dtype == torch.int8:
        _loader.require_kernels("pack_int4_to_int32")
        from . import capi
        return capi.pack_int4_to_int32(tensor if tensor.stride(1) == 1 else tensor.contiguous())
    nib = (tensor + 8).to(torch.uint8).view(rows, feats // 8, 8).to(torch.int32)
    words = (nib << _shifts(tensor.device)).sum(dim=2, dtype=torch.int64)
    return torch.where(words >= 2**31, words - 2**32, words).to(torch.int32)


def unpack_int32_to_int4(packed: torch.Tensor) -> torch.Tensor:
    """int32 [rows, W] -> int8 codes [rows, 8W] (``int4_matmul/ops.py:48-66``).

    GPU int32 tensors use the HIP kernel ``qo_unpack_int32_to_int4``.
    """
    if packed.is_cuda and packed.dtype == torch.int32:
        _loader.require_kernels("unpack_int32_to_int4")
        from . import capi
        return capi.unpack_int32_to_int4(packed if packed.stride(1) == 1 else packed.contiguous())
    rows, words = packed.shape
    nib = (packed.unsqueeze(-1) >> _shifts(packed.device)) & 0xF
    return (nib - 8).to(torch.int8).reshape(rows, words * 8)


def transpose_packed(packed: torch.Tensor) -> torch.Tensor:
    """Contiguous transpose of a packed int32 matrix: converts a weight between
    the GEMM's B layouts [K/8, N] and [N, K/8], which hold the same words.

    The reference spells this ``.t().contiguous()`` / ``pack(b.T).T``
    (``examples/int4_matmul_benchmark.py:21-22``,
    ``w4a4_flatquant_dynamic.py:290-292``). GPU tensors use the HIP kernel
    ``qo_transpose_int32``.
    """
    assert packed.dtype == torch.int32 and packed.dim() == 2, "int32 [rows, cols] expected"
    if packed.is_cuda:
        _loader.require_kernels("transpose_packed")
        from . import capi
        return capi.transpose_int32(packed if packed.stride(1) == 1 else packed.contiguous())
    return packed.t().contiguous()


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
