"""W4A4 FlatQuant linear layer: the product-level consumer of the two kernels.

Mirrors the reference's vLLM linear method
(``w4a4_flatquant_dynamic.py:168-304``, ``AscendW4A4FlatQuantDynamicLinearMethod``):

* ``prepare_w4a4_weight`` is ``process_weights_after_loading``'s packing step
  (``:268-292``): int8 codes [out, in] (clamped to [-8, 7] as
  ``pack_int4_to_int32_manual``, ``:43-67``) -> int32 [out, in/8].
* ``w4a4_flatquant_linear`` is ``apply`` (``:168-266``): per-token dynamic
  quantization of x with the Kronecker transform, the int4 GEMM against the
  packed weight's ``.t()`` view with per-token x per-channel scales, output in
  x's dtype, then ``+ bias``. On the GPU this is one operator
  (``quant_ops::w4a4_linear``, C ABI ``qo_w4a4_linear``): the two kernels on
  the current stream, with the bias in the GEMM epilogue (same two
  roundings).

Differences, each deliberate:

* ``left_trans`` / ``right_trans`` mean what they mean in
  ``flatquant_dynamic_quantize`` (y = Lᵀ·X·R per token). The reference's
  ``process_weights_after_loading`` stores ``left_trans.t()`` because its NPU
  operator takes the other convention (``:296``); callers porting weights
  pass the untransposed matrix here.
* No 8192-token chunking: the reference splits calls because the NPU operator
  is limited to 8192 tokens (``:206-240``); the HIP kernels loop over any
  number of tokens, so one call gives the same result.
"""
from typing import Optional

import torch

from . import _loader
from .flatquant import flatquant_dynamic_quantize
from .int4_matmul import int4_matmul, pack_int4_to_int32


def _scale_dtype(s: torch.Tensor) -> torch.Tensor:
    """Weight scales as the operator takes them (float32 / float16 / bfloat16;
    anything else as float32, which the fallback's float32 product also uses)."""
    return s if s.dtype in (torch.float32, torch.float16, torch.bfloat16) else s.to(torch.float32)


def prepare_w4a4_weight(weight_codes: torch.Tensor) -> torch.Tensor:
    """int4 weight codes stored as integers [out, in] -> packed int32 [out, in/8]."""
    assert weight_codes.dim() == 2 and weight_codes.shape[1] % 8 == 0, "[out, in] with in % 8 == 0"
    return pack_int4_to_int32(weight_codes.clamp(-8, 7).to(torch.int8))


def w4a4_flatquant_linear(
    x: torch.Tensor,
    left_trans: torch.Tensor,
    right_trans: torch.Tensor,
    weight_packed: torch.Tensor,
    weight_scale: torch.Tensor,
    clip_ratio: float = 1.0,
    bias: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """y = dequant(Q(x)) · dequant(W)ᵀ (+ bias) in x.dtype.

    x [..., in] with in = M·N (M, N the transform sizes); weight_packed int32
    [out, in/8]; weight_scale [out] or [out, 1] (per output channel).
    """
    m, n = left_trans.shape[0], right_trans.shape[0]
    in_features = x.shape[-1]
    assert m * n == in_features, f"transform sizes M({m}) * N({n}) != in_features({in_features})"
    out_features = weight_packed.shape[0]
    assert weight_packed.shape[1] * 8 == in_features, "weight_packed must be [out, in/8]"
    dtype = x.dtype
    x2 = x.reshape(-1, in_features)
    if x2.is_cuda:
        # one operator: quantize + GEMM (bias in the GEMM epilogue, with the same
        # two roundings)
        _loader.require_kernels("w4a4_flatquant_linear")
        out = torch.ops.quant_ops.w4a4_linear(x2, left_trans.to(dtype), right_trans.to(dtype), weight_packed,
                                              _scale_dtype(weight_scale.reshape(-1)), float(clip_ratio), bias)
        return out.view(*x.shape[:-1], out_features)
    codes, act_scale = flatquant_dynamic_quantize(
        x2, left_trans.to(dtype), right_trans.to(dtype), clip_ratio, pack_int32=True)
    sa, sb = act_scale.to(torch.float32), weight_scale.reshape(-1).to(torch.float32)
    out = int4_matmul(codes, weight_packed.t(), sa, sb, out_dtype=dtype)
    if bias is not None:
        out = out + bias.to(dtype)
    return out.view(*x.shape[:-1], out_features)
