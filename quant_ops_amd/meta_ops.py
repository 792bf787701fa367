"""Fake (meta) kernels so FakeTensor / torch.compile can trace the operators.

Shapes and dtypes follow the reference (``src/quant_ops/meta_ops.py:22-37``):
int4_matmul -> float16 [M, N]; flatquant_dynamic_quantize -> int32 [T, F/8] or
int8 [T, F] plus float32 scales [T]. The two operators this build adds get
fakes of their own. Registered only when the native library defined the
schemas.
"""
import torch

from . import _loader

if _loader.KERNELS_AVAILABLE:

    @torch.library.register_fake("quant_ops::int4_matmul")
    def _int4_matmul_fake(a, b, scale_a, scale_b):
        return a.new_empty((a.size(0), b.size(1)), dtype=torch.float16)

    @torch.library.register_fake("quant_ops::int4_matmul_ex")
    def _int4_matmul_ex_fake(a, b, scale_a, scale_b, out_dtype=None):
        return a.new_empty((a.size(0), b.size(1)), dtype=out_dtype or torch.float16)

    # defined by libraries built from this version on (a stale build lacks it)
    if hasattr(torch.ops.quant_ops, "int4_matmul_bias"):

        @torch.library.register_fake("quant_ops::int4_matmul_bias")
        def _int4_matmul_bias_fake(a, b, scale_a, scale_b, bias, out_dtype=None):
            return a.new_empty((a.size(0), b.size(1)), dtype=out_dtype or torch.float16)

    if hasattr(torch.ops.quant_ops, "w4a4_linear"):

        @torch.library.register_fake("quant_ops::w4a4_linear")
        def _w4a4_linear_fake(x, left_trans, right_trans, weight_packed, weight_scale, clip_ratio=1.0, bias=None):
            return x.new_empty((x.size(0), weight_packed.size(0)), dtype=x.dtype)

    @torch.library.register_fake("quant_ops::flatquant_dynamic_quantize")
    def _flatquant_fake(input_tensor, left_trans, right_trans, clip_ratio=1.0, pack_int32=False):
        tokens, feats = input_tensor.shape
        if pack_int32:
            codes = input_tensor.new_empty((tokens, feats // 8), dtype=torch.int32)
        else:
            codes = input_tensor.new_empty((tokens, feats), dtype=torch.int8)
        return codes, input_tensor.new_empty((tokens,), dtype=torch.float32)

    @torch.library.register_fake("quant_ops::dequantize_int4")
    def _dequant_fake(quantized, scales, packed_int32=False):
        feats = quantized.size(1) * (8 if packed_int32 else 1)
        return quantized.new_empty((quantized.size(0), feats), dtype=torch.float32)
