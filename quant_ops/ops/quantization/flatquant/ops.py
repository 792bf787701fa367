"""FlatQuant operator entry points (reference ``flatquant/ops.py:1-178``), defined in
``quant_ops_amd.flatquant``."""
from quant_ops_amd.flatquant import (  # noqa: F401
    _FlatQuantCUDA,
    dequantize_int4,
    flatquant_cuda,
    flatquant_dynamic_quantize,
    flatquant_pytorch,
)
from .kernels import CUDA_KERNELS_AVAILABLE, cuda_quant_ops  # noqa: F401
