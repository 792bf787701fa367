"""quant_ops_amd — MI355X (gfx950) FlatQuant W4A4 hot path.

Drop-in for the public API of libarry/quant_ops (``src/quant_ops/__init__.py:16-45``):
``flatquant_dynamic_quantize``, ``dequantize_int4``, ``int4_matmul``,
``get_decompose_dim``, ``CUDA_AVAILABLE`` and ``__version__``, backed by
hand-written HIP kernels behind a C ABI (``include/quant_ops_hip.h``).

Import order matches the reference's (``__init__.py:20-37``): load the native
library (defines the ``quant_ops::*`` schemas), register the fake kernels, then
compute ``CUDA_AVAILABLE``.
"""

__version__ = "0.1.0"

from . import _loader
from .flatquant import (
    _FlatQuantCUDA,
    dequantize_int4,
    flatquant_cuda,
    flatquant_dynamic_quantize,
    flatquant_pytorch,
)
from .int4_matmul import (
    int4_matmul,
    int4_matmul_cuda,
    int4_matmul_pytorch,
    pack_int4_to_int32,
    transpose_packed,
    unpack_int32_to_int4,
)
from .linear import prepare_w4a4_weight, w4a4_flatquant_linear
from .decompose import get_decompose_dim
from . import meta_ops  # noqa: F401  (registers fakes once the schemas exist)

# True when the HIP operators are registered (the reference: the flatquant
# extension loaded, __init__.py:33-37).
CUDA_AVAILABLE = _loader.KERNELS_AVAILABLE

__all__ = [
    "flatquant_dynamic_quantize",
    "dequantize_int4",
    "int4_matmul",
    "get_decompose_dim",
    "CUDA_AVAILABLE",
]
