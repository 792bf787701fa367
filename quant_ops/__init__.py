"""quant_ops — the reference's import surface over the MI355X build.

Callers written against libarry/quant_ops import from here unchanged
(``src/quant_ops/__init__.py:16-45``): the public names, ``__version__`` and
``CUDA_AVAILABLE``, and the subpackages ``quant_ops.ops.quantization.flatquant``,
``quant_ops.ops.quantization.int4_matmul``, ``quant_ops.utils`` and
``quant_ops.meta_ops``. Every name is the one defined in ``quant_ops_amd``;
nothing is computed here.

Import order follows the reference's: the operators (which load the native
library and define the ``quant_ops::*`` schemas), the fake kernels, then the
availability flag.
"""
__version__ = "0.1.0"

from .ops.quantization.flatquant import dequantize_int4, flatquant_dynamic_quantize
from .ops.quantization.int4_matmul.ops import int4_matmul
from .utils.decompose import get_decompose_dim
from . import meta_ops  # noqa: F401

try:
    from .ops.quantization.flatquant.kernels import CUDA_KERNELS_AVAILABLE, cuda_quant_ops
    CUDA_AVAILABLE = CUDA_KERNELS_AVAILABLE and cuda_quant_ops is not None
except ImportError:  # pragma: no cover - the kernels module never raises here
    CUDA_AVAILABLE = False

__all__ = [
    "flatquant_dynamic_quantize",
    "dequantize_int4",
    "int4_matmul",
    "get_decompose_dim",
    "CUDA_AVAILABLE",
]
