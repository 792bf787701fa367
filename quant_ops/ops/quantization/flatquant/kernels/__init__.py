"""The FlatQuant extension module and its availability flag (reference
``flatquant/kernels/__init__.py:7-34``): ``cuda_quant_ops.cuda_kronecker_quant_int8``
runs the HIP kernel; ``cuda_quant_ops`` is None and the flag False when the HIP
library is not loaded (the reference raises ImportError instead)."""
from quant_ops_amd.extension import CUDA_KERNELS_AVAILABLE, cuda_quant_ops

__all__ = ["cuda_quant_ops", "CUDA_KERNELS_AVAILABLE"]
