"""The int4 matmul extension module and its availability flag (reference
``int4_matmul/kernels/__init__.py:5-44``): ``cuda_int4_matmul_ops.cuda_int4_matmul``
runs the HIP GEMM; None and False when the HIP library is not loaded."""
from quant_ops_amd.extension import CUDA_KERNELS_AVAILABLE, cuda_int4_matmul_ops

__all__ = ["cuda_int4_matmul_ops", "CUDA_KERNELS_AVAILABLE"]
