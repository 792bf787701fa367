"""Int4 matmul entry points and the packing helpers (reference ``int4_matmul/ops.py:1-157``),
defined in ``quant_ops_amd.int4_matmul``."""
from quant_ops_amd.int4_matmul import (  # noqa: F401
    int4_matmul,
    int4_matmul_cuda,
    int4_matmul_pytorch,
    pack_int4_to_int32,
    unpack_int32_to_int4,
)
from .kernels import CUDA_KERNELS_AVAILABLE, cuda_int4_matmul_ops  # noqa: F401
