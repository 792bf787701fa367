"""Int4 matrix multiplication (reference ``int4_matmul/__init__.py``)."""
from .ops import int4_matmul, int4_matmul_cuda, int4_matmul_pytorch

__all__ = ["int4_matmul_cuda", "int4_matmul_pytorch", "int4_matmul"]
