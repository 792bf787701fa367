"""Helpers (reference ``src/quant_ops/utils/__init__.py``)."""
from .decompose import get_decompose_dim

__all__ = ["get_decompose_dim"]
