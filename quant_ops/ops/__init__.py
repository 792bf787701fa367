"""Operators by family (reference ``src/quant_ops/ops/__init__.py``)."""
from .quantization import flatquant

__all__ = ["flatquant"]
