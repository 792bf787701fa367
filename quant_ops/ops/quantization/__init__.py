"""Quantization operators (reference ``src/quant_ops/ops/quantization/__init__.py``)."""
from . import flatquant

__all__ = ["flatquant"]
