"""FlatQuant dynamic quantization (reference ``flatquant/__init__.py``)."""
from .ops import dequantize_int4, flatquant_cuda, flatquant_dynamic_quantize, flatquant_pytorch

__all__ = [
    "flatquant_cuda",
    "flatquant_pytorch",
    "flatquant_dynamic_quantize",
    "dequantize_int4",
]
