"""Kronecker factor search (reference ``utils/decompose.py:11-39``), defined in ``quant_ops_amd.decompose``."""
from quant_ops_amd.decompose import get_decompose_dim  # noqa: F401
