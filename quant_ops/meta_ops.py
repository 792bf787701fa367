"""Fake (meta) kernels of the ``quant_ops::*`` operators (reference ``src/quant_ops/meta_ops.py:22-37``).

Importing this module registers them; the registration itself lives in
``quant_ops_amd.meta_ops`` and runs once per process.
"""
from quant_ops_amd import meta_ops as _registered  # noqa: F401
