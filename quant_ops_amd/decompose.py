"""``get_decompose_dim`` — the Kronecker factorisation used to size L and R.

Same contract as the reference (``src/quant_ops/utils/decompose.py:11-39``):
for ``n``, take the smallest ``a >= ceil(sqrt(n))`` such that ``a*a - n`` is a
perfect square ``b*b`` and return ``(a - b, a + b)``; their product is ``n``.
"""
import math
from typing import Tuple


def get_decompose_dim(n: int) -> Tuple[int, int]:
    """Return ``(M, N)`` with ``M * N == n`` and ``M <= N`` as close as possible.

    >>> get_decompose_dim(4096)
    (64, 64)
    >>> get_decompose_dim(2048)
    (32, 64)
    >>> get_decompose_dim(14336)
    (112, 128)
    """
    n = int(n)
    if n < 0:
        raise ValueError(f"get_decompose_dim needs a non-negative size, got {n}")
    if n % 4 == 2:
        # No a, b with a^2 - b^2 == n exist; the reference's search would loop forever.
        raise ValueError(f"get_decompose_dim: {n} is not a difference of two squares (n % 4 == 2)")
    a = math.isqrt(n)
    if a * a < n:
        a += 1
    while True:
        b2 = a * a - n
        b = math.isqrt(b2)
        if b * b == b2:
            return a - b, a + b
        a += 1
