"""Oracle restatement of ``get_decompose_dim`` — test infrastructure only.

Follows ``src/quant_ops/utils/decompose.py:11-39`` of the reference: starting
from ``a = ceil(sqrt(n))`` it looks for the first ``a`` for which ``a*a - n`` is a
perfect square ``b*b`` and returns ``(a - b, a + b)``; the product is ``n``.
"""
import math


def get_decompose_dim(n: int):
    """Return ``(M, N)`` with ``M * N == n`` from the difference of squares.

    Reference: ``utils/decompose.py:30-39`` (``a`` from ``int(math.sqrt)``
    rounded up, then a linear search on ``a``).
    """
    if n % 4 == 2:
        # a^2 - b^2 == n has no integer solution; the reference's search loop
        # never terminates for such n (decompose.py:33-38).
        raise ValueError(f"{n} is not a difference of two squares")
    a = math.isqrt(n)
    if a * a < n:
        a += 1
    while True:
        d = a * a - n
        b = math.isqrt(d)
        if b * b == d:
            return a - b, a + b
        a += 1
