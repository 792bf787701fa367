"""The arithmetic the FP6 GEMM route relies on, checked on the CPU.

* Every int4 code q (-8 .. 7) divided by 8 is an FP6 e2m3 value, and its
  encoding is sign-magnitude (sign in bit 5, |q| in bits 0 .. 3, bit 4 zero).
  The decoder below follows the OCP Microscaling (MX) v1.0 definition of
  e2m3: 1 sign bit, 2 exponent bits with bias 1, 3 mantissa bits, exponent
  field 0 subnormal (value m / 8), otherwise 2^(e - 1) (1 + m / 8); no
  infinities or NaNs. A wrong sign position, a wrong bias or a code that
  sets bit 4 fails it.
* With block scales 2^3 on both operands each product is q_a q_b exactly, and
  every partial sum of a K-long dot product is an integer of magnitude at
  most 64 K; float32 holds all integers below 2^24, so sums are exact for
  K <= 65536 (the route's limit, 64 K = 2^22), and not beyond 2^18.
"""
import numpy as np


def e2m3_value(code: int) -> float:
    sign = -1.0 if code & 0b100000 else 1.0
    e = (code >> 3) & 0b11
    m = code & 0b111
    if e == 0:
        return sign * m / 8.0
    return sign * 2.0 ** (e - 1) * (1.0 + m / 8.0)


def sign_magnitude(q: int) -> int:
    return (32 if q < 0 else 0) | abs(q)


def test_every_int4_code_over_8_is_its_sign_magnitude_e2m3_code():
    for q in range(-8, 8):
        code = sign_magnitude(q)
        assert code < 64 and code & 0b10000 == 0
        assert e2m3_value(code) == q / 8.0


def test_e2m3_decoder_matches_the_format_table():
    # the largest magnitude is 7.5, the smallest nonzero 1/8; 64 codes, 63 distinct values (+0 and -0)
    vals = [e2m3_value(c) for c in range(64)]
    assert max(vals) == 7.5 and min(vals) == -7.5
    assert min(v for v in vals if v > 0) == 0.125
    assert len(set(vals)) == 63


def test_float32_sums_are_exact_up_to_the_route_limit():
    # 64 K is the largest |sum| (every code -8); float32 represents it and every
    # smaller integer exactly for K <= 65536, and the next integer is still exact
    for k in (8, 4096, 14336, 65536):
        bound = 64 * k
        assert bound <= 2 ** 22
        x = np.float32(bound)
        assert int(x) == bound and int(np.float32(bound - 1)) == bound - 1
    # a product of two codes scaled by 2^3 each: (q_a / 8 * 8) * (q_b / 8 * 8) = q_a q_b exactly
    for qa in range(-8, 8):
        for qb in range(-8, 8):
            assert np.float32(e2m3_value(sign_magnitude(qa)) * 8) * np.float32(e2m3_value(sign_magnitude(qb)) * 8) \
                == qa * qb
