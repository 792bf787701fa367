"""Pins the CPU oracle against things other than itself (runs on the CPU).

Each check is chosen so that a plausible transcription mistake in the oracle
(transposed L, L instead of L^T, missing clip factor, rounding at the wrong
point, wrong nibble order, wrong sign convention) fails at least one of them.
"""
import math

import numpy as np
import pytest
import torch

from oracle import decompose as odec
from oracle import fq_reference as ofq
from oracle import int4_reference as oi4

DTYPES = [torch.float32, torch.float16, torch.bfloat16]


# --------------------------------------------------------------------------- decompose

def test_decompose_docstring_kats():
    # utils/decompose.py:24-28
    assert odec.get_decompose_dim(4096) == (64, 64)
    assert odec.get_decompose_dim(2048) == (32, 64)


def test_decompose_closed_form_exhaustive():
    # (a-b)(a+b) == n with the smallest a >= ceil(sqrt n), by brute force over a.
    for n in range(1, 3000):
        if n % 4 == 2:
            with pytest.raises(ValueError):
                odec.get_decompose_dim(n)
            continue
        m, k = odec.get_decompose_dim(n)
        assert m * k == n and m <= k
        a = (m + k) // 2
        lo = math.isqrt(n) + (0 if math.isqrt(n) ** 2 == n else 1)
        for a2 in range(lo, a):
            r = a2 * a2 - n
            assert math.isqrt(r) ** 2 != r, (n, a2)
    assert odec.get_decompose_dim(14336) == (112, 128)


# --------------------------------------------------------------------------- pack / unpack

def test_pack_known_answers():
    codes = np.array([[-8, -7, -6, -5, -4, -3, -2, -1]], dtype=np.int8)
    assert oi4.pack_int4_to_int32(codes)[0, 0] == 0x76543210
    assert oi4.pack_int4_to_int32(np.full((1, 8), 7, np.int8))[0, 0] == -1
    assert oi4.pack_int4_to_int32(np.full((1, 8), -8, np.int8))[0, 0] == 0
    # code 0 everywhere is 0x88888888 as a signed int32
    assert oi4.pack_int4_to_int32(np.zeros((1, 8), np.int8))[0, 0] == np.int32(np.uint32(0x88888888).view(np.int32))


def test_pack_known_answers_out_of_range_codes():
    # (q + 8) mod 256 per code, shifted sums mod 2^32 (int8 add, uint8 cast and
    # int32 sum of int4_matmul/ops.py:36-43), worked by hand:
    #   127 -> 0x87: 0x87 * 0x11111111 = 0x8FFFFFFF7 -> 0xFFFFFFF7
    #  -128 -> 0x88: 0x88 * 0x11111111 = 0x911111108 -> 0x11111108
    #   -9  -> 0xFF in slot 0 only: 0xFF + 0x88888880 (the seven zero codes)
    def word(codes):
        return int(np.uint32(oi4.pack_int4_to_int32(np.array([codes], dtype=np.int8))[0, 0].view(np.uint32)))

    assert word([127] * 8) == 0xFFFFFFF7
    assert word([-128] * 8) == 0x11111108
    assert word([-9] + [0] * 7) == 0x8888897F


def test_pack_closed_form_and_roundtrip():
    rng = np.random.default_rng(0)
    q = rng.integers(-8, 8, size=(17, 64), dtype=np.int8)
    w = oi4.pack_int4_to_int32(q)
    for r in range(q.shape[0]):
        for p in range(8):
            expect = sum(int(q[r, 8 * p + i] + 8) << (4 * i) for i in range(8))
            assert int(np.uint32(w[r, p].view(np.uint32))) == expect
    assert np.array_equal(oi4.unpack_int32_to_int4(w), q)


# --------------------------------------------------------------------------- GEMM

@pytest.mark.parametrize("m,n,k", [(1, 1, 8), (5, 7, 16), (16, 33, 64), (3, 4, 1024)])
def test_gemm_oracle_matches_int64_bruteforce(m, n, k):
    rng = np.random.default_rng(m * 100 + n)
    qa = rng.integers(-8, 8, size=(m, k), dtype=np.int8)
    qb = rng.integers(-8, 8, size=(k, n), dtype=np.int8)
    a = oi4.pack_int4_to_int32(qa)
    b = oi4.pack_int4_to_int32(qb.T).T.copy()     # examples/int4_matmul_benchmark.py:22
    exact = qa.astype(np.int64) @ qb.astype(np.int64)
    assert np.array_equal(oi4.int4_gemm_int64(a, b), exact)
    assert np.array_equal(oi4.int4_matmul_int32(torch.from_numpy(a), torch.from_numpy(b)).numpy(), exact)
    sa = torch.rand(m) * 0.1 + 0.01
    sb = torch.rand(n) * 0.01 + 0.001
    out = oi4.int4_matmul_pytorch(torch.from_numpy(a), torch.from_numpy(b), sa, sb)
    # (acc * sa) * sb in float32, one rounding to float16 (int4_matmul/ops.py:96-103)
    ref = ((exact.astype(np.float32) * sa.numpy()[:, None]).astype(np.float32) * sb.numpy()[None, :]).astype(np.float16)
    assert out.dtype == torch.float16
    assert np.array_equal(out.numpy().view(np.uint16), ref.view(np.uint16))


def test_gemm_extreme_accumulator_exact():
    # all -8 x -8: the largest |acc| = 64 K, still exact in float32 for K = 14336
    k = 14336
    a = oi4.pack_int4_to_int32(np.full((2, k), -8, np.int8))
    b = oi4.pack_int4_to_int32(np.full((3, k), -8, np.int8)).T.copy()
    acc = oi4.int4_matmul_int32(torch.from_numpy(a), torch.from_numpy(b))
    assert (acc == 64 * k).all()


# --------------------------------------------------------------------------- transform + quantize

def _case(t, m, n, dtype, seed=0, outliers=False):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(t, m * n, generator=g)
    if outliers:
        x[:, :: max(1, (m * n) // 16)] *= 20
    L = torch.linalg.qr(torch.randn(m, m, generator=g))[0]
    R = torch.linalg.qr(torch.randn(n, n, generator=g))[0]
    return x.to(dtype), L.to(dtype), R.to(dtype)


@pytest.mark.parametrize("m,n", [(2, 4), (4, 4), (3, 5), (8, 16)])
def test_transform_matches_kron_bruteforce_fp32(m, n):
    # y_row = x_row @ kron(L, R): catches L vs L^T, R vs R^T and the m/n order.
    g = torch.Generator().manual_seed(1)
    x = torch.randn(6, m * n, generator=g, dtype=torch.float64)
    L = torch.randn(m, m, generator=g, dtype=torch.float64)   # non-symmetric on purpose
    R = torch.randn(n, n, generator=g, dtype=torch.float64)
    y_ref = ofq.kron_transform_f64(x.numpy(), L.numpy(), R.numpy())
    y = torch.matmul(L.T, torch.matmul(x.reshape(-1, m, n), R)).reshape(6, m * n)
    np.testing.assert_allclose(y.numpy(), y_ref, rtol=1e-12, atol=1e-12)
    # and the oracle's own codes equal the closed form from that transform (fp32)
    xq = x.float()
    codes, scale = ofq.flatquant_pytorch(xq, L.float(), R.float(), 0.9, False)
    y32 = torch.matmul(L.float().T, torch.matmul(xq.reshape(-1, m, n), R.float())).reshape(6, m * n)
    np.testing.assert_allclose(y32.double().numpy(), y_ref, rtol=1e-4, atol=1e-4)
    s_cf, q_cf = ofq.quantize_rows_closed_form(y32.double().numpy(), torch.float32, 0.9)
    np.testing.assert_array_equal(scale.double().numpy(), s_cf)
    np.testing.assert_array_equal(codes.numpy(), q_cf.astype(np.int8))


@pytest.mark.parametrize("dtype", DTYPES)
def test_scale_and_codes_closed_form_with_rounding_points(dtype):
    x, L, R = _case(32, 8, 16, dtype, seed=3, outliers=True)
    codes, scale = ofq.flatquant_pytorch(x, L, R, 0.9, False)
    assert scale.dtype == dtype and scale.shape == (32,)
    # Y with both rounding points taken explicitly, then the closed-form scale/codes
    z = torch.matmul(x.reshape(-1, 8, 16), R)           # rnd_D(X R)
    y = torch.matmul(L.T, z).reshape(32, 128)            # rnd_D(L^T Z)
    s_cf, q_cf = ofq.quantize_rows_closed_form(y.double().numpy(), dtype, 0.9)
    np.testing.assert_array_equal(scale.double().numpy(), s_cf)
    np.testing.assert_array_equal(codes.numpy().astype(np.int64), q_cf.astype(np.int64))


@pytest.mark.parametrize("m,n", [(4, 4), (16, 16), (7, 8)])
def test_orthogonal_transform_preserves_norm(m, n):
    g = torch.Generator().manual_seed(5)
    x = torch.randn(4, m * n, generator=g, dtype=torch.float64)
    L = torch.linalg.qr(torch.randn(m, m, generator=g, dtype=torch.float64))[0]
    R = torch.linalg.qr(torch.randn(n, n, generator=g, dtype=torch.float64))[0]
    y = ofq.kron_transform_f64(x.numpy(), L.numpy(), R.numpy())
    np.testing.assert_allclose(np.linalg.norm(y, axis=1), np.linalg.norm(x.numpy(), axis=1), rtol=1e-12)
    # the oracle's fp32 transform agrees with the float64 one to fp32 accuracy
    yo = torch.matmul(L.float().T, torch.matmul(x.float().reshape(-1, m, n), R.float())).reshape(4, m * n)
    np.testing.assert_allclose(yo.double().numpy(), y, rtol=0, atol=1e-5)


@pytest.mark.parametrize("dtype", DTYPES)
def test_identity_transforms_reduce_to_absmax_quantization(dtype):
    g = torch.Generator().manual_seed(7)
    x = (torch.randn(5, 64, generator=g) * 3).to(dtype)
    eye8 = torch.eye(8, dtype=dtype)
    codes, scale = ofq.flatquant_pytorch(x, eye8, eye8, 1.0, False)
    xd = x.double().numpy()
    s_cf, q_cf = ofq.quantize_rows_closed_form(xd, dtype, 1.0)
    np.testing.assert_array_equal(scale.double().numpy(), s_cf)
    np.testing.assert_array_equal(codes.numpy(), q_cf.astype(np.int8))
    # with clip 1 the largest |x| maps to +-7 (or -8 is never reached from a positive max)
    assert (codes.abs().amax(dim=1) == 7).all()


def test_round_half_even_and_clamp_known_answers():
    # identity transforms, scale fixed by a row maximum of 7 -> s = 1: codes are round(x)
    row = torch.tensor([[7.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5]])
    eye = torch.eye(2, dtype=torch.float32)
    eye4 = torch.eye(4, dtype=torch.float32)
    codes, scale = ofq.flatquant_pytorch(row, eye, eye4, 1.0, False)
    assert scale.item() == 1.0
    assert codes.tolist() == [[7, 0, 2, 2, 0, -2, -2, 4]]
    # clip 0.5 doubles |y/s|: values beyond the range clamp to -8 / 7
    codes, scale = ofq.flatquant_pytorch(torch.tensor([[7.0, -7.0, 3.0, -3.0, 0.0, 1.0, -1.0, 2.0]]), eye, eye4, 0.5, False)
    assert scale.item() == 0.5
    assert codes.tolist() == [[7, -8, 6, -6, 0, 2, -2, 4]]


def test_packed_matches_int8_codes():
    x, L, R = _case(9, 8, 8, torch.bfloat16, seed=11)
    q8, s8 = ofq.flatquant_pytorch(x, L, R, 0.95, False)
    q32, s32 = ofq.flatquant_pytorch(x, L, R, 0.95, True)
    assert torch.equal(s8, s32)
    assert np.array_equal(oi4.pack_int4_to_int32(q8.numpy()), q32.numpy())


def test_all_zero_fp16_token_reference_behaviour():
    # rnd_fp16(1e-8) == 0, so the fallback divides 0/0: NaN -> int8 0, and the
    # uint8 cast before packing gives nibble 0 (code -8).
    x = torch.zeros(2, 16, dtype=torch.float16)
    x[1] = torch.arange(16, dtype=torch.float16)
    eye = torch.eye(4, dtype=torch.float16)
    q8, s = ofq.flatquant_pytorch(x, eye, eye, 1.0, False)
    q32, _ = ofq.flatquant_pytorch(x, eye, eye, 1.0, True)
    assert s[0].item() == 0.0
    assert (q8[0] == 0).all()
    assert (q32[0] == 0).all()          # all nibbles 0
    # bf16 keeps a positive floor: codes 0, packed 0x88888888
    xb = x.to(torch.bfloat16)
    eyeb = eye.to(torch.bfloat16)
    qb, sb = ofq.flatquant_pytorch(xb, eyeb, eyeb, 1.0, True)
    assert sb[0].item() > 0 and (qb[0] == np.uint32(0x88888888).view(np.int32)).all()


def test_dequantize_closed_form():
    q = torch.tensor([[-8, 7, 0, 1, -1, 3, -3, 5]], dtype=torch.int8)
    s = torch.tensor([0.25], dtype=torch.float16)
    out = ofq.dequantize_int4(q, s)
    assert out.dtype == torch.float32
    assert out.tolist() == [[-2.0, 1.75, 0.0, 0.25, -0.25, 0.75, -0.75, 1.25]]
    packed = torch.from_numpy(oi4.pack_int4_to_int32(q.numpy()))
    assert torch.equal(ofq.dequantize_int4(packed, s, True), out)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_sequential_variant_matches_closed_form(dtype):
    # sequential float32 accumulation written out element by element on a tiny case
    x, L, R = _case(3, 4, 8, dtype, seed=13, outliers=True)
    q, s = ofq.flatquant_sequential(x, L, R, 0.9, True)
    xd = x.reshape(3, 4, 8).double().numpy()
    Ld, Rd = L.double().numpy(), R.double().numpy()
    z = np.zeros((3, 4, 8))
    for t in range(3):
        for i in range(4):
            for j in range(8):
                acc = np.float32(0)
                for k in range(8):
                    acc = np.float32(acc + np.float32(xd[t, i, k] * Rd[k, j]))
                z[t, i, j] = acc
    zd = torch.from_numpy(z).float().to(dtype).double().numpy()
    y = np.zeros((3, 4, 8))
    for t in range(3):
        for i in range(4):
            for j in range(8):
                acc = np.float32(0)
                for k in range(4):
                    acc = np.float32(acc + np.float32(Ld[k, i] * zd[t, k, j]))
                y[t, i, j] = acc
    yd = torch.from_numpy(y.reshape(3, 32)).float().to(dtype).double().numpy()
    s_cf, q_cf = ofq.quantize_rows_closed_form(yd, dtype, 0.9)
    np.testing.assert_array_equal(s.double().numpy(), s_cf)
    np.testing.assert_array_equal(oi4.unpack_int32_to_int4(q.numpy()), q_cf.astype(np.int8))
