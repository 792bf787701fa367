"""GPU parity at the sizes bench.py times and on the inputs of the reference's
own examples.

* The linear entry point (qo_w4a4_linear) at config 5's prefill size, the call
  bench.py times as ``linear_cfg5_T4096``: 4096 tokens of bf16 x 14336
  features (112 x 128 transforms, clip 0.9) against a [4096, 14336] weight,
  bf16 out. Its codes and scales equal the quantize entry point's bit for bit
  and meet the quantize bars against the oracle on sampled tokens; its output
  equals the fallback's GEMM on them, bit for bit, on sampled rows.
* ``examples/basic_usage.py:28-38,76``: 16384 x 4096 bf16 with L, R =
  randn / 64 (not orthogonal), clip 0.6, int8 codes.
* ``examples/int4_matmul_benchmark.py:15-27,62-66``: (M, K, N) = (1024, 256,
  256), (1024, 512, 512), (1024, 1024, 1024), codes uniform in [-8, 7], B
  packed as ``pack(b.T).T`` (the [K/8, N] layout), float32 scales
  U(0.01, 0.11) on both sides; bit-exact against int4_matmul_pytorch.

Inputs come from seeded CPU generators, as everywhere in these tests (the
examples seed torch's CUDA generator, whose draws this container cannot
reproduce; the shapes, distributions and call arguments are the examples').
"""
import pytest
import torch

import quant_ops_amd as qo
from quant_ops_amd import capi
from quant_ops_amd import workloads as wl
from oracle import fq_reference as ofq
from oracle import int4_reference as oi4

from test_gpu_parity import check_quant

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-benched] {msg}", flush=True)


def test_linear_entry_point_cfg5_prefill(gpu):
    tokens, m, n, out_f = 4096, 112, 128, 4096
    x = wl.activations(tokens, m * n, torch.bfloat16, seed=31, outlier_frac=0.005, outlier_scale=30.0)
    L, R = wl.orthogonal(m, 32, torch.bfloat16), wl.orthogonal(n, 33, torch.bfloat16)
    w = wl.random_packed(out_f, m * n // 8, 34)                # [out, in/8], passed as W.t()
    sw = wl.uniform(out_f, 0.001, 0.01, 35)
    _say(f"qo_w4a4_linear T={tokens} {m}x{n} -> {out_f} bf16 clip 0.9")
    xd, Ld, Rd, wd, swd = x.to(gpu), L.to(gpu), R.to(gpu), w.to(gpu), sw.to(gpu)
    y, q, s = capi.w4a4_linear(xd, Ld, Rd, wd, swd, 0.9)
    q2, s2 = capi.flatquant_quantize(xd, Ld, Rd, 0.9, True)
    torch.cuda.synchronize()
    assert y.shape == (tokens, out_f) and y.dtype == torch.bfloat16
    assert torch.equal(q, q2) and torch.equal(s, s2)
    rows = torch.cat([torch.arange(0, tokens, 11), torch.tensor([tokens - 1])])
    check_quant(x[rows], L, R, 0.9, True, q.cpu()[rows], s.cpu()[rows], f"linear T={tokens} (sampled tokens)")
    ref = oi4.int4_matmul_pytorch(q.cpu()[rows], w.t(), s.cpu()[rows], sw, out_dtype=torch.bfloat16)
    assert torch.equal(y.cpu()[rows], ref)


def test_basic_usage_example_inputs(gpu):
    tokens, features, m = 16384, 4096, 64
    g = torch.Generator().manual_seed(42)
    x = torch.randn(tokens, features, generator=g).to(torch.bfloat16)
    left = torch.randn(m, m, generator=g).to(torch.bfloat16) / m
    right = torch.randn(m, m, generator=g).to(torch.bfloat16) / m
    _say(f"basic_usage: {tokens} x {features} bf16, L, R = randn / {m}, clip 0.6, int8 codes")
    q, s = qo.flatquant_cuda(x.to(gpu), left.to(gpu), right.to(gpu), 0.6)
    torch.cuda.synchronize()
    assert q.dtype == torch.int8 and q.shape == (tokens, features) and s.shape == (tokens,)
    rows = torch.cat([torch.arange(0, tokens, 8), torch.tensor([tokens - 1])])
    check_quant(x[rows], left, right, 0.6, False, q.cpu()[rows], s.cpu()[rows], "basic_usage (sampled tokens)")


@pytest.mark.parametrize("m,k,n", [(1024, 256, 256), (1024, 512, 512), (1024, 1024, 1024)])
def test_int4_matmul_benchmark_example_inputs(gpu, m, k, n):
    g = torch.Generator().manual_seed(42)
    a = torch.randint(-8, 8, (m, k), generator=g, dtype=torch.int8)
    b = torch.randint(-8, 8, (k, n), generator=g, dtype=torch.int8)
    a_packed = torch.from_numpy(oi4.pack_int4_to_int32(a.numpy()))
    b_packed = torch.from_numpy(oi4.pack_int4_to_int32(b.T.contiguous().numpy())).T.contiguous()
    scale_a = torch.rand(m, generator=g) * 0.1 + 0.01
    scale_b = torch.rand(n, generator=g) * 0.1 + 0.01
    _say(f"int4_matmul_benchmark: ({m}, {k}, {n}), float32 scales U(0.01, 0.11), [K/8, N] B")
    out = qo.int4_matmul_cuda(a_packed.to(gpu), b_packed.to(gpu), scale_a.to(gpu), scale_b.to(gpu))
    out_op = qo.int4_matmul(a_packed.to(gpu), b_packed.to(gpu), scale_a.to(gpu), scale_b.to(gpu))
    torch.cuda.synchronize()
    ref = oi4.int4_matmul_pytorch(a_packed, b_packed, scale_a, scale_b)
    assert out.dtype == torch.float16 and out.shape == (m, n)
    assert torch.equal(out.cpu(), ref) and torch.equal(out_op.cpu(), ref)
    # the example's own accuracy figure: against the matmul of the codes, scaled
    base = (a.float() @ b.float()) * scale_a.view(-1, 1) * scale_b.view(1, -1)
    assert float((out.cpu().float() - base).abs().max()) <= 1e-2 * float(base.abs().max())
