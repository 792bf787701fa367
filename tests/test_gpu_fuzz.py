"""Seeded random sweep of the two HIP entry points against the oracle.

Quantize: random feature counts of the form M x N (M from 16 to 128, N from
32 to 128; at least 3584 codes per case, so that check_quant's flip budget
is meaningful), token counts, dtypes,
clip ratios and both code layouts, with a few zero tokens; codes and scales
checked with check_quant's tolerances. GEMM: random M, N, K (K a multiple of
8), both B layouts, output dtypes and scale dtypes, with and without bias;
every output bit-exact against int4_matmul_pytorch (int4_matmul/ops.py:69-103)
plus the reference's bias addition, on the integer kernels and (16-bit
outputs) on the FP6 route, through the workspace entry point and through
prepare / run at every M. Each case prints its parameters first, so
a failure names its case.
"""
import random

import pytest
import torch

from quant_ops_amd import capi
from quant_ops_amd import workloads as wl
from oracle import int4_reference as oi4

from test_gpu_parity import check_quant

pytestmark = pytest.mark.gpu

QUANT_CASES = 24
GEMM_CASES = 32


def _say(msg):
    print(f"[gpu-fuzz] {msg}", flush=True)


def _quant_case(i):
    r = random.Random(1000 + i)
    m = r.choice([16, 24, 32, 48, 64, 80, 96, 112, 128])
    n = r.choice([32, 48, 64, 96, 128])
    tokens = r.choice([7, 16, 33, 100, 257, 600])
    dtype = r.choice([torch.float16, torch.bfloat16, torch.float32])
    clip = r.choice([1.0, 0.95, 0.9, 0.8, 0.6])
    pack = r.random() < 0.7
    return m, n, tokens, dtype, clip, pack


@pytest.mark.parametrize("i", range(QUANT_CASES))
def test_quantize_random_case(gpu, i):
    m, n, tokens, dtype, clip, pack = _quant_case(i)
    _say(f"quantize case {i}: T={tokens} {m}x{n} {dtype} clip={clip} pack={pack}")
    case = wl.quant_case("fuzz", tokens, m, n, dtype, clip, pack, seed=2000 + i, outlier_frac=0.01,
                         outlier_scale=25.0)
    if tokens > 2:
        case.x[tokens // 3].zero_()
    x, L, R = case.x.to(gpu), case.left.to(gpu), case.right.to(gpu)
    q, s = capi.flatquant_quantize(x, L, R, clip, pack)
    torch.cuda.synchronize()
    check_quant(case.x, case.left, case.right, clip, pack, q, s, f"fuzz quantize {i}")


def _gemm_case(i):
    r = random.Random(5000 + i)
    m = r.choice([1, 3, 16, 17, 64, 65, 128, 200, 256, 300, 513])
    n = r.choice([1, 5, 16, 31, 64, 100, 224, 256, 300, 1000])
    k = 8 * r.choice([1, 3, 8, 16, 17, 64, 129, 256])
    bview = r.random() < 0.5
    odt = r.choice([torch.float16, torch.bfloat16, torch.float32])
    sdt = r.choice([torch.float32, torch.float16, torch.bfloat16])
    with_bias = odt != torch.float32 and r.random() < 0.4
    return m, n, k, bview, odt, sdt, with_bias


@pytest.mark.parametrize("i", range(GEMM_CASES))
def test_gemm_random_case(gpu, i):
    m, n, k, bview, odt, sdt, with_bias = _gemm_case(i)
    _say(f"gemm case {i}: {m}x{n}x{k} bview={bview} out={odt} scales={sdt} bias={with_bias}")
    case = wl.gemm_case(m, n, k, seed=7000 + i, b_transposed_view=bview, out_dtype=odt)
    sa, sb = case.scale_a.to(sdt), case.scale_b.to(sdt)
    bias = None
    if with_bias:
        g = torch.Generator().manual_seed(8000 + i)
        bias = (torch.randn(n, generator=g) * 0.5).to(odt)
    out = capi.int4_gemm(case.a.to(gpu), case.b.to(gpu), sa.to(gpu), sb.to(gpu), out_dtype=odt,
                         bias=None if bias is None else bias.to(gpu))
    torch.cuda.synchronize()
    ref = oi4.int4_matmul_pytorch(case.a, case.b, sa.float(), sb.float(), out_dtype=odt)
    if bias is not None:
        ref = ref + bias
    assert torch.equal(out.cpu(), ref)
    if odt != torch.float32:
        # the same call with a workspace (the FP6 route above 256 rows) and the
        # FP6 kernels at any M through prepare / run
        out_ws = capi.int4_gemm(case.a.to(gpu), case.b.to(gpu), sa.to(gpu), sb.to(gpu), out_dtype=odt,
                                bias=None if bias is None else bias.to(gpu), workspace=True)
        ws = torch.empty(capi.f6_workspace_bytes(m, n, k), dtype=torch.uint8, device=gpu)
        capi.f6_prepare(ws, m, n, k, a=case.a.to(gpu), b=case.b.to(gpu))
        out_f6 = capi.f6_run(ws, m, n, k, sa.to(gpu), sb.to(gpu), out_dtype=odt,
                             bias=None if bias is None else bias.to(gpu))
        torch.cuda.synchronize()
        assert torch.equal(out_ws.cpu(), ref)
        assert torch.equal(out_f6.cpu(), ref)
