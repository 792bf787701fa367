"""GPU parity of the 256-row tiled GEMM kernels (gemm_i4_pp2 for 16-bit
outputs, gemm_i4_pp for float32) at shapes that route to them: more than half
a round of 256 x 224 / 256 x 256 tiles, ragged row and column edges, short K
(one, three and five 128-deep stages: the copy ring's tail and the last load
slot that converts the scales), both B layouts, fp16 / bf16 / fp32 outputs,
with and without bias. Every output is compared bit for bit with the oracle
(int4_matmul_pytorch, int4_matmul/ops.py:69-103) and with the register-staged
kernel on the same inputs."""
import pytest
import torch

from quant_ops_amd import capi
from quant_ops_amd import workloads as wl
from oracle import int4_reference as oi4

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-gemm-tiles] {msg}", flush=True)


# (4000, 2100): 160 tiles of 256 x 224 (last row tile 160 rows, last column tile 84 columns);
# (4000, 4000): 256 tiles of 256 x 256 (last tiles 160 rows, 160 columns)
CASES = [(4000, 2100, 128), (4000, 2100, 384), (4000, 4000, 640), (4000, 2100, 1152)]


@pytest.mark.parametrize("m,n,k", CASES)
@pytest.mark.parametrize("bview", [False, True])
@pytest.mark.parametrize("odt", [torch.float16, torch.bfloat16, torch.float32])
def test_tiled_gemm_edges_and_short_k(gpu, m, n, k, bview, odt, routing):
    case = wl.gemm_case(m, n, k, seed=m + 7 * n + k + int(bview), b_transposed_view=bview, out_dtype=odt)
    _say(f"tiled gemm {m}x{n}x{k} bview={bview} {odt}")
    a, b = case.a.to(gpu), case.b.to(gpu)
    sa, sb = case.scale_a.to(gpu), case.scale_b.to(gpu)
    out = capi.int4_gemm(a, b, sa, sb, out_dtype=odt)
    routing.on("GEMM_NO_DMA")
    out_ref_kernel = capi.int4_gemm(a, b, sa, sb, out_dtype=odt)
    routing.off("GEMM_NO_DMA")
    torch.cuda.synchronize()
    assert torch.equal(out, out_ref_kernel)
    ref = oi4.int4_matmul_pytorch(case.a, case.b, case.scale_a, case.scale_b, out_dtype=odt)
    assert torch.equal(out.cpu(), ref)


@pytest.mark.parametrize("bview", [False, True])
@pytest.mark.parametrize("odt", [torch.float16, torch.bfloat16])
def test_tiled_gemm_bias_and_scale_dtypes(gpu, bview, odt):
    m, n, k = 4000, 2100, 640
    case = wl.gemm_case(m, n, k, seed=91 + int(bview), b_transposed_view=bview, out_dtype=odt)
    g = torch.Generator().manual_seed(92)
    bias = (torch.randn(n, generator=g) * 0.5).to(odt)
    for sdt in (torch.float32, torch.float16, torch.bfloat16):
        _say(f"tiled gemm bias {m}x{n}x{k} bview={bview} {odt} scales {sdt}")
        sa, sb = case.scale_a.to(sdt), case.scale_b.to(sdt)
        out = capi.int4_gemm(case.a.to(gpu), case.b.to(gpu), sa.to(gpu), sb.to(gpu), out_dtype=odt,
                             bias=bias.to(gpu))
        torch.cuda.synchronize()
        ref = oi4.int4_matmul_pytorch(case.a, case.b, sa.float(), sb.float(), out_dtype=odt) + bias
        assert torch.equal(out.cpu(), ref)
