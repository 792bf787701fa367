"""GPU test of qo_w4a4_linear_noalloc, the linear layer whose activation codes
and scales are staged in the library's per-GPU array instead of caller
buffers: consecutive calls, each smaller than the one before, each equal bit
for bit to qo_w4a4_linear on the same inputs (the existing entry point's own
parity against the oracle is covered by the linear tests)."""
import pytest
import torch

from quant_ops_amd import capi
from quant_ops_amd import workloads as wl

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-noalloc] {msg}", flush=True)


def _inputs(tokens, m, n, out_f, dtype, seed, with_bias):
    x = wl.activations(tokens, m * n, dtype, seed=seed, outlier_frac=0.01, outlier_scale=20.0)
    L, R = wl.orthogonal(m, seed + 1, dtype), wl.orthogonal(n, seed + 2, dtype)
    w = wl.random_packed(out_f, m * n // 8, seed + 3)
    sw = wl.uniform(out_f, 0.001, 0.01, seed + 4)
    g = torch.Generator().manual_seed(seed + 5)
    bias = (torch.randn(out_f, generator=g) * 0.5).to(dtype) if with_bias else None
    return x, L, R, w, sw, bias


def test_linear_noalloc_matches_linear(gpu):
    # a prefill-sized call (tiled GEMM), then a smaller decode call (skinny GEMM
    # and the weight read-ahead), then a smaller one with another row length
    cases = [(300, 112, 128, 4096, torch.bfloat16, True, 0.9),
             (16, 112, 128, 4096, torch.bfloat16, True, 0.9),
             (5, 64, 64, 272, torch.float16, False, 1.0)]
    for i, (tokens, m, n, out_f, dtype, with_bias, clip) in enumerate(cases):
        x, L, R, w, sw, bias = _inputs(tokens, m, n, out_f, dtype, 900 + 7 * i, with_bias)
        _say(f"call {i}: T={tokens} {m}x{n} out={out_f} {dtype} bias={with_bias}")
        xd, Ld, Rd, wd, swd = x.to(gpu), L.to(gpu), R.to(gpu), w.to(gpu), sw.to(gpu)
        bd = bias.to(gpu) if bias is not None else None
        y_ref, _, _ = capi.w4a4_linear(xd, Ld, Rd, wd, swd, clip, bd)
        y = capi.w4a4_linear_noalloc(xd, Ld, Rd, wd, swd, clip, bd)
        torch.cuda.synchronize()
        assert torch.equal(y, y_ref), f"call {i}: noalloc output differs from qo_w4a4_linear"


def test_linear_noalloc_on_a_side_stream(gpu):
    # a non-null stream of the current device (its device is checked), after
    # the calls above left the staging array holding other codes
    x, L, R, w, sw, bias = _inputs(12, 112, 128, 1000, torch.bfloat16, 950, True)
    xd, Ld, Rd, wd, swd, bd = (t.to(gpu) for t in (x, L, R, w, sw, bias))
    y_ref, _, _ = capi.w4a4_linear(xd, Ld, Rd, wd, swd, 0.9, bd)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        y = capi.w4a4_linear_noalloc(xd, Ld, Rd, wd, swd, 0.9, bd)
    side.synchronize()
    assert torch.equal(y, y_ref)


def test_linear_noalloc_rejects_oversize(gpu):
    # staging need above the limit: 5000 tokens x 14336 features (35.8 MB of codes)
    x = torch.zeros(5000, 14336, dtype=torch.bfloat16, device=gpu)
    L = torch.eye(112, dtype=torch.bfloat16, device=gpu)
    R = torch.eye(128, dtype=torch.bfloat16, device=gpu)
    w = torch.zeros(16, 14336 // 8, dtype=torch.int32, device=gpu)
    sw = torch.ones(16, device=gpu)
    with pytest.raises(capi.QuantOpsError, match="staging"):
        capi.w4a4_linear_noalloc(x, L, R, w, sw, 1.0)
