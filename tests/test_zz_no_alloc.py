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


def test_linear_noalloc_in_graph_capture(gpu):
    """Captured in a HIP graph (the first no-alloc call of this file runs inside
    the capture, so the staging array's address lookup happens there too) and
    replayed with new inputs copied in, with eager work between the replays:
    every replay equals qo_w4a4_linear on the same inputs, bit for bit."""
    m, n, out_f, dtype = 112, 128, 4096, torch.bfloat16
    inputs = [_inputs(16, m, n, out_f, dtype, 970 + 7 * i, True) for i in range(3)]
    _, L, R, w, sw, bias = inputs[0]
    Ld, Rd, wd, swd, bd = (t.to(gpu) for t in (L, R, w, sw, bias))
    xs = [inp[0].to(gpu) for inp in inputs]
    eager = [capi.w4a4_linear(x, Ld, Rd, wd, swd, 0.9, bd)[0].clone() for x in xs]
    x_static = xs[0].clone()
    out = torch.empty_like(eager[0])
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    _say("capture of qo_w4a4_linear_noalloc")
    with torch.cuda.stream(stream):
        with torch.cuda.graph(g, stream=stream):
            capi.w4a4_linear_noalloc(x_static, Ld, Rd, wd, swd, 0.9, bd, out=out)
    torch.cuda.synchronize()
    for rep in range(4):
        k = rep % 3
        x_static.copy_(xs[k])
        out.zero_()
        g.replay()
        capi.w4a4_linear(xs[(k + 1) % 3], Ld, Rd, wd, swd, 0.9, bd)   # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(out, eager[k]), f"replay {rep}"


def test_linear_noalloc_allocates_nothing(gpu):
    """With the output preallocated, a call changes neither the device's free
    memory (hipMemGetInfo) nor torch's allocated bytes."""
    import ctypes

    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemGetInfo.argtypes = [ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)]
    hip.hipMemGetInfo.restype = ctypes.c_int

    def free_bytes():
        f, t = ctypes.c_size_t(), ctypes.c_size_t()
        assert hip.hipMemGetInfo(ctypes.byref(f), ctypes.byref(t)) == 0
        return f.value

    x, L, R, w, sw, bias = _inputs(64, 112, 128, 4096, torch.bfloat16, 990, True)
    xd, Ld, Rd, wd, swd, bd = (t.to(gpu) for t in (x, L, R, w, sw, bias))
    out = torch.empty(64, 4096, dtype=torch.bfloat16, device=gpu)
    capi.w4a4_linear_noalloc(xd, Ld, Rd, wd, swd, 0.9, bd, out=out)   # warm: the address lookup
    torch.cuda.synchronize()
    f0, a0 = free_bytes(), torch.cuda.memory_allocated()
    for _ in range(3):
        capi.w4a4_linear_noalloc(xd, Ld, Rd, wd, swd, 0.9, bd, out=out)
    torch.cuda.synchronize()
    assert free_bytes() == f0 and torch.cuda.memory_allocated() == a0
    ref = capi.w4a4_linear(xd, Ld, Rd, wd, swd, 0.9, bd)[0]
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


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


def test_linear_noalloc_at_its_token_limit(gpu):
    """The largest call the staging array holds at 14336 features (4678 tokens:
    4678 x 7168 bytes of codes, rounded up to 256, plus 4678 x 4 bytes of
    scales fit in 32 MiB; 4679 do not), equal to qo_w4a4_linear bit for bit."""
    tokens = 4678
    assert (tokens * 7168 + 255) // 256 * 256 + tokens * 4 <= capi.LINEAR_NOALLOC_MAX_BYTES
    assert (4679 * 7168 + 255) // 256 * 256 + 4679 * 4 > capi.LINEAR_NOALLOC_MAX_BYTES
    x, L, R, w, sw, bias = _inputs(tokens, 112, 128, 4096, torch.bfloat16, 995, True)
    _say(f"noalloc at {tokens} tokens")
    xd, Ld, Rd, wd, swd, bd = (t.to(gpu) for t in (x, L, R, w, sw, bias))
    y_ref, _, _ = capi.w4a4_linear(xd, Ld, Rd, wd, swd, 0.9, bd)
    y = capi.w4a4_linear_noalloc(xd, Ld, Rd, wd, swd, 0.9, bd)
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref)
    with pytest.raises(capi.QuantOpsError, match="staging"):
        capi.w4a4_linear_noalloc(torch.cat([xd, xd[:1]]), Ld, Rd, wd, swd, 0.9, bd)


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
