"""The FP6 route of the W4A4 GEMM (qo_int4_gemm_ws, qo_int4_gemm_f6_prepare /
qo_int4_gemm_f6_run) against the oracle and against the integer route.

The route rewrites the int4 codes as FP6 e2m3 values q / 8 and multiplies
them on the f8f6f4 matrix cores with block scales 2^3; its float32 sums are
exact, so every output must equal int4_matmul_pytorch's
(int4_matmul/ops.py:69-103) bit for bit, the same bar as the integer kernels.
Cases: ragged M, N and K (K not a multiple of 128, K = 8), both B layouts,
both 16-bit outputs, the three scale dtypes, bias; operands and output as
slices of wider buffers (unaligned row strides, an output pitch); the full config 4 and
config 5 (T = 4096) products against qo_int4_gemm's integer route; the
largest K with every product at its extreme (|sum| = 64 K); a weight
converted once and reused; fallback and error paths; graph replay.
"""
import ctypes

import pytest
import torch

from quant_ops_amd import capi
from quant_ops_amd import workloads as wl
from oracle import int4_reference as oi4

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-f6] {msg}", flush=True)


def _ref(case, sa, sb, odt, bias=None):
    ref = oi4.int4_matmul_pytorch(case.a, case.b, sa.float(), sb.float(), out_dtype=odt)
    return ref if bias is None else ref + bias


CASES = [
    # m, n, k, W.t() view, out dtype, scale dtype, bias
    (257, 224, 128, False, torch.float16, torch.float16, False),
    (300, 250, 1000, True, torch.bfloat16, torch.float32, True),
    (513, 1000, 8 * 129, False, torch.float16, torch.bfloat16, False),
    (777, 31, 136, True, torch.float16, torch.float16, True),
    (1024, 1024, 1024, False, torch.bfloat16, torch.float16, True),
    (600, 5, 8, False, torch.float16, torch.float32, False),
    (2000, 3000, 256, True, torch.bfloat16, torch.bfloat16, False),
]


@pytest.mark.parametrize("case_i", range(len(CASES)))
def test_f6_route_matches_oracle(gpu, case_i):
    m, n, k, bview, odt, sdt, with_bias = CASES[case_i]
    _say(f"ws route {m}x{n}x{k} W.t()={bview} out={odt} scales={sdt} bias={with_bias}")
    case = wl.gemm_case(m, n, k, seed=100 + case_i, b_transposed_view=bview, out_dtype=odt)
    sa, sb = case.scale_a.to(sdt), case.scale_b.to(sdt)
    bias = (torch.randn(n, generator=torch.Generator().manual_seed(case_i)) * 0.5).to(odt) if with_bias else None
    assert capi.gemm_workspace_size(m, n, k, odt) > 0   # M > 256: the route is taken
    out = capi.int4_gemm(case.a.to(gpu), case.b.to(gpu), sa.to(gpu), sb.to(gpu), out_dtype=odt,
                         bias=None if bias is None else bias.to(gpu), workspace=True)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), _ref(case, sa, sb, odt, bias))


@pytest.mark.parametrize("m", [1, 16, 200])
def test_prepare_run_small_m_matches_oracle(gpu, m):
    """prepare / run take any M (the ws entry point keeps M <= 256 on the integer kernels)."""
    n, k = 448, 512
    _say(f"prepare/run {m}x{n}x{k}")
    case = wl.gemm_case(m, n, k, seed=200 + m, b_transposed_view=True, out_dtype=torch.bfloat16)
    ws = torch.empty(capi.f6_workspace_bytes(m, n, k), dtype=torch.uint8, device=gpu)
    capi.f6_prepare(ws, m, n, k, a=case.a.to(gpu), b=case.b.to(gpu))
    out = capi.f6_run(ws, m, n, k, case.scale_a.to(gpu), case.scale_b.to(gpu), out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), _ref(case, case.scale_a, case.scale_b, torch.bfloat16))


@pytest.mark.parametrize("cfg", ["cfg4", "cfg5_T4096"])
def test_full_size_equals_integer_route(gpu, cfg):
    if cfg == "cfg4":
        case = wl.gemm_cfg4(seed=3)
    else:
        case = wl.gemm_case(4096, 4096, 14336, seed=4, b_transposed_view=True, out_dtype=torch.bfloat16)
    m, n, k = case.mnk
    _say(f"full size {cfg} {m}x{n}x{k}")
    a, b, sa, sb = case.a.to(gpu), case.b.to(gpu), case.scale_a.to(gpu), case.scale_b.to(gpu)
    f6 = capi.int4_gemm(a, b, sa, sb, out_dtype=case.out_dtype, workspace=True)
    i8 = capi.int4_gemm(a, b, sa, sb, out_dtype=case.out_dtype)
    torch.cuda.synchronize()
    assert torch.equal(f6, i8)
    # and sampled rows against the oracle
    rows = torch.tensor([0, 1, 255, 256, 2047, m - 1])
    sub = wl.GemmCase("rows", case.a[rows], case.b, case.scale_a[rows], case.scale_b, case.out_dtype)
    assert torch.equal(f6[rows.to(gpu)].cpu(), _ref(sub, sub.scale_a, sub.scale_b, case.out_dtype))


def test_extreme_sums_at_largest_k(gpu):
    """K = 65536 with every code -8: each sum is 64 K = 2^22, the largest the route takes."""
    m, n, k = 300, 260, 65536
    _say(f"extreme sums {m}x{n}x{k}")
    a = torch.zeros(m, k // 8, dtype=torch.int32)          # offset code 0 = q -8 in every nibble
    b = torch.zeros(k // 8, n, dtype=torch.int32)
    a[1::2] = 0x7F7F7F7F                                     # rows of alternating q = -1 / 7 codes
    sa = torch.full((m,), 2.0 ** -20, dtype=torch.float32)
    sb = torch.full((n,), 1.0, dtype=torch.float32)
    case = wl.GemmCase("extreme", a, b, sa, sb, torch.float16)
    out = capi.int4_gemm(a.to(gpu), b.to(gpu), sa.to(gpu), sb.to(gpu), workspace=True)
    torch.cuda.synchronize()
    ref = _ref(case, sa, sb, torch.float16)
    assert float(ref[0, 0]) == 4.0                           # 2^22 * 2^-20
    assert torch.equal(out.cpu(), ref)


def test_weight_prepared_once(gpu):
    """B converted once, then several A's converted and multiplied against it."""
    m, n, k = 512, 1000, 2048
    _say(f"weight prepared once {m}x{n}x{k}")
    w = wl.random_packed(n, k // 8, 300)                     # [N, K/8] weight, used as W.t()
    sb = wl.uniform(n, 0.001, 0.01, 301)
    ws = torch.empty(capi.f6_workspace_bytes(m, n, k), dtype=torch.uint8, device=gpu)
    capi.f6_prepare(ws, m, n, k, b=w.to(gpu).t())
    for s in range(3):
        a = wl.random_packed(m, k // 8, 310 + s)
        sa = wl.uniform(m, 0.01, 0.1, 320 + s)
        capi.f6_prepare(ws, m, n, k, a=a.to(gpu))
        out = capi.f6_run(ws, m, n, k, sa.to(gpu), sb.to(gpu))
        torch.cuda.synchronize()
        case = wl.GemmCase("prep", a, w.t(), sa, sb, torch.float16)
        assert torch.equal(out.cpu(), _ref(case, sa, sb, torch.float16))


def test_small_workspace_falls_back_and_run_rejects(gpu):
    m, n, k = 512, 512, 1024
    case = wl.gemm_case(m, n, k, seed=400)
    a, b, sa, sb = case.a.to(gpu), case.b.to(gpu), case.scale_a.to(gpu), case.scale_b.to(gpu)
    need = capi.gemm_workspace_size(m, n, k)
    small = torch.empty(need - 256, dtype=torch.uint8, device=gpu)
    out = capi.int4_gemm(a, b, sa, sb, workspace=small)       # integer route
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), _ref(case, case.scale_a, case.scale_b, torch.float16))
    with pytest.raises(capi.QuantOpsError):
        capi.f6_run(small, m, n, k, sa, sb)
    with pytest.raises(capi.QuantOpsError):
        capi.f6_prepare(small, m, n, k, a=a)
    ws = torch.empty(need + 512, dtype=torch.uint8, device=gpu)
    with pytest.raises(capi.QuantOpsError):                 # not 256-byte aligned
        capi.f6_run(ws[16:], m, n, k, sa, sb)
    with pytest.raises(capi.QuantOpsError):                 # float32 outputs are not on this route
        capi.f6_run(ws, m, n, k, sa, sb, out_dtype=torch.float32)


@pytest.mark.parametrize("bview", [False, True])
def test_padded_operands_and_output_pitch(gpu, bview):
    """A, B and the output as slices of wider buffers: row strides that are
    not multiples of four words (the conversion's word-by-word loads) and an
    output pitch above N; bit-exact against the oracle, the padding left
    untouched."""
    m, n, k = 520, 300, 640
    kp = k // 8
    _say(f"padded operands {m}x{n}x{k} W.t()={bview}")
    case = wl.gemm_case(m, n, k, seed=1400 + int(bview), b_transposed_view=bview, out_dtype=torch.bfloat16)
    a_buf = torch.zeros(m, kp + 5, dtype=torch.int32)
    a_buf[:, :kp] = case.a
    a = a_buf.to(gpu)[:, :kp]
    if bview:
        w_buf = torch.zeros(n, kp + 3, dtype=torch.int32)
        w_buf[:, :kp] = case.b.t()
        b = w_buf.to(gpu)[:, :kp].t()
    else:
        b_buf = torch.zeros(kp, n + 7, dtype=torch.int32)
        b_buf[:, :n] = case.b
        b = b_buf.to(gpu)[:, :n]
    out_buf = torch.full((m, n + 9), 7.0, dtype=torch.bfloat16, device=gpu)
    out = out_buf[:, :n]
    capi.int4_gemm(a, b, case.scale_a.to(gpu), case.scale_b.to(gpu), out_dtype=torch.bfloat16, out=out,
                   workspace=True)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), _ref(case, case.scale_a, case.scale_b, torch.bfloat16))
    assert bool((out_buf[:, n:] == 7.0).all())


def test_route_switch(gpu, routing):
    m, n, k = 1024, 512, 512
    assert capi.gemm_workspace_size(m, n, k) > 0
    assert capi.gemm_workspace_size(m, n, k, torch.float32) == 0
    assert capi.gemm_workspace_size(256, n, k) == 0
    routing.on("GEMM_NO_F6")
    assert capi.gemm_workspace_size(m, n, k) == 0
    case = wl.gemm_case(m, n, k, seed=500)
    ws = torch.empty(capi.f6_workspace_bytes(m, n, k), dtype=torch.uint8, device=gpu)
    out = capi.int4_gemm(case.a.to(gpu), case.b.to(gpu), case.scale_a.to(gpu), case.scale_b.to(gpu), workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), _ref(case, case.scale_a, case.scale_b, torch.float16))


def test_torch_operator_takes_the_route(gpu):
    """quant_ops' int4_matmul (the torch operator) allocates the workspace itself."""
    import quant_ops

    m, n, k = 2048, 2048, 1024
    case = wl.gemm_case(m, n, k, seed=600)
    out = quant_ops.int4_matmul(case.a.to(gpu), case.b.to(gpu), case.scale_a.to(gpu), case.scale_b.to(gpu))
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), _ref(case, case.scale_a, case.scale_b, torch.float16))


def test_graph_replay(gpu):
    """Both launches captured in a HIP graph, replayed with eager work between the replays."""
    m, n, k = 1024, 896, 1024
    case = wl.gemm_case(m, n, k, seed=700, b_transposed_view=True)
    a, b, sa, sb = case.a.to(gpu), case.b.to(gpu), case.scale_a.to(gpu), case.scale_b.to(gpu)
    ws = torch.empty(capi.gemm_workspace_size(m, n, k), dtype=torch.uint8, device=gpu)
    out = torch.empty(m, n, dtype=torch.float16, device=gpu)
    ref = _ref(case, case.scale_a, case.scale_b, torch.float16)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        capi.int4_gemm(a, b, sa, sb, out=out, workspace=ws, stream=s)
        s.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            capi.int4_gemm(a, b, sa, sb, out=out, workspace=ws, stream=s)
    for r in range(3):
        out.zero_()
        ws.fill_(r + 1)                                       # eager work on the workspace between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.cpu(), ref), f"replay {r}"


@pytest.mark.parametrize("tokens,out_f", [(300, 272), (1024, 4096)])
def test_linear_workspace_entry_point(gpu, tokens, out_f):
    """qo_w4a4_linear_ws (the GEMM on the FP6 route above 256 tokens) equals
    qo_w4a4_linear bit for bit, and its GEMM output equals the oracle's
    product of the codes the call returned."""
    from test_gpu_parity import _linear_inputs, _linear_ref

    m, n, dtype = 112, 128, torch.bfloat16
    x, L, R, w, sw, bias = _linear_inputs(tokens, m, n, out_f, dtype, 900 + tokens)
    args = (x.to(gpu), L.to(gpu), R.to(gpu), w.to(gpu), sw.to(gpu), 0.9, bias.to(gpu))
    _say(f"linear ws T={tokens} {m}x{n} -> {out_f}")
    assert capi.gemm_workspace_size(tokens, out_f, m * n, dtype) > 0
    y_ws, q_ws, s_ws = capi.w4a4_linear(*args, workspace=True)
    y, q, s = capi.w4a4_linear(*args)
    torch.cuda.synchronize()
    assert torch.equal(q_ws, q) and torch.equal(s_ws, s)
    assert torch.equal(y_ws, y)
    assert torch.equal(y_ws.cpu(), _linear_ref(q_ws.cpu(), s_ws.cpu(), w, sw, bias, dtype))


def test_linear_torch_operator_large_tokens(gpu):
    """The torch operator w4a4_linear passes a workspace: at 512 tokens its
    output equals the entry point without one."""
    m, n, out_f, dtype = 64, 128, 1024, torch.float16
    from test_gpu_parity import _linear_inputs

    x, L, R, w, sw, bias = _linear_inputs(512, m, n, out_f, dtype, 950)
    args = (x.to(gpu), L.to(gpu), R.to(gpu), w.to(gpu), sw.to(gpu))
    y_op = torch.ops.quant_ops.w4a4_linear(*args, 0.9, bias.to(gpu))
    y, _, _ = capi.w4a4_linear(*args, 0.9, bias.to(gpu))
    torch.cuda.synchronize()
    assert torch.equal(y_op, y)


@pytest.mark.parametrize("tokens,m,n,out_f,dtype", [(300, 112, 128, 272, torch.bfloat16), (1024, 64, 128, 1000,
                                                   torch.float16), (40, 112, 128, 512, torch.bfloat16)])
def test_linear_prepared_f6_weight(gpu, tokens, m, n, out_f, dtype):
    """qo_w4a4_linear_f6w against a weight converted once (qo_int4_gemm_f6_convert)
    equals qo_w4a4_linear bit for bit (outputs, codes, scales); the same
    converted weight serves two calls."""
    from test_gpu_parity import _linear_inputs

    _say(f"linear f6w T={tokens} {m}x{n} -> {out_f} {dtype}")
    x, L, R, w, sw, bias = _linear_inputs(tokens, m, n, out_f, dtype, 1200 + tokens)
    Ld, Rd, wd, swd, bd = L.to(gpu), R.to(gpu), w.to(gpu), sw.to(gpu), bias.to(gpu)
    w6 = capi.f6_convert(wd, m * n)
    for rep in range(2):
        xd = x.to(gpu) if rep == 0 else (x * 0.5).to(dtype).to(gpu)
        y6, q6, s6 = capi.w4a4_linear_f6w(xd, Ld, Rd, w6, out_f, swd, 0.9, bd)
        y, q, s = capi.w4a4_linear(xd, Ld, Rd, wd, swd, 0.9, bd)
        torch.cuda.synchronize()
        assert torch.equal(q6, q) and torch.equal(s6, s), f"call {rep}"
        assert torch.equal(y6, y), f"call {rep}"


def test_operand_convert_and_run2_match_workspace_route(gpu):
    """qo_int4_gemm_f6_convert of A and of a row-major [K/8, N] B, then
    qo_int4_gemm_f6_run2, equals qo_int4_gemm_ws; the error paths reject
    short buffers."""
    m, n, k = 640, 700, 1152
    case = wl.gemm_case(m, n, k, seed=1300)
    a, b, sa, sb = case.a.to(gpu), case.b.to(gpu), case.scale_a.to(gpu), case.scale_b.to(gpu)
    a6 = capi.f6_convert(a, k)
    b6 = capi.f6_convert(b, k, rows_are_columns=True)
    out = torch.empty(m, n, dtype=torch.float16, device=gpu)
    capi._check(capi.lib().qo_int4_gemm_f6_run2(
        ctypes.c_void_p(a6.data_ptr()), a6.numel(), ctypes.c_void_p(b6.data_ptr()), b6.numel(),
        ctypes.c_void_p(sa.data_ptr()), capi.DTYPE_F16, ctypes.c_void_p(sb.data_ptr()), capi.DTYPE_F16, None,
        ctypes.c_void_p(out.data_ptr()), capi.DTYPE_F16, n, m, n, k,
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    ref = capi.int4_gemm(a, b, sa, sb, workspace=True)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    st = capi.lib().qo_int4_gemm_f6_run2(
        ctypes.c_void_p(a6.data_ptr()), a6.numel() - 1, ctypes.c_void_p(b6.data_ptr()), b6.numel(),
        ctypes.c_void_p(sa.data_ptr()), capi.DTYPE_F16, ctypes.c_void_p(sb.data_ptr()), capi.DTYPE_F16, None,
        ctypes.c_void_p(out.data_ptr()), capi.DTYPE_F16, n, m, n, k, None)
    assert st != 0
    b6_off = torch.empty(b6.numel() + 256, dtype=torch.uint8, device=gpu)[16:]   # 16 bytes past 256
    st = capi.lib().qo_int4_gemm_f6_run2(
        ctypes.c_void_p(a6.data_ptr()), a6.numel(), ctypes.c_void_p(b6_off.data_ptr()), b6.numel(),
        ctypes.c_void_p(sa.data_ptr()), capi.DTYPE_F16, ctypes.c_void_p(sb.data_ptr()), capi.DTYPE_F16, None,
        ctypes.c_void_p(out.data_ptr()), capi.DTYPE_F16, n, m, n, k, None)
    assert st != 0 and "256-byte aligned" in capi.lib().qo_last_error().decode()
    with pytest.raises(capi.QuantOpsError):
        capi.f6_convert(a, k, out=torch.empty(16, dtype=torch.uint8, device=gpu))
