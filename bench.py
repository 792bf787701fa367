#!/usr/bin/env python3
"""Benchmark of the FlatQuant W4A4 hot path on one MI355X.

Prints ONE JSON line. The headline (``value``) is BASELINE config 4, the W4A4
GEMM 4096 x 14336 x 4096 the north-star target names: int32-packed int4 codes
times int32-packed int4 codes, fp16 per-token and per-channel scales, fp16
output. One step is one GEMM call as the torch operator makes it (with a
workspace: the operands converted to exact FP6 e2m3 values, then the FP6
matrix-core GEMM; the int32 route of the same call is timed beside it);
``value`` is 2 M N K per step over the time of exactly ``--steps`` steps, and
the roofline is the FP6 GEMM kernel's own rate against the dense FP6 peak.

Every BASELINE config has an object in ``lines`` with its own ``roofline``
(achieved rate of the config's dominant kernel against the MI355X peak of its
bound) and ``cpu_baseline`` (this repo's CPU restatement of the reference
fallback, timed on the host cores on a bounded sample, in the same unit):

* ``gemm_cfg4`` (the headline), ``quantize_cfg2``, ``quantize_cfg3``;
* ``linear_cfg5_T16`` and ``linear_cfg5_T4096``: one call of the linear layer
  (qo_w4a4_linear: quantize, then the GEMM against W.t()) as the step, and
  each kernel timed alone; T = 16 is judged on the HBM rate of the GEMM, whose
  bytes are the 29.4 MB weight read;
* ``quantize_cfg1``: the fp32 CPU-plumbing config, with the round-trip errors
  of ``dequantize_int4`` for the CPU fallback and for the GPU kernel.

Beside them: ``copy_probe_cfg2_bytes`` (a plain elementwise copy moving config
2's byte count, the launch + streaming floor that quantize is compared with),
``layout_cfg4_weight`` and ``dequant_cfg2``.

Timing: inputs already in HBM. Each measurement captures ``--steps`` launches in
one HIP graph, replays it untimed (at least ``--warm-s`` seconds), then replays
it once between two HIP events recorded on the stream that launches it. Every
step has its own buffer set (inputs and outputs) while the sets fit in 48 GiB,
and there are always enough sets to exceed 1.25 x the 256 MB MALL, so a timed
step never finds its inputs left in the MALL by an earlier step.

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--warm-s 0.2] [--no-secondary] [--no-cpu]
       python bench.py --pmc-pass                       (under rocprofv3 --pmc FETCH_SIZE or WRITE_SIZE)
       python bench.py --pmc-summary FETCH_DIR WRITE_DIR
       python bench.py --pmc-table PMC_DIR [PMC_DIR ...]
       python bench.py --ceilings                       (MFMA rates, LDS-DMA and LDS reads, empty launch, streaming copy)
       python bench.py --power                          (board power and clock while each kernel loops)
       python bench.py --ceilings-summary KERNEL_TRACE_CSV
       python bench.py --trace-summary KERNEL_TRACE_CSV [--trace-last K]
                                                        (rocprofv3 --kernel-trace --output-format csv)
"""
import argparse
import json
import math
import os
import sys
import time

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
INT8_PEAK_TOPS = 5000.0        # MI355X dense int8 MFMA, TOP/s
FP6_PEAK_TOPS = 10100.0        # MI355X dense FP6 / FP4 MFMA, TFLOP/s
MALL_BYTES = 256 * 2**20
ROTATION_CAP_BYTES = 48 * 2**30
METRIC = "quantize GB/s + W4A4 GEMM TOPS on 1 MI355X; % of HBM / i8-MFMA roofline"
ROOT = os.path.dirname(os.path.abspath(__file__))

# config 5: Llama-3-8B down_proj, bf16 X [T, 14336] -> W [4096, 14336] packed, passed as W.t()
LIN_K, LIN_N, LIN_M, LIN_NT = 14336, 4096, 112, 128


def _log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _nsets(bytes_per_set, steps):
    """Buffer sets to rotate: one per step while they fit in ROTATION_CAP_BYTES,
    never fewer than 1.25 x the MALL's worth."""
    per = max(1, bytes_per_set)
    return max(2, math.ceil(1.25 * MALL_BYTES / per), min(steps, ROTATION_CAP_BYTES // per))


WARM_S = 0.2   # minimum untimed warm-up per measurement
MARKER_KERNEL = "FillFunctor<float>"   # ends every measurement in a kernel trace
_MARKER = []


def _marker(torch):
    """One float32 fill of a single element: a dispatch that separates measurements
    in a kernel trace (trace_summary starts new segments after it)."""
    if not _MARKER:
        _MARKER.append(torch.empty(1, dtype=torch.float32, device="cuda"))
    _MARKER[0].fill_(0.0)


def _time_graph(torch, launch, steps, warmup):
    """Warm up, capture ``steps`` launches in one graph, replay it once timed.

    Warm-up: ``warmup`` eager launches, then untimed replays of the same graph
    for at least WARM_S seconds (the time floor covers the clock ramp of a GPU
    that has been idle). Returns (gpu_ms_total, wall_s_total) of the timed
    replay. ``launch(i)`` issues step i on the current stream.
    """
    for i in range(warmup):
        launch(i)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(g, stream=stream):
            for i in range(steps):
                launch(i)
    torch.cuda.synchronize()
    deadline = time.perf_counter() + WARM_S
    while True:
        g.replay()
        torch.cuda.synchronize()
        if time.perf_counter() >= deadline:
            break
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    cur = torch.cuda.current_stream()
    t0 = time.perf_counter()
    start.record(cur)
    g.replay()
    end.record(cur)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    _marker(torch)
    return start.elapsed_time(end), wall


def _hbm(gbs):
    return {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS}


def _mfma(tops):
    return {"bound": "mfma", "achieved": tops, "peak": INT8_PEAK_TOPS, "unit": "TOP/s",
            "frac": tops / INT8_PEAK_TOPS}


def _mfma_f6(tops):
    """The FP6 route's GEMM kernel against the dense FP6 matrix-core peak (the
    format it computes in); the int8 peak fraction beside it for comparison."""
    return {"bound": "mfma", "achieved": tops, "peak": FP6_PEAK_TOPS, "unit": "TOP/s", "frac": tops / FP6_PEAK_TOPS,
            "format": "fp6 e2m3 (int4 codes / 8, exact), fp32 accumulation",
            "int8_peak": INT8_PEAK_TOPS, "frac_of_int8_peak": tops / INT8_PEAK_TOPS}


# --------------------------------------------------------------------------- GPU measurements

def bench_quant(torch, case, steps, warmup, dev):
    from quant_ops_amd import capi

    t, f = case.x.shape
    per_set = case.algorithmic_bytes()
    nbuf = _nsets(per_set, steps)
    x0 = case.x.to(dev)
    xs = [x0] + [x0.clone() for _ in range(nbuf - 1)]
    L, R = case.left.to(dev), case.right.to(dev)
    codes = [torch.empty((t, f // 8) if case.pack_int32 else (t, f),
                         dtype=torch.int32 if case.pack_int32 else torch.int8, device=dev) for _ in range(nbuf)]
    scales = [torch.empty(t, dtype=torch.float32, device=dev) for _ in range(nbuf)]

    def launch(i):
        j = i % nbuf
        capi.flatquant_quantize(xs[j], L, R, case.clip_ratio, case.pack_int32, out_codes=codes[j],
                                out_scales=scales[j])

    gpu_ms, wall = _time_graph(torch, launch, steps, warmup)
    per_step_s = gpu_ms / 1e3 / steps
    gbs = per_set / per_step_s / 1e9
    out = {
        "workload": case.name, "tokens": t, "features": f, "M": case.left.shape[0], "N": case.right.shape[0],
        "dtype": str(case.x.dtype).replace("torch.", ""), "clip_ratio": case.clip_ratio,
        "pack_int32": case.pack_int32, "bytes_per_step": per_set, "flops_per_step": case.flops(),
        "buffers_rotated": nbuf, "us_per_step": per_step_s * 1e6, "GBps": gbs,
        "TFLOPs": case.flops() / per_step_s / 1e12, "wall_s": wall, "roofline": _hbm(gbs),
    }
    del xs, codes, scales
    torch.cuda.empty_cache()
    return out


def bench_gemm(torch, case, steps, warmup, dev):
    """One step = one int4 GEMM call as the torch operator makes it: with a
    workspace, so that products of more than 256 rows take the FP6 route (the
    operand conversion, then the FP6 GEMM). Beside it, each of the two
    kernels timed alone (the GEMM on a converted workspace gives the
    roofline's kernel rate) and the integer route of the same call."""
    from quant_ops_amd import capi

    m, n, k = case.mnk
    per_set = case.algorithmic_bytes()
    nbuf = _nsets(per_set, steps)
    a0, b0 = case.a.to(dev), case.b.to(dev)
    As = [a0] + [a0.clone() for _ in range(nbuf - 1)]
    Bs = [b0] + [b0.clone() for _ in range(nbuf - 1)] if b0.is_contiguous() else \
        [b0] + [b0.t().clone().t() for _ in range(nbuf - 1)]
    sa, sb = case.scale_a.to(dev), case.scale_b.to(dev)
    outs = [torch.empty((m, n), dtype=case.out_dtype, device=dev) for _ in range(nbuf)]
    ws_bytes = capi.gemm_workspace_size(m, n, k, case.out_dtype)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev) if ws_bytes else None

    def launch(i):
        j = i % nbuf
        capi.int4_gemm(As[j], Bs[j], sa, sb, out=outs[j], workspace=ws)

    gpu_ms, wall = _time_graph(torch, launch, steps, warmup)
    per_step_s = gpu_ms / 1e3 / steps
    tops = case.ops() / per_step_s / 1e12
    out = {
        "workload": case.name, "M": m, "N": n, "K": k, "b_layout": "KN" if b0.is_contiguous() else "W.t()",
        "out_dtype": str(case.out_dtype).replace("torch.", ""), "route": "fp6" if ws_bytes else "int8",
        "ops_per_step": case.ops(), "bytes_per_step": per_set, "buffers_rotated": nbuf,
        "us_per_step": per_step_s * 1e6, "TOPS": tops, "GBps": per_set / per_step_s / 1e9, "wall_s": wall,
        "roofline": _mfma(tops),
    }
    if ws_bytes:
        def convert(i):
            capi.f6_prepare(ws, m, n, k, a=As[i % nbuf], b=Bs[i % nbuf])

        def f6_gemm(i):
            capi.f6_run(ws, m, n, k, sa, sb, out_dtype=case.out_dtype, out=outs[i % nbuf])

        def int8_route(i):
            capi.int4_gemm(As[i % nbuf], Bs[i % nbuf], sa, sb, out=outs[i % nbuf])

        ms_c, _ = _time_graph(torch, convert, steps, warmup)
        ms_g, _ = _time_graph(torch, f6_gemm, steps, warmup)      # on the last set's converted operands
        ms_i, _ = _time_graph(torch, int8_route, steps, warmup)
        t_c, t_g, t_i = (ms / 1e3 / steps for ms in (ms_c, ms_g, ms_i))
        conv_bytes = (m + n) * k // 2 + (m + n) * k * 3 // 4
        out.update({
            "convert_us": t_c * 1e6, "convert_bytes": conv_bytes, "convert_GBps": conv_bytes / t_c / 1e9,
            "f6_gemm_kernel_us": t_g * 1e6, "f6_gemm_kernel_TOPS": case.ops() / t_g / 1e12,
            "int8_route_us": t_i * 1e6, "int8_route_TOPS": case.ops() / t_i / 1e12,
            "roofline": _mfma_f6(case.ops() / t_g / 1e12),
        })
    del As, Bs, outs, ws
    torch.cuda.empty_cache()
    return out


def linear_inputs(torch, tokens):
    """Config 5's seeded inputs (host tensors): X, L, R, packed W [4096, 1792], its fp16 scales."""
    from quant_ops_amd import workloads as wl

    x = wl.activations(tokens, LIN_K, torch.bfloat16, seed=21, outlier_frac=0.005, outlier_scale=30.0)
    L, R = wl.orthogonal(LIN_M, 22, torch.bfloat16), wl.orthogonal(LIN_NT, 23, torch.bfloat16)
    w = wl.random_packed(LIN_N, LIN_K // 8, 24)
    sw = wl.uniform(LIN_N, 0.001, 0.01, 25)
    return x, L, R, w, sw


def bench_linear(torch, tokens, steps, warmup, dev):
    """Config 5 at ``tokens``: the step is one call of the linear layer's entry
    point (qo_w4a4_linear: quantize, then the GEMM against W.t() with bf16
    output), every buffer rotated (X, W, codes, scales, output); beside it
    each of the two kernels timed alone."""
    from quant_ops_amd import capi

    x_h, L_h, R_h, w_h, sw_h = linear_inputs(torch, tokens)
    L, R, sw = L_h.to(dev), R_h.to(dev), sw_h.to(dev)
    w_bytes = LIN_N * LIN_K // 2
    q_bytes = _lin_q_bytes(tokens)
    g_bytes = w_bytes + tokens * LIN_K // 2 + tokens * 4 + LIN_N * 2 + tokens * LIN_N * 2
    # one step from HBM: X, L, R in, codes and scales out, W and its scales in, output out
    s_bytes = q_bytes + w_bytes + LIN_N * 2 + tokens * LIN_N * 2
    per_set = tokens * LIN_K * 2 + w_bytes + tokens * LIN_K // 2 + tokens * 4 + tokens * LIN_N * 2
    nbuf = _nsets(per_set, steps)
    x0, w0 = x_h.to(dev), w_h.to(dev)
    xs = [x0] + [x0.clone() for _ in range(nbuf - 1)]
    ws = [w0] + [w0.clone() for _ in range(nbuf - 1)]
    codes = [torch.empty(tokens, LIN_K // 8, dtype=torch.int32, device=dev) for _ in range(nbuf)]
    scales = [torch.empty(tokens, dtype=torch.float32, device=dev) for _ in range(nbuf)]
    outs = [torch.empty(tokens, LIN_N, dtype=torch.bfloat16, device=dev) for _ in range(nbuf)]

    # the GEMM's workspace, as the torch operator passes it (FP6 route above 256 tokens)
    wsb = capi.gemm_workspace_size(tokens, LIN_N, LIN_K, torch.bfloat16)
    work = torch.empty(wsb, dtype=torch.uint8, device=dev) if wsb else None

    def quant(j):
        capi.flatquant_quantize(xs[j], L, R, 0.9, True, out_codes=codes[j], out_scales=scales[j])

    def gemm(j):
        capi.int4_gemm(codes[j], ws[j].t(), scales[j], sw, out=outs[j], workspace=work)

    def step(j):
        capi.w4a4_linear(xs[j], L, R, ws[j], sw, 0.9, out=outs[j], codes=codes[j], scales=scales[j],
                         workspace=work)

    for j in range(nbuf):      # codes of every set, for the GEMM timed alone
        quant(j)
    torch.cuda.synchronize()
    ms_q, _ = _time_graph(torch, lambda i: quant(i % nbuf), steps, warmup)
    ms_g, _ = _time_graph(torch, lambda i: gemm(i % nbuf), steps, warmup)
    f6 = {}
    if work is not None:      # the FP6 route's two launches timed apart
        ms_c, _ = _time_graph(torch, lambda i: capi.f6_prepare(work, tokens, LIN_N, LIN_K, a=codes[i % nbuf],
                                                                 b=ws[i % nbuf].t()), steps, warmup)
        ms_r, _ = _time_graph(torch, lambda i: capi.f6_run(work, tokens, LIN_N, LIN_K, scales[i % nbuf], sw,
                                                             out_dtype=torch.bfloat16, out=outs[i % nbuf]),
                              steps, warmup)
        f6 = {"convert_us": ms_c / steps * 1e3, "f6_gemm_kernel_us": ms_r / steps * 1e3}
    ms_s, wall = _time_graph(torch, lambda i: step(i % nbuf), steps, warmup)
    t_q, t_g, t_s = (ms / 1e3 / steps for ms in (ms_q, ms_g, ms_s))
    if work is not None:
        # the serving form of the same step: the weight converted to the FP6
        # layout once (outside the timed region), only the codes per call
        w6s = [capi.f6_convert(ws[j], LIN_K) for j in range(nbuf)]
        a_ws = torch.empty(capi.f6_operand_bytes(tokens, LIN_K), dtype=torch.uint8, device=dev)

        def step_f6w(j):
            capi.w4a4_linear_f6w(xs[j], L, R, w6s[j], LIN_N, sw, 0.9, out=outs[j], codes=codes[j], scales=scales[j],
                                 a_workspace=a_ws)

        ms_p, _ = _time_graph(torch, lambda i: step_f6w(i % nbuf), steps, warmup)
        f6["prepared_weight_us_per_step"] = ms_p / steps * 1e3
        del w6s, a_ws
    ops = 2 * tokens * LIN_N * LIN_K
    gemm_gbs = g_bytes / t_g / 1e9
    out = {
        "workload": f"cfg5_w4a4_linear_down_proj_T{tokens}", "tokens": tokens, "K": LIN_K, "N": LIN_N,
        "buffers_rotated": nbuf, "us_per_step": t_s * 1e6, "quantize_us": t_q * 1e6,
        "gemm_us": t_g * 1e6, "ops_per_step": ops, "TOPS": ops / t_s / 1e12, "gemm_TOPS": ops / t_g / 1e12,
        "step_bytes": s_bytes, "step_GBps": s_bytes / t_s / 1e9,
        "quantize_bytes": q_bytes, "quantize_GBps": q_bytes / t_q / 1e9,
        "gemm_bytes": g_bytes, "gemm_GBps": gemm_gbs, "weight_bytes": w_bytes,
        "weight_GBps_gemm": w_bytes / t_g / 1e9, "weight_GBps_step": w_bytes / t_s / 1e9, "wall_s": wall,
    }
    # the dominant kernel: the GEMM; at 16 tokens it is a weight stream (HBM), at 4096 MFMA work
    out["route"] = "fp6" if work is not None else "int8"
    out.update(f6)
    if f6:
        out["f6_gemm_kernel_TOPS"] = ops / (f6["f6_gemm_kernel_us"] * 1e-6) / 1e12
        out["roofline"] = _mfma_f6(out["f6_gemm_kernel_TOPS"])
    else:
        out["roofline"] = _hbm(gemm_gbs) if tokens <= 64 else _mfma(ops / t_g / 1e12)
    del xs, ws, codes, scales, outs
    torch.cuda.empty_cache()
    return out


def roundtrip_cfg1(torch, dev):
    """Config 1's round trip through the public API: quantize (int8 codes), then
    dequantize_int4, on the CPU fallback (use_cuda=False) and on the GPU kernels.

    Errors: ||Yhat - Y|| / ||Y|| with Y = the fallback's transformed X
    (flatquant/ops.py:99-103) and Yhat the dequantized codes, and
    ||L Yhat R^T - X|| / ||X|| (X recovered through the inverse of the
    orthogonal transforms; equal to the first up to rounding).
    """
    import quant_ops_amd as qo
    from quant_ops_amd import workloads as wl

    case = wl.quant_cfg1()
    t, f = case.x.shape
    m, n = case.left.shape[0], case.right.shape[0]
    x, L, R = case.x, case.left, case.right
    y = torch.matmul(L.T, torch.matmul(x.reshape(-1, m, n), R)).reshape(t, f)

    def errs(yhat):
        yhat = yhat.float().cpu()
        xhat = torch.matmul(L, torch.matmul(yhat.reshape(-1, m, n), R.T)).reshape(t, f)
        return {"rel_err_Y": float((yhat - y).norm() / y.norm()),
                "rel_err_X": float((xhat - x).norm() / x.norm())}

    q_c, s_c = qo.flatquant_dynamic_quantize(x, L, R, case.clip_ratio, False, use_cuda=False)
    cpu = errs(qo.dequantize_int4(q_c, s_c, False))
    q_g, s_g = qo.flatquant_dynamic_quantize(x.to(dev), L.to(dev), R.to(dev), case.clip_ratio, False)
    gpu = errs(qo.dequantize_int4(q_g, s_g, False))
    torch.cuda.synchronize()
    same = bool(torch.equal(q_g.cpu(), q_c) and torch.equal(s_g.cpu(), s_c.float()))
    return {"cpu_fallback": cpu, "gpu": gpu, "gpu_codes_and_scales_equal_cpu": same,
            "note": "Y = L^T X R per token (the fallback's transformed X), Yhat = dequantize_int4(codes, scales)"}


def bench_copy_probe(torch, steps, warmup, dev, nbytes=20996096):
    """A plain elementwise copy (torch.neg on fp16) reading and writing half of
    ``nbytes`` each: config 2's byte count through the simplest streaming kernel,
    in the same graph timing. Its rate is the floor the config 2 quantize is
    compared with (launch plus streaming at this size)."""
    n_el = nbytes // 4
    per_set = 4 * n_el
    nbuf = _nsets(per_set, steps)
    src0 = torch.randn(n_el, dtype=torch.float16, device=dev)
    srcs = [src0] + [src0.clone() for _ in range(nbuf - 1)]
    dsts = [torch.empty_like(src0) for _ in range(nbuf)]

    def launch(i):
        torch.neg(srcs[i % nbuf], out=dsts[i % nbuf])

    gpu_ms, _ = _time_graph(torch, launch, steps, warmup)
    per_step_s = gpu_ms / 1e3 / steps
    gbs = per_set / per_step_s / 1e9
    del srcs, dsts
    torch.cuda.empty_cache()
    return {"workload": "torch.neg fp16, 10.5 MB in + 10.5 MB out (config 2's 21.0 MB)", "bytes_per_step": per_set,
            "buffers_rotated": nbuf, "us_per_step": per_step_s * 1e6, "GBps": gbs, "roofline": _hbm(gbs)}


def bench_dequant(torch, steps, warmup, dev):
    """dequantize_int4 of config 2's output: packed int32 [2048, 512] codes + fp32
    scales -> fp32 [2048, 4096]. HBM-bound: 4 B of codes and 32 B of float32 per
    8 features, plus the scales."""
    from quant_ops_amd import capi

    t, f = 2048, 4096
    g = torch.Generator().manual_seed(52)
    codes0 = torch.randint(-2**31, 2**31, (t, f // 8), generator=g, dtype=torch.int64).to(torch.int32).to(dev)
    scales0 = torch.rand(t, generator=g).to(dev)
    nbytes = t * f // 2 + t * 4 + t * f * 4
    nbuf = _nsets(nbytes, steps)
    codes = [codes0] + [codes0.clone() for _ in range(nbuf - 1)]
    outs = [torch.empty(t, f, dtype=torch.float32, device=dev) for _ in range(nbuf)]

    def launch(i):
        capi.dequantize_int4(codes[i % nbuf], scales0, True, out=outs[i % nbuf])

    gpu_ms, _ = _time_graph(torch, launch, steps, warmup)
    per_step_s = gpu_ms / 1e3 / steps
    gbs = nbytes / per_step_s / 1e9
    del codes, outs
    torch.cuda.empty_cache()
    return {"workload": "dequantize_int4 packed [2048, 512] -> fp32 [2048, 4096]", "bytes_per_step": nbytes,
            "us_per_step": per_step_s * 1e6, "GBps": gbs, "buffers_rotated": nbuf, "roofline": _hbm(gbs)}


LAYOUT_ROWS, LAYOUT_K = 14336, 4096   # the config 4 weight W [N, K] as int8 codes


def bench_layout(torch, steps, warmup, dev):
    """Weight-prep kernels at the config 4 weight: pack int8 codes [14336, 4096] ->
    int32 [14336, 512], unpack it back, and transpose the packed words to the
    [K/8, N] = [512, 14336] layout. HBM-bound; bytes are input + output."""
    from quant_ops_amd import capi

    g = torch.Generator().manual_seed(51)
    codes0 = torch.randint(-8, 8, (LAYOUT_ROWS, LAYOUT_K), generator=g, dtype=torch.int8).to(dev)
    words0 = capi.pack_int4_to_int32(codes0)
    res = {}
    cases = (
        ("pack", codes0, lambda src, dst: capi.pack_int4_to_int32(src, out=dst), (LAYOUT_ROWS, LAYOUT_K // 8),
         torch.int32),
        ("unpack", words0, lambda src, dst: capi.unpack_int32_to_int4(src, out=dst), (LAYOUT_ROWS, LAYOUT_K),
         torch.int8),
        ("transpose", words0, lambda src, dst: capi.transpose_int32(src, out=dst), (LAYOUT_K // 8, LAYOUT_ROWS),
         torch.int32),
    )
    for name, src0, fn, out_shape, out_dtype in cases:
        nbytes = src0.numel() * src0.element_size() + math.prod(out_shape) * torch.empty((), dtype=out_dtype).element_size()
        nbuf = _nsets(nbytes, steps)
        srcs = [src0] + [src0.clone() for _ in range(nbuf - 1)]
        dsts = [torch.empty(out_shape, dtype=out_dtype, device=dev) for _ in range(nbuf)]

        def launch(i, fn=fn, srcs=srcs, dsts=dsts, nbuf=nbuf):
            fn(srcs[i % nbuf], dsts[i % nbuf])

        gpu_ms, _ = _time_graph(torch, launch, steps, warmup)
        per_step_s = gpu_ms / 1e3 / steps
        gbs = nbytes / per_step_s / 1e9
        res[name] = {"bytes_per_step": nbytes, "us_per_step": per_step_s * 1e6, "GBps": gbs, "buffers_rotated": nbuf,
                     "roofline": _hbm(gbs)}
        del srcs, dsts
    del codes0, words0
    torch.cuda.empty_cache()
    return res


# --------------------------------------------------------------------------- CPU baselines

def _cpu_model():
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _cpu_median(fn, budget_s, min_runs=3):
    """Median seconds of ``fn()`` after one warm-up call, over at least ``min_runs``
    runs and ``budget_s`` seconds."""
    fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < min_runs:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times)


def _cpu_line(torch, value, unit, sample, med, runs):
    return {"value": value, "unit": unit, "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"{sample}; median of {runs} runs ({med * 1e3:.1f} ms each) of the oracle's restatement of "
                      f"the reference's torch-CPU fallback; cpu: {_cpu_model()}; torch {torch.__version__}"}


def cpu_quant(torch, case, budget_s, sample):
    from oracle import fq_reference as ofq

    med, runs = _cpu_median(lambda: ofq.flatquant_pytorch(case.x, case.left, case.right, case.clip_ratio,
                                                          case.pack_int32), budget_s)
    return _cpu_line(torch, case.algorithmic_bytes() / med / 1e9, "GB/s", sample, med, runs)


def cpu_gemm_cfg4(torch, budget_s):
    """The oracle GEMM (unpack + float32 matmul + scales) on a 128-row slab of config 4."""
    from oracle import int4_reference as oi4
    from quant_ops_amd import workloads as wl

    case = wl.gemm_case(128, 14336, 4096, seed=0)
    med, runs = _cpu_median(lambda: oi4.int4_matmul_pytorch(case.a, case.b, case.scale_a, case.scale_b), budget_s,
                            min_runs=2)
    return _cpu_line(torch, case.ops() / med / 1e12, "TOP/s", "128 x 14336 x 4096 slab of config 4 (1/32 of its rows)",
                     med, runs)


def cpu_linear(torch, tokens, sample_tokens, budget_s):
    """Config 5's step on the CPU (fallback quantize, then the fallback GEMM against
    W.t()) on ``sample_tokens`` of the ``tokens``-token workload."""
    from oracle import fq_reference as ofq
    from oracle import int4_reference as oi4

    x, L, R, w, sw = linear_inputs(torch, sample_tokens)

    def step():
        q, s = ofq.flatquant_pytorch(x, L, R, 0.9, True)
        oi4.int4_matmul_pytorch(q, w.t(), s, sw)

    med, runs = _cpu_median(step, budget_s, min_runs=2)
    ops = 2 * sample_tokens * LIN_N * LIN_K
    what = "all 16 tokens" if sample_tokens == tokens else f"{sample_tokens} of its {tokens} tokens"
    return _cpu_line(torch, ops / med / 1e12, "TOP/s", f"config 5 step (quantize + GEMM, bf16 out) on {what}",
                     med, runs)


def cpu_dequant(torch, budget_s):
    from oracle import fq_reference as ofq

    t, f = 2048, 4096
    g = torch.Generator().manual_seed(52)
    codes = torch.randint(-2**31, 2**31, (t, f // 8), generator=g, dtype=torch.int64).to(torch.int32)
    scales = torch.rand(t, generator=g)
    med, runs = _cpu_median(lambda: ofq.dequantize_int4(codes, scales, True), budget_s)
    return _cpu_line(torch, (t * f // 2 + t * 4 + t * f * 4) / med / 1e9, "GB/s",
                     "config 2's packed codes in full", med, runs)


# --------------------------------------------------------------------------- profiling helpers

# Kernel of each benched workload, as rocprofv3 names it (a substring of the demangled name).
KERNEL_OF = {
    "gemm_cfg4": "gemm_f6_pp2<256, 224, qo::OutF16>",
    "convert_cfg4": "f6_convert_kernel",
    "quantize_cfg2": "fq_wave_kernel<qo::F16T, 4, 2, true>",
    "quantize_cfg3": "fq_few2_kernel<qo::BF16T, 7, true, true, true>",
    "gemm_cfg5_T16": "gemm_i4_skinny_nk",
    "gemm_cfg5_T4096": "gemm_f6_pp2<256, 256, qo::OutBF16>",
}
COPY_PROBE_BYTES = 1 << 30      # float32 negation of 1 GiB: reads and writes exactly this many bytes
COPY_PROBE_KERNEL = "neg_kernel"


def pmc_pass(torch, dev):
    """Eager launches for a rocprofv3 --pmc run (one counter block per run).

    Each benched kernel runs 4 times on fresh buffers, then a plain copy kernel
    of known size (float32 negation, 1 GiB in, 1 GiB out) runs 4 times: its
    counter readings give the scale from FETCH_SIZE / WRITE_SIZE to bytes.
    """
    from quant_ops_amd import capi
    from quant_ops_amd import workloads as wl

    case = wl.gemm_cfg4()
    a, b = case.a.to(dev), case.b.to(dev)
    sa, sb = case.scale_a.to(dev), case.scale_b.to(dev)
    for _ in range(4):
        out = torch.empty(case.mnk[:2], dtype=case.out_dtype, device=dev)
        capi.int4_gemm(a.clone(), b.clone(), sa, sb, out=out, workspace=True)
        torch.cuda.synchronize()
    del a, b, out
    for case in (wl.quant_cfg2(), wl.quant_cfg3()):
        t, f = case.x.shape
        x = case.x.to(dev)
        L, R = case.left.to(dev), case.right.to(dev)
        for _ in range(4):
            xi = x.clone()
            codes = torch.empty((t, f // 8), dtype=torch.int32, device=dev)
            scales = torch.empty(t, dtype=torch.float32, device=dev)
            capi.flatquant_quantize(xi, L, R, case.clip_ratio, True, out_codes=codes, out_scales=scales)
            torch.cuda.synchronize()
        del x, xi, codes, scales
    for tokens in (16, 4096):
        x_h, L_h, R_h, w_h, sw_h = linear_inputs(torch, tokens)
        L, R, sw = L_h.to(dev), R_h.to(dev), sw_h.to(dev)
        codes = torch.empty(tokens, LIN_K // 8, dtype=torch.int32, device=dev)
        scales = torch.empty(tokens, dtype=torch.float32, device=dev)
        capi.flatquant_quantize(x_h.to(dev), L, R, 0.9, True, out_codes=codes, out_scales=scales)
        w = w_h.to(dev)
        for _ in range(4):
            out = torch.empty(tokens, LIN_N, dtype=torch.bfloat16, device=dev)
            capi.int4_gemm(codes.clone(), w.clone().t(), scales, sw, out=out, workspace=True)
            torch.cuda.synchronize()
        del w, out, codes, scales
    src = torch.randn(COPY_PROBE_BYTES // 4, device=dev)
    dst = torch.empty_like(src)
    for _ in range(4):
        torch.neg(src, out=dst)
        torch.cuda.synchronize()
    print(json.dumps({"pmc_pass": True, "copy_probe_bytes": COPY_PROBE_BYTES, "kernels": KERNEL_OF}), flush=True)


def pmc_table(dirs):
    """Counter table of the benched kernels from rocprofv3 --pmc runs of --pmc-pass.

    For every counter found in the counter_collection CSVs under ``dirs``: the
    value per dispatch (rows of one dispatch summed), median over the dispatches
    of each kernel in KERNEL_OF.
    """
    import csv
    import glob
    import statistics

    vals = {}
    for root in dirs:
        for path in glob.glob(os.path.join(root, "**", "*counter_collection.csv"), recursive=True):
            with open(path, newline="") as fh:
                for row in csv.DictReader(fh):
                    key = (row["Counter_Name"], row["Kernel_Name"], row["Dispatch_Id"])
                    vals[key] = vals.get(key, 0.0) + float(row["Counter_Value"])
    counters = sorted({c for c, _, _ in vals})
    names = list(KERNEL_OF)
    print(f"{'counter':34s} " + " ".join(f"{n:>16s}" for n in names))
    for c in counters:
        cells = []
        for n in names:
            hits = [v for (cc, kn, _), v in vals.items() if cc == c and KERNEL_OF[n] in kn]
            cells.append(f"{statistics.median(hits):16.4g}" if hits else f"{'-':>16s}")
        print(f"{c:34s} " + " ".join(cells))


def pmc_summary(fetch_dir, write_dir):
    """Per-launch HBM bytes of each benched kernel from two rocprofv3 --pmc runs.

    Reads the counter_collection CSVs of a FETCH_SIZE run and a WRITE_SIZE run
    (KiB per dispatch), takes the median over dispatches of each kernel, and
    divides by what the same counter reads per byte for the copy probe.
    """
    import csv
    import glob
    import statistics

    def per_kernel(root, counter):
        vals = {}
        files = glob.glob(os.path.join(root, "**", "*counter_collection.csv"), recursive=True)
        if not files:
            raise SystemExit(f"no counter_collection.csv under {root}")
        for path in files:
            with open(path, newline="") as fh:
                for row in csv.DictReader(fh):
                    if row.get("Counter_Name") != counter:
                        continue
                    vals.setdefault((row["Kernel_Name"], row["Dispatch_Id"]), 0.0)
                    vals[(row["Kernel_Name"], row["Dispatch_Id"])] += float(row["Counter_Value"])
        by_name = {}
        for (name, _), v in vals.items():
            by_name.setdefault(name, []).append(v)
        return by_name

    def pick(by_name, key):
        hits = [v for name, v in by_name.items() if key in name]
        if not hits:
            return None
        return statistics.median([x for v in hits for x in v]) * 1024.0   # KiB -> bytes

    fetch, write = per_kernel(fetch_dir, "FETCH_SIZE"), per_kernel(write_dir, "WRITE_SIZE")
    f_copy, w_copy = pick(fetch, COPY_PROBE_KERNEL), pick(write, COPY_PROBE_KERNEL)
    if not f_copy or not w_copy:
        raise SystemExit("copy probe kernel not found in the counter files")
    ff, wf = f_copy / COPY_PROBE_BYTES, w_copy / COPY_PROBE_BYTES
    out = {"copy_probe": {"bytes": COPY_PROBE_BYTES, "fetch_factor": ff, "write_factor": wf}}
    for key, kname in KERNEL_OF.items():
        fb, wb = pick(fetch, kname), pick(write, kname)
        if fb is None or wb is None:
            continue
        out[key] = {"kernel": kname, "fetch_bytes_raw": fb, "write_bytes_raw": wb,
                    "fetch_bytes": fb / ff, "write_bytes": wb / wf, "hbm_bytes_per_launch": fb / ff + wb / wf}
    print(json.dumps(out, indent=1))


def _lin_q_bytes(t):
    return t * LIN_K * 2 + t * LIN_K // 2 + t * 4 + 2 * (LIN_M ** 2 + LIN_NT ** 2)


F6_CONVERT_BYTES_CFG4 = (4096 + 14336) * 4096 * 5 // 4   # int4 in, FP6 out
F6_CONVERT_BYTES_CFG5 = (4096 + 4096) * 14336 * 5 // 4

# Workloads in the order the default bench run dispatches them (one segment of
# launches each, in order of first dispatch; a config 5 step interleaves its
# two kernels, which then form one segment each).
BENCH_SEGMENTS = [
    ("gemm cfg4 step: convert", F6_CONVERT_BYTES_CFG4, None), ("gemm cfg4 step: f6 gemm", None, 481036337152),
    ("gemm cfg4 convert alone", F6_CONVERT_BYTES_CFG4, None), ("gemm cfg4 f6 gemm alone", None, 481036337152),
    ("gemm cfg4 int8 route", None, 481036337152), ("quantize cfg2", 20996096, None),
    ("copy probe cfg2 bytes", 20996096, None), ("quantize cfg3", 293691904, None),
    ("cfg5 T=16 quantize", _lin_q_bytes(16), None), ("cfg5 T=16 gemm", None, 2 * 16 * LIN_N * LIN_K),
    ("cfg5 T=16 step quant", _lin_q_bytes(16), None), ("cfg5 T=16 step gemm", None, 2 * 16 * LIN_N * LIN_K),
    ("cfg5 T=4096 quantize", _lin_q_bytes(4096), None),
    ("cfg5 T=4096 gemm: convert", F6_CONVERT_BYTES_CFG5, None), ("cfg5 T=4096 gemm: f6 gemm", None, 2 * 4096 * LIN_N * LIN_K),
    ("cfg5 T=4096 convert alone", F6_CONVERT_BYTES_CFG5, None),
    ("cfg5 T=4096 f6 gemm alone", None, 2 * 4096 * LIN_N * LIN_K),
    ("cfg5 T=4096 step quant", _lin_q_bytes(4096), None), ("cfg5 T=4096 step convert", F6_CONVERT_BYTES_CFG5, None),
    ("cfg5 T=4096 step f6 gemm", None, 2 * 4096 * LIN_N * LIN_K),
    # (the weight's one-time conversion has the A conversion's grid, so their
    # segment is dispatched first)
    ("cfg5 T=4096 f6w step convert A", 4096 * LIN_K * 5 // 4, None),
    ("cfg5 T=4096 f6w step quant", _lin_q_bytes(4096), None),
    ("cfg5 T=4096 f6w step f6 gemm", None, 2 * 4096 * LIN_N * LIN_K),
    ("quantize cfg1", 128 * 4096 * 4 + 128 * 4096 + 128 * 4 + 2 * 64 * 64 * 4, None),
    ("pack cfg4 weight", 14336 * 4096 + 14336 * 512 * 4, None),
    ("unpack cfg4 weight", 14336 * 4096 + 14336 * 512 * 4, None),
    ("transpose cfg4 weight", 2 * 14336 * 512 * 4, None),
    ("dequantize cfg2 codes", 2048 * 4096 // 2 + 2048 * 4 + 2048 * 4096 * 4, None),
]


def ceilings_summary(trace_csv):
    """Per-probe kernel durations from a rocprofv3 --kernel-trace CSV of
    ``bench.py --ceilings`` (the MFMA probe split by workgroup size: 512
    threads = two waves per SIMD, 256 = one)."""
    import csv
    from collections import defaultdict

    groups = defaultdict(list)
    for r in csv.DictReader(open(trace_csv)):
        name = r["Kernel_Name"]
        if "probe_" not in name:
            continue
        short = name.split("(anonymous namespace)::", 1)[-1].split("(")[0]
        groups[(short, int(r["Workgroup_Size_X"]), int(r["Grid_Size_X"]))].append(
            (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    print(f"{'probe':28s} {'block':>5s} {'grid':>9s} {'calls':>6s} {'avg_us':>9s} {'median_us':>9s}  rate")
    for (short, block, grid), v in sorted(groups.items(), key=lambda kv: (kv[0][0], -kv[0][1])):
        v.sort()
        avg, med = sum(v) / len(v), v[len(v) // 2]
        rate = ""
        if short.startswith("probe_mfma_i8"):
            waves = grid // 64   # the data probe's rows mix its zero and random runs; bench.py's log splits them
            rate = f"{2 * 16 * 16 * 64 * 8 * 4096 * waves / (med * 1e-6) / 1e12:.0f} TOP/s (median)"
        elif short.startswith("probe_mfma_f6"):
            waves = grid // 64   # rows mix the zero, int4-code and random-field runs; bench.py's log splits them
            rate = f"{2 * 16 * 16 * 128 * 8 * 4096 * waves / (med * 1e-6) / 1e12:.0f} TOP/s (median)"
        elif short.startswith("probe_lds_dma"):
            rate = "modes 1-3 in call order: copies, reads, four waves each"
        elif short.startswith("probe_stream"):
            rate = f"{2048 * 4096 * 2 * 5 / 4 / (med * 1e-6) / 1e9:.0f} GB/s (median)"
        print(f"{short:28s} {block:5d} {grid:9d} {len(v):6d} {avg:9.2f} {med:9.2f}  {rate}")


def trace_summary(trace_csv, tail=None):
    """Per-workload kernel durations from a rocprofv3 --kernel-trace CSV of a default bench run.

    Every measurement ends with one marker dispatch (MARKER_KERNEL). Between two
    markers, the dispatches of each of this library's kernels (and of the copy
    probe) form one segment; segments in order of first dispatch are matched to
    BENCH_SEGMENTS. With ``tail``, only the last ``tail`` dispatches of each
    segment count (the timed steps; the warm-up comes first) and segments with
    fewer dispatches (single eager calls outside the measurements) are left out.
    """
    import csv
    import statistics

    rows = sorted(csv.DictReader(open(trace_csv)), key=lambda r: int(r["Dispatch_Id"]))
    segs, cur, epoch = [], {}, 0
    for r in rows:
        name = r["Kernel_Name"]
        if MARKER_KERNEL in name:
            epoch += 1
            cur = {}
            continue
        if "qo::" not in name and COPY_PROBE_KERNEL not in name:
            continue
        key = (name, r["Grid_Size_X"], r["Workgroup_Size_X"])
        if key not in cur:
            cur[key] = {"key": key, "first": int(r["Dispatch_Id"]), "dur": []}
            segs.append(cur[key])
        cur[key]["dur"].append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    if tail:
        segs = [s for s in segs if len(s["dur"]) >= tail]
    segs.sort(key=lambda s: s["first"])
    labelled = len(segs) == len(BENCH_SEGMENTS)
    lines = [f"{'workload':24s} {'calls':>5s} {'avg_us':>9s} {'median_us':>9s} {'min_us':>9s} {'max_us':>9s} "
             f"{'GB/s':>7s} {'TOP/s':>7s}  kernel [grid x block]"]
    for i, s in enumerate(segs):
        d = s["dur"][-tail:] if tail else s["dur"]
        avg = sum(d) / len(d) / 1e3
        name, nbytes, ops = BENCH_SEGMENTS[i] if labelled else (f"segment {i}", None, None)
        gbs = f"{nbytes / avg / 1e3:7.0f}" if nbytes else f"{'':7s}"
        tops = f"{ops / avg / 1e6:7.0f}" if ops else f"{'':7s}"
        kname = s["key"][0].replace("(anonymous namespace)::", "").split("(")[0].replace("void ", "")[:110]
        lines.append(f"{name:24s} {len(d):5d} {avg:9.2f} {statistics.median(d) / 1e3:9.2f} {min(d) / 1e3:9.2f} "
                     f"{max(d) / 1e3:9.2f} {gbs} {tops}  {kname} [{s['key'][1]} x {s['key'][2]}]")
    print("\n".join(lines))


def _traffic_from_profiles(kernel_key):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE), if committed."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as fh:
            data = json.load(fh)
        entry = data.get(kernel_key)
        return None if entry is None else entry.get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


# --------------------------------------------------------------------------- ceilings

def _f6_probe_operands(torch, g, int4):
    """16 x 1024 FP6 fragments of 32 bytes (24 used): 32 six-bit fields per
    lane, either int4 codes as the FP6 route encodes them (sign in bit 5,
    |q| <= 8 below it) or random fields."""
    n = 16 * 1024
    if int4:
        q = torch.randint(-8, 8, (n, 32), generator=g)
        fields = torch.where(q < 0, 32, 0) | q.abs()
    else:
        fields = torch.randint(0, 64, (n, 32), generator=g)
    words = torch.zeros(n, 8, dtype=torch.int64)
    for j in range(32):
        bit = 6 * j
        w, o = divmod(bit, 32)
        words[:, w] |= (fields[:, j] << o) & 0xFFFFFFFF
        if o > 26:
            words[:, w + 1] |= fields[:, j] >> (32 - o)
    words = torch.where(words >= 2**31, words - 2**32, words)
    return words.to(torch.int32).reshape(-1)


def ceilings(torch, steps, warmup, dev):
    """Microbenchmarks of the ceilings the kernels are compared with
    (libquant_ops_probes.so): the int8 MFMA rate with 0-8 independent VALU
    instructions per MFMA (two waves per SIMD on every CU), the same on
    operands from memory and for the FP6 matrix cores, FP6 MFMAs beside LDS
    reads, LDS-DMA copies from L2 beside LDS reads, an empty kernel's launch
    in a graph, and a streaming kernel moving config 2's bytes (16.8 MB in,
    4.2 MB out). Each is timed like the workloads (graph of ``steps``
    launches, HIP events); one JSON line."""
    import ctypes

    lib = ctypes.CDLL(os.path.join(ROOT, "quant_ops_amd", "libquant_ops_probes.so"))
    c_vp, c_int, c_i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
    lib.qo_probe_mfma_i8.argtypes = [c_int, c_int, c_int, c_vp, c_vp, c_int]
    lib.qo_probe_empty.argtypes = [c_vp]
    lib.qo_probe_stream.argtypes = [c_vp, c_vp, c_i64, c_int, c_vp]
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    stream = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    out = {"cus": cus}
    sink = torch.empty(cus * 512, dtype=torch.int32, device=dev)
    iters = 4096
    for threads, key in ((512, "mfma_i8"), (256, "mfma_i8_one_wave_per_simd")):
        mfma = {}
        for kv in (0, 1, 2, 3, 4, 8):
            def launch(i, kv=kv, threads=threads):
                assert lib.qo_probe_mfma_i8(kv, cus, iters, ctypes.c_void_p(sink.data_ptr()), stream(), threads) == 0
            ms, _ = _time_graph(torch, launch, steps, warmup)
            ops = 2 * 16 * 16 * 64 * 8 * iters * (threads // 64) * cus   # per MFMA x MFMAs per wave x waves
            mfma[f"valu_per_mfma_{kv}"] = {"us_per_launch": ms / steps * 1e3, "TOPS": ops / (ms / steps * 1e-3) / 1e12}
            _log(f"ceiling: int8 MFMA, {threads // 256} wave(s) per SIMD, {kv} VALU per MFMA: "
                 f"{mfma[f'valu_per_mfma_{kv}']['TOPS']:.0f} TOP/s")
        out[key] = mfma

    # operands from memory: all-zero bytes, random bytes, random bytes with the
    # low nibble cleared (the GEMM's widened int4 codes, 16 q), and random bytes
    # with the high nibble cleared (offset codes q + 8 in 0 .. 15)
    lib.qo_probe_mfma_i8_data.argtypes = [c_int, c_int, c_int, c_vp, c_vp, c_vp, c_vp, c_int]
    cycles = torch.empty(cus * 8, dtype=torch.int64, device=dev)
    g = torch.Generator(device="cpu").manual_seed(5)
    rnd = torch.randint(-2**31, 2**31 - 1, (16 * 1024 * 4,), generator=g, dtype=torch.int64).to(torch.int32)
    srcs = {"zero": torch.zeros_like(rnd).to(dev), "random": rnd.to(dev),
            "widened_int4": (rnd & int(0xF0F0F0F0 - 2**32)).to(dev), "low_nibble": (rnd & 0x0F0F0F0F).to(dev)}
    data = {}
    for name, src in srcs.items():
        for kv in (0, 2, 4):
            def launch(i, kv=kv, src=src):
                assert lib.qo_probe_mfma_i8_data(kv, cus, iters, ctypes.c_void_p(src.data_ptr()),
                                                 ctypes.c_void_p(sink.data_ptr()), ctypes.c_void_p(cycles.data_ptr()),
                                                 stream(), 512) == 0
            ms, _ = _time_graph(torch, launch, steps, warmup)
            us = ms / steps * 1e3
            ops = 2 * 16 * 16 * 64 * 8 * iters * 8 * cus
            data[f"{name}_valu_per_mfma_{kv}"] = {"us_per_launch": us, "TOPS": ops / (us * 1e-6) / 1e12}
            _log(f"ceiling: int8 MFMA on {name} operands, two waves per SIMD, {kv} VALU per MFMA: "
                 f"{ops / (us * 1e-6) / 1e12:.0f} TOP/s")
    out["mfma_i8_operands_from_memory"] = data

    # the FP6 matrix cores on FP6 operands: zeros, int4 codes as the FP6 route
    # stores them (q / 8: sign-magnitude, 6-bit fields), random 6-bit fields
    lib.qo_probe_mfma_f6_data.argtypes = [c_int, c_int, c_int, c_vp, c_vp, c_vp, c_vp]
    fsink = torch.empty(cus * 512, dtype=torch.float32, device=dev)
    f6_srcs = {"zero": torch.zeros(16 * 1024 * 8, dtype=torch.int32, device=dev),
               "int4_codes": _f6_probe_operands(torch, g, True).to(dev),
               "random_fields": _f6_probe_operands(torch, g, False).to(dev)}
    f6 = {}
    for name, src in f6_srcs.items():
        for kv in (0, 2):
            def launch(i, kv=kv, src=src):
                assert lib.qo_probe_mfma_f6_data(kv, cus, iters, ctypes.c_void_p(src.data_ptr()),
                                                 ctypes.c_void_p(fsink.data_ptr()), ctypes.c_void_p(cycles.data_ptr()),
                                                 stream()) == 0
            ms, _ = _time_graph(torch, launch, steps, warmup)
            us = ms / steps * 1e3
            ops = 2 * 16 * 16 * 128 * 8 * iters * 8 * cus
            f6[f"{name}_valu_per_mfma_{kv}"] = {"us_per_launch": us, "TOPS": ops / (us * 1e-6) / 1e12}
            _log(f"ceiling: FP6 MFMA on {name} operands, two waves per SIMD, {kv} VALU per MFMA: "
                 f"{ops / (us * 1e-6) / 1e12:.0f} TOP/s")
    out["mfma_f6_operands_from_memory"] = f6

    # FP6 MFMAs on one wave per SIMD and 16-byte LDS reads on the other, apart and together
    lib.qo_probe_mfma_lds_overlap.argtypes = [c_int, c_int, c_int, c_vp, c_vp]
    ovl = {}
    for mode, name in ((1, "mfma_only"), (2, "lds_reads_only"), (3, "both")):
        def launch(i, mode=mode):
            assert lib.qo_probe_mfma_lds_overlap(mode, cus, iters, ctypes.c_void_p(fsink.data_ptr()), stream()) == 0
        ms, _ = _time_graph(torch, launch, steps, warmup)
        ovl[name] = ms / steps * 1e3
    ovl["both_over_longer"] = ovl["both"] / max(ovl["mfma_only"], ovl["lds_reads_only"])
    _log(f"ceiling: FP6 MFMA wave + LDS-read wave per SIMD: {ovl['mfma_only']:.0f} / {ovl['lds_reads_only']:.0f} us "
         f"apart, {ovl['both']:.0f} us together ({ovl['both_over_longer']:.2f} x the longer)")
    out["mfma_lds_overlap_us"] = ovl

    # LDS-DMA copies from L2 into LDS and 16-byte LDS reads per CU, apart and on four waves each
    lib.qo_probe_lds_dma.argtypes = [c_int, c_int, c_int, c_vp, c_vp, c_vp]
    dsrc = torch.randint(0, 255, (32 * 1024,), dtype=torch.uint8, device=dev, generator=None)
    dma_iters = 1024
    dma = {}
    for mode, name, copy_waves, read_waves in ((1, "copies_only", 8, 0), (2, "reads_only", 0, 8),
                                               (3, "four_waves_each", 4, 4)):
        def launch(i, mode=mode):
            assert lib.qo_probe_lds_dma(mode, cus, dma_iters, ctypes.c_void_p(dsrc.data_ptr()),
                                        ctypes.c_void_p(fsink.data_ptr()), stream()) == 0
        ms, _ = _time_graph(torch, launch, steps, warmup)
        us = ms / steps * 1e3
        # bytes per CU over the launch (both kinds end together only in the mixed mode's
        # slower half; the per-CU rates below take the whole launch)
        copy_b, read_b = copy_waves * dma_iters * 8 * 1024, read_waves * dma_iters * 16 * 1024
        dma[name] = {"us_per_launch": us, "copy_GBps_per_cu": copy_b / (us * 1e-6) / 1e9,
                     "read_GBps_per_cu": read_b / (us * 1e-6) / 1e9}
        _log(f"ceiling: LDS {name}: {us:.0f} us, per CU {dma[name]['copy_GBps_per_cu']:.0f} GB/s copied "
             f"from L2, {dma[name]['read_GBps_per_cu']:.0f} GB/s read")
    out["lds_dma_per_cu"] = dma

    def launch_empty(i):
        assert lib.qo_probe_empty(stream()) == 0
    ms, _ = _time_graph(torch, launch_empty, steps, warmup)
    out["empty_kernel_us"] = ms / steps * 1e3
    _log(f"ceiling: empty kernel {out['empty_kernel_us']:.2f} us per launch in a graph")

    bytes_in = 2048 * 4096 * 2
    nsets = _nsets(bytes_in * 5 // 4, steps)
    ins = [torch.empty(bytes_in // 4, dtype=torch.int32, device=dev).fill_(i) for i in range(nsets)]
    outs = [torch.empty(bytes_in // 16, dtype=torch.int32, device=dev) for _ in range(nsets)]
    stream_res = {}
    for blocks in (1024, 4096, 16384):
        def launch_stream(i, blocks=blocks):
            j = i % nsets
            assert lib.qo_probe_stream(ctypes.c_void_p(ins[j].data_ptr()), ctypes.c_void_p(outs[j].data_ptr()),
                                       bytes_in, blocks, stream()) == 0
        ms, _ = _time_graph(torch, launch_stream, steps, warmup)
        us = ms / steps * 1e3
        stream_res[f"blocks_{blocks}"] = {"us_per_launch": us, "GBps": bytes_in * 5 / 4 / (us * 1e-6) / 1e9}
        _log(f"ceiling: stream of config 2's bytes, {blocks} blocks: {us:.2f} us")
    out["stream_cfg2_bytes"] = stream_res
    print(json.dumps({"ceilings": out}), flush=True)


def _smi_sample():
    """(board power W, shader clock MHz) read by amd-smi and rocm-smi (child processes); None where absent."""
    import re
    import subprocess

    def run(cmd):
        try:
            return subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                                  timeout=20).stdout
        except (OSError, subprocess.SubprocessError):
            return ""
    pw = re.search(r"SOCKET_POWER:\s*([\d.]+)\s*W", run(["amd-smi", "metric", "-p"]))
    clk = re.search(r"sclk clock level:\s*\d+:\s*\((\d+)\s*Mhz\)", run(["rocm-smi", "--showclocks"]), re.I)
    return (float(pw.group(1)) if pw else None), (float(clk.group(1)) if clk else None)


def power(torch, dev, seconds=2.0):
    """Board power and shader clock while each workload runs back to back:
    the int8 MFMA probe on zero, widened-int4 and random operands, the FP6 MFMA
    probe on zero and int4-code operands, the config 4 and config 5 (T = 4096)
    GEMMs as the torch operator runs them and the config 2 and config 3
    quantizes. Each
    runs in a loop on a thread for ``seconds`` before three samples are taken
    (medians reported); one JSON line."""
    import ctypes
    import statistics
    import threading
    from quant_ops_amd import capi
    from quant_ops_amd import workloads as wl

    lib = ctypes.CDLL(os.path.join(ROOT, "quant_ops_amd", "libquant_ops_probes.so"))
    c_vp, c_int = ctypes.c_void_p, ctypes.c_int
    lib.qo_probe_mfma_i8_data.argtypes = [c_int, c_int, c_int, c_vp, c_vp, c_vp, c_vp, c_int]
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    sink = torch.empty(cus * 512, dtype=torch.int32, device=dev)
    cycles = torch.empty(cus * 8, dtype=torch.int64, device=dev)
    g = torch.Generator(device="cpu").manual_seed(5)
    rnd = torch.randint(-2**31, 2**31 - 1, (16 * 1024 * 4,), generator=g, dtype=torch.int64).to(torch.int32)
    srcs = {"zero": torch.zeros_like(rnd).to(dev), "widened_int4": (rnd & int(0xF0F0F0F0 - 2**32)).to(dev),
            "random": rnd.to(dev)}

    lib.qo_probe_mfma_f6_data.argtypes = [c_int, c_int, c_int, c_vp, c_vp, c_vp, c_vp]
    fsink = torch.empty(cus * 512, dtype=torch.float32, device=dev)
    f6_srcs = {"zero": torch.zeros(16 * 1024 * 8, dtype=torch.int32, device=dev),
               "int4_codes": _f6_probe_operands(torch, g, True).to(dev)}

    def probe_f6(src, kv):
        return lambda: lib.qo_probe_mfma_f6_data(kv, cus, 8192, ctypes.c_void_p(src.data_ptr()),
                                                 ctypes.c_void_p(fsink.data_ptr()),
                                                 ctypes.c_void_p(cycles.data_ptr()), None)

    def probe(src, kv):
        return lambda: lib.qo_probe_mfma_i8_data(kv, cus, 16384, ctypes.c_void_p(src.data_ptr()),
                                                 ctypes.c_void_p(sink.data_ptr()),
                                                 ctypes.c_void_p(cycles.data_ptr()), None, 512)

    def gemm(case):
        a, b, sa, sb = case.a.to(dev), case.b.to(dev), case.scale_a.to(dev), case.scale_b.to(dev)
        out = torch.empty(case.mnk[:2], dtype=case.out_dtype, device=dev)
        m, n, k = case.mnk
        ws = torch.empty(max(1, capi.gemm_workspace_size(m, n, k, case.out_dtype)), dtype=torch.uint8, device=dev)
        return lambda: capi.int4_gemm(a, b, sa, sb, out_dtype=case.out_dtype, out=out, workspace=ws)

    def quant(case):
        x, L, R = case.x.to(dev), case.left.to(dev), case.right.to(dev)
        return lambda: capi.flatquant_quantize(x, L, R, case.clip_ratio, case.pack_int32)

    work = [("idle", None)]
    for name in srcs:
        for kv in (0, 2):
            work.append((f"mfma_i8 probe, {name} operands, {kv} VALU per MFMA", probe(srcs[name], kv)))
    for name in f6_srcs:
        for kv in (0, 2):
            work.append((f"mfma_f6 probe, {name} operands, {kv} VALU per MFMA", probe_f6(f6_srcs[name], kv)))
    work += [("gemm cfg4 (FP6 route: conversion + FP6 GEMM)", gemm(wl.gemm_cfg4())),
             ("gemm cfg5 T=4096", gemm(wl.gemm_case(4096, 4096, 14336, seed=2, b_transposed_view=True,
                                                    out_dtype=torch.bfloat16))),
             ("quantize cfg3", quant(wl.quant_cfg3())), ("quantize cfg2", quant(wl.quant_cfg2()))]
    out = {}
    for name, fn in work:
        stop = []

        def loop():
            while not stop:
                for _ in range(20):
                    fn()
                torch.cuda.synchronize()
        th = threading.Thread(target=loop) if fn else None
        if th:
            th.start()
        time.sleep(seconds if th else 0.5)
        samples = [_smi_sample() for _ in range(3)]
        stop.append(True)
        if th:
            th.join()
        pw = [p for p, _ in samples if p is not None]
        ck = [c for _, c in samples if c is not None]
        out[name] = {"power_W": statistics.median(pw) if pw else None,
                     "sclk_MHz": statistics.median(ck) if ck else None}
        _log(f"power: {name}: {out[name]['power_W']} W, {out[name]['sclk_MHz']} MHz")
    print(json.dumps({"power": out}), flush=True)


# --------------------------------------------------------------------------- main

def main():
    global WARM_S
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--warm-s", type=float, default=WARM_S,
                    help="minimum seconds of untimed warm-up replays per measurement (default %(default)s)")
    ap.add_argument("--no-secondary", action="store_true", help="only the headline workload")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--pmc-pass", action="store_true",
                    help="eager launches of each benched kernel and a copy probe, for rocprofv3 --pmc")
    ap.add_argument("--trace-summary", metavar="KERNEL_TRACE_CSV",
                    help="per-workload kernel durations from a rocprofv3 kernel trace of a default run")
    ap.add_argument("--trace-last", type=int, default=None, metavar="K",
                    help="with --trace-summary: only the last K dispatches of each workload (the timed steps)")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="print per-launch HBM bytes from two rocprofv3 --pmc output folders")
    ap.add_argument("--pmc-table", nargs="+", metavar="PMC_DIR",
                    help="per-kernel medians of every counter in rocprofv3 --pmc output folders of --pmc-pass")
    ap.add_argument("--ceilings", action="store_true",
                    help="microbenchmarks of the int8 MFMA rate, an empty launch and a streaming copy")
    ap.add_argument("--power", action="store_true",
                    help="board power and shader clock (amd-smi, rocm-smi) while each benched kernel loops")
    ap.add_argument("--ceilings-summary", metavar="KERNEL_TRACE_CSV",
                    help="per-probe kernel durations from a rocprofv3 kernel trace of --ceilings")
    args = ap.parse_args()
    if args.pmc_summary:
        pmc_summary(*args.pmc_summary)
        return
    if args.pmc_table:
        pmc_table(args.pmc_table)
        return
    if args.trace_summary:
        trace_summary(args.trace_summary, args.trace_last)
        return
    if args.ceilings_summary:
        ceilings_summary(args.ceilings_summary)
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (the hot path shards over tokens with no "
              f"communication); --gpus {args.gpus} is not supported", file=sys.stderr)
        sys.exit(2)
    if args.steps < 1 or args.warmup < 0 or args.warm_s < 0:
        print("bench.py: --steps must be >= 1, --warmup and --warm-s >= 0", file=sys.stderr)
        sys.exit(2)
    WARM_S = args.warm_s

    import torch

    sys.path.insert(0, ROOT)
    import quant_ops_amd as qo
    from quant_ops_amd import workloads as wl

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    if not qo.CUDA_AVAILABLE:
        print(f"bench.py: HIP library not loaded: {qo._loader.LOAD_ERROR}", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda", 0)
    if args.pmc_pass:
        pmc_pass(torch, dev)
        return
    if args.ceilings:
        ceilings(torch, args.steps, args.warmup, dev)
        return
    if args.power:
        power(torch, dev)
        return
    steps, warmup = args.steps, args.warmup

    _log("headline: config 4 GEMM")
    head = bench_gemm(torch, wl.gemm_cfg4(), steps, warmup, dev)
    head["roofline"]["traffic"] = _traffic_from_profiles("gemm_cfg4")
    _log(f"config 4: {head['us_per_step']:.1f} us/step, {head['TOPS']:.0f} TOP/s"
         + (f" (convert {head['convert_us']:.1f} us, FP6 GEMM {head['f6_gemm_kernel_us']:.1f} us; "
            f"int32 route {head['int8_route_us']:.1f} us)" if head.get("route") == "fp6" else ""))
    lines = {"gemm_cfg4": head}
    if not args.no_secondary:
        _log("config 2 quantize")
        lines["quantize_cfg2"] = bench_quant(torch, wl.quant_cfg2(), steps, warmup, dev)
        lines["quantize_cfg2"]["roofline"]["traffic"] = _traffic_from_profiles("quantize_cfg2")
        lines["copy_probe_cfg2_bytes"] = bench_copy_probe(torch, steps, warmup, dev)
        _log(f"config 2: {lines['quantize_cfg2']['us_per_step']:.2f} us/step "
             f"(copy of the same bytes {lines['copy_probe_cfg2_bytes']['us_per_step']:.2f} us)")
        _log("config 3 quantize")
        lines["quantize_cfg3"] = bench_quant(torch, wl.quant_cfg3(), steps, warmup, dev)
        lines["quantize_cfg3"]["roofline"]["traffic"] = _traffic_from_profiles("quantize_cfg3")
        _log(f"config 3: {lines['quantize_cfg3']['us_per_step']:.1f} us/step")
        for t in (16, 4096):
            _log(f"config 5 linear T={t}")
            key = f"linear_cfg5_T{t}"
            lines[key] = bench_linear(torch, t, steps, warmup, dev)
            lines[key]["roofline"]["traffic"] = _traffic_from_profiles(f"gemm_cfg5_T{t}")
            _log(f"config 5 T={t}: {lines[key]['us_per_step']:.1f} us/step (quantize {lines[key]['quantize_us']:.1f}, "
                 f"GEMM {lines[key]['gemm_us']:.1f})"
                 + (f"; weight converted once: {lines[key]['prepared_weight_us_per_step']:.1f} us/step"
                    if "prepared_weight_us_per_step" in lines[key] else ""))
        _log("config 1 round trip + quantize")
        rt = roundtrip_cfg1(torch, dev)
        lines["quantize_cfg1"] = bench_quant(torch, wl.quant_cfg1(), steps, warmup, dev)
        lines["quantize_cfg1"]["round_trip"] = rt
        _log("weight layout kernels (config 4 weight)")
        lines["layout_cfg4_weight"] = bench_layout(torch, steps, warmup, dev)
        _log("dequantize (config 2 codes)")
        lines["dequant_cfg2"] = bench_dequant(torch, steps, warmup, dev)

    if not args.no_cpu:
        _log("cpu baselines (oracle on host cores)")
        torch.set_num_threads(len(os.sched_getaffinity(0)))
        head["cpu_baseline"] = cpu_gemm_cfg4(torch, 6.0)
        if not args.no_secondary:
            lines["quantize_cfg2"]["cpu_baseline"] = cpu_quant(torch, wl.quant_cfg2(), 5.0, "config 2 in full")
            lines["quantize_cfg3"]["cpu_baseline"] = cpu_quant(torch, wl.quant_cfg3(tokens=1024), 4.0,
                                                               "1024 of config 3's 8192 tokens")
            lines["linear_cfg5_T16"]["cpu_baseline"] = cpu_linear(torch, 16, 16, 4.0)
            lines["linear_cfg5_T4096"]["cpu_baseline"] = cpu_linear(torch, 4096, 128, 4.0)
            lines["quantize_cfg1"]["cpu_baseline"] = cpu_quant(torch, wl.quant_cfg1(), 2.0, "config 1 in full")
            lines["dequant_cfg2"]["cpu_baseline"] = cpu_dequant(torch, 2.0)

    line = {
        "metric": METRIC,
        "value": head["TOPS"],
        "unit": "TOP/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": head["us_per_step"] / 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp6",
        "data": "synthetic: seeded uniform int4 codes in [-8, 7] packed 8 per int32, fp16 scales U(0.01, 0.1) per "
                "token and U(0.001, 0.01) per channel; quantize lines: seeded N(0,1) activations with outlier "
                "channels, orthogonal transforms from QR of seeded Gaussians",
        "config": {
            "workload": "BASELINE config 4: int4_matmul A [4096, 4096/8] x B [4096/8, 14336] int32-packed int4, "
                        "fp16 out; one step = one GEMM call as the torch operator makes it: both operands "
                        "converted to FP6 e2m3 (q / 8, exact), then the f8f6f4 MFMA with fp32 accumulation "
                        "(exact integer sums, outputs bit-identical to the int32 path)",
            "M": 4096, "N": 14336, "K": 4096,
        },
        "roofline": head["roofline"],
        "cpu_baseline": head.get("cpu_baseline"),
        "lines": lines,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
