#!/usr/bin/env python3
"""Benchmark of the FlatQuant W4A4 hot path on one MI355X.

Prints ONE JSON line. The primary workload (``value``) is BASELINE config 2:
the fused quantize of fp16 X [2048, 4096] with 64 x 64 orthogonal transforms,
clip 0.9, packed int32 codes — one "step" is one quantize call over that batch.
``value`` is algorithmic HBM bytes (X in + codes out + fp32 scales + L, R) per
second over exactly ``--steps`` back-to-back steps (a captured HIP graph,
inputs already in HBM, rotated over enough buffers to exceed the 256 MB MALL),
timed with HIP events on the stream the kernels run on.

Secondary objects carry the W4A4 GEMM (config 4, TOPS vs the int8 MFMA peak),
the wide quantize (config 3) and the end-to-end W4A4 linear (config 5).
``cpu_baseline`` times this repo's CPU restatement of the reference PyTorch
fallback on a bounded sample on the host cores (a reported baseline, not a target).

Usage: python bench.py [--gpus 1] [--steps 100] [--warmup 10] [--warm-s 0.2] [--no-secondary] [--no-cpu]
       python bench.py --pmc-pass                       (under rocprofv3 --pmc FETCH_SIZE or WRITE_SIZE)
       python bench.py --pmc-summary FETCH_DIR WRITE_DIR
       python bench.py --pmc-table PMC_DIR [PMC_DIR ...]
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
MALL_BYTES = 256 * 2**20
METRIC = "quantize GB/s + W4A4 GEMM TOPS on 1 MI355X; % of HBM / i8-MFMA roofline"
ROOT = os.path.dirname(os.path.abspath(__file__))


def _log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _nbuf(bytes_per_set, minimum=2):
    return max(minimum, math.ceil(1.25 * MALL_BYTES / max(1, bytes_per_set)))


WARM_S = 0.2   # minimum untimed warm-up per measurement


def _time_graph(torch, launch, steps, warmup):
    """Warm up, capture ``steps`` launches in one graph, replay it once timed.

    Warm-up: ``warmup`` eager launches, then untimed replays of the same graph
    for at least WARM_S seconds. Replaying the timed graph itself touches every
    rotated buffer in the timed order before the timed replay (a shorter
    warm-up graph left the last buffers' first touch inside the timed
    replay), and the time floor covers the clock ramp of a GPU that has been
    idle. Returns (gpu_ms_total, wall_s_total) of the timed replay.
    ``launch(i)`` issues step i on the current stream.
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
    return start.elapsed_time(end), wall


def bench_quant(torch, case, steps, warmup, dev):
    from quant_ops_amd import capi

    t, f = case.x.shape
    per_set = case.algorithmic_bytes()
    nbuf = _nbuf(per_set)
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
        "TFLOPs": case.flops() / per_step_s / 1e12, "wall_s": wall,
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": gbs / HBM_PEAK_GBS},
    }
    del xs, codes, scales
    torch.cuda.empty_cache()
    return out


def bench_gemm(torch, case, steps, warmup, dev):
    from quant_ops_amd import capi

    m, n, k = case.mnk
    per_set = case.algorithmic_bytes()
    nbuf = _nbuf(per_set)
    a0, b0 = case.a.to(dev), case.b.to(dev)
    As = [a0] + [a0.clone() for _ in range(nbuf - 1)]
    Bs = [b0] + [b0.clone() for _ in range(nbuf - 1)] if b0.is_contiguous() else \
        [b0] + [b0.t().clone().t() for _ in range(nbuf - 1)]
    sa, sb = case.scale_a.to(dev), case.scale_b.to(dev)
    outs = [torch.empty((m, n), dtype=case.out_dtype, device=dev) for _ in range(nbuf)]

    def launch(i):
        j = i % nbuf
        capi.int4_gemm(As[j], Bs[j], sa, sb, out=outs[j])

    gpu_ms, wall = _time_graph(torch, launch, steps, warmup)
    per_step_s = gpu_ms / 1e3 / steps
    tops = case.ops() / per_step_s / 1e12
    out = {
        "workload": case.name, "M": m, "N": n, "K": k, "b_layout": "KN" if b0.is_contiguous() else "W.t()",
        "out_dtype": str(case.out_dtype).replace("torch.", ""), "ops_per_step": case.ops(),
        "bytes_per_step": per_set, "buffers_rotated": nbuf, "us_per_step": per_step_s * 1e6, "TOPS": tops,
        "GBps": per_set / per_step_s / 1e9, "wall_s": wall,
        "roofline": {"bound": "mfma", "achieved": tops, "peak": INT8_PEAK_TOPS, "unit": "TOP/s",
                     "frac": tops / INT8_PEAK_TOPS},
    }
    del As, Bs, outs
    torch.cuda.empty_cache()
    return out


def bench_linear(torch, tokens, steps, warmup, dev):
    """Config 5: bf16 X [T, 14336] -> quantize (112 x 128, clip 0.9) -> GEMM vs W.t() -> bf16 [T, 4096]."""
    from quant_ops_amd import capi
    from quant_ops_amd import workloads as wl

    x = wl.activations(tokens, 14336, torch.bfloat16, seed=21, outlier_frac=0.005, outlier_scale=30.0).to(dev)
    L, R = wl.orthogonal(112, 22, torch.bfloat16).to(dev), wl.orthogonal(128, 23, torch.bfloat16).to(dev)
    w = wl.random_packed(4096, 1792, 24).to(dev)
    sw = wl.uniform(4096, 0.001, 0.01, 25).to(dev)
    codes = torch.empty(tokens, 1792, dtype=torch.int32, device=dev)
    scales = torch.empty(tokens, dtype=torch.float32, device=dev)
    out = torch.empty(tokens, 4096, dtype=torch.bfloat16, device=dev)

    def launch(i):
        capi.flatquant_quantize(x, L, R, 0.9, True, out_codes=codes, out_scales=scales)
        capi.int4_gemm(codes, w.t(), scales, sw, out=out)

    gpu_ms, wall = _time_graph(torch, launch, steps, warmup)
    per_step_s = gpu_ms / 1e3 / steps
    ops = 2 * tokens * 4096 * 14336
    return {"workload": f"cfg5_w4a4_linear_down_proj_T{tokens}", "tokens": tokens,
            "us_per_step": per_step_s * 1e6, "TOPS": ops / per_step_s / 1e12,
            "weight_GBps": 4096 * 1792 * 4 / per_step_s / 1e9, "note": "quantize + GEMM, L2/MALL-warm inputs"}


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
    nbuf = _nbuf(nbytes)
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
            "us_per_step": per_step_s * 1e6, "GBps": gbs, "buffers_rotated": nbuf,
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": gbs / HBM_PEAK_GBS}}


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
        nbuf = _nbuf(nbytes)
        srcs = [src0] + [src0.clone() for _ in range(nbuf - 1)]
        dsts = [torch.empty(out_shape, dtype=out_dtype, device=dev) for _ in range(nbuf)]

        def launch(i, fn=fn, srcs=srcs, dsts=dsts, nbuf=nbuf):
            fn(srcs[i % nbuf], dsts[i % nbuf])

        gpu_ms, _ = _time_graph(torch, launch, steps, warmup)
        per_step_s = gpu_ms / 1e3 / steps
        gbs = nbytes / per_step_s / 1e9
        res[name] = {"bytes_per_step": nbytes, "us_per_step": per_step_s * 1e6, "GBps": gbs, "buffers_rotated": nbuf,
                     "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                  "frac": gbs / HBM_PEAK_GBS}}
        del srcs, dsts
    del codes0, words0
    torch.cuda.empty_cache()
    return res


def cpu_baseline(torch, budget_s=12.0):
    """The oracle (CPU restatement of the reference fallback) on config 2, bounded in time."""
    from oracle import fq_reference as ofq
    from quant_ops_amd import workloads as wl

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    case = wl.quant_cfg2()
    ofq.flatquant_pytorch(case.x, case.left, case.right, case.clip_ratio, True)   # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        ofq.flatquant_pytorch(case.x, case.left, case.right, case.clip_ratio, True)
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    cpu_model = ""
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"value": case.algorithmic_bytes() / med / 1e9, "unit": "GB/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"config 2 in full ([2048, 4096] fp16, packed), median of {len(times)} runs of the "
                      f"oracle's torch-CPU fallback restatement ({med * 1e3:.1f} ms each); cpu: {cpu_model}; "
                      f"torch {torch.__version__}"}


def cpu_baseline_gemm(torch, budget_s=8.0):
    """The oracle GEMM (unpack + float32 matmul + scales) on a 128-row slab of config 4."""
    from oracle import int4_reference as oi4
    from quant_ops_amd import workloads as wl

    case = wl.gemm_case(128, 14336, 4096, seed=0)
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 2:
        t0 = time.perf_counter()
        oi4.int4_matmul_pytorch(case.a, case.b, case.scale_a, case.scale_b)
        times.append(time.perf_counter() - t0)
    med = sorted(times)[len(times) // 2]
    return {"value": case.ops() / med / 1e12, "unit": "TOP/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"128 x 14336 x 4096 slab of config 4, median of {len(times)} runs ({med:.2f} s each)"}


# Kernel of each benched workload, as rocprofv3 names it (a substring of the demangled name).
KERNEL_OF = {
    "quantize_cfg2": "fq_wave_kernel<qo::F16T, 4, 2, true>",
    "quantize_cfg3": "fq_duo_kernel<qo::BF16T, 7, true>",
    "gemm_cfg4": "gemm_i4_pp<256, 224, 4, 2, 4, false, qo::OutF16>",
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
    case = wl.gemm_cfg4()
    a, b = case.a.to(dev), case.b.to(dev)
    sa, sb = case.scale_a.to(dev), case.scale_b.to(dev)
    for _ in range(4):
        out = torch.empty(case.mnk[:2], dtype=case.out_dtype, device=dev)
        capi.int4_gemm(a.clone(), b.clone(), sa, sb, out=out)
        torch.cuda.synchronize()
    del a, b, out
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
    print(f"{'counter':34s} " + " ".join(f"{n:>14s}" for n in names))
    for c in counters:
        cells = []
        for n in names:
            hits = [v for (cc, kn, _), v in vals.items() if cc == c and KERNEL_OF[n] in kn]
            cells.append(f"{statistics.median(hits):14.4g}" if hits else f"{'-':>14s}")
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


# Workloads in the order the default bench run dispatches them (one segment of
# launches each; the config 5 linear interleaves its two kernels).
BENCH_SEGMENTS = [
    ("quantize cfg2", 20996096, None), ("gemm cfg4", None, 481036337152), ("quantize cfg3", 293691904, None),
    ("cfg5 T=16 quantize", 16 * 14336 * 2 + 16 * 1792 * 4 + 16 * 4 + 2 * (112 * 112 + 128 * 128), None),
    ("cfg5 T=16 gemm", None, 2 * 16 * 4096 * 14336),
    ("cfg5 T=4096 quantize", 4096 * 14336 * 2 + 4096 * 1792 * 4 + 4096 * 4 + 2 * (112 * 112 + 128 * 128), None),
    ("cfg5 T=4096 gemm", None, 2 * 4096 * 4096 * 14336),
    ("pack cfg4 weight", 14336 * 4096 + 14336 * 512 * 4, None),
    ("unpack cfg4 weight", 14336 * 4096 + 14336 * 512 * 4, None),
    ("transpose cfg4 weight", 2 * 14336 * 512 * 4, None),
    ("dequantize cfg2 codes", 2048 * 4096 // 2 + 2048 * 4 + 2048 * 4096 * 4, None),
]


def trace_summary(trace_csv, tail=None):
    """Per-workload kernel durations from a rocprofv3 --kernel-trace CSV of a default bench run.

    Dispatches of this library's kernels are split into segments (a new segment
    starts when a kernel reappears after more than 16 other dispatches) and the
    segments, in dispatch order, are matched to BENCH_SEGMENTS. With ``tail``,
    only the last ``tail`` dispatches of each segment count (the timed steps;
    the warm-up replays come first).
    """
    import csv
    import statistics

    rows = [r for r in csv.DictReader(open(trace_csv)) if "qo::" in r["Kernel_Name"]]
    rows.sort(key=lambda r: int(r["Dispatch_Id"]))
    segs, last = [], {}
    for r in rows:
        key = (r["Kernel_Name"], r["Grid_Size_X"], r["Workgroup_Size_X"])
        did = int(r["Dispatch_Id"])
        if key not in last or did - last[key][0] > 16:
            seg = {"key": key, "first": did, "dur": []}
            segs.append(seg)
            last[key] = (did, seg)
        seg = last[key][1]
        last[key] = (did, seg)
        seg["dur"].append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    segs.sort(key=lambda s: s["first"])
    labelled = len(segs) == len(BENCH_SEGMENTS)
    lines = [f"{'workload':22s} {'calls':>5s} {'avg_us':>9s} {'median_us':>9s} {'min_us':>9s} {'max_us':>9s} "
             f"{'GB/s':>7s} {'TOP/s':>7s}  kernel [grid x block]"]
    for i, s in enumerate(segs):
        d = s["dur"][-tail:] if tail else s["dur"]
        avg = sum(d) / len(d) / 1e3
        name, nbytes, ops = BENCH_SEGMENTS[i] if labelled else (f"segment {i}", None, None)
        gbs = f"{nbytes / avg / 1e3:7.0f}" if nbytes else f"{'':7s}"
        tops = f"{ops / avg / 1e6:7.0f}" if ops else f"{'':7s}"
        kname = s["key"][0].split("(")[0].replace("void ", "")
        lines.append(f"{name:22s} {len(d):5d} {avg:9.2f} {statistics.median(d) / 1e3:9.2f} {min(d) / 1e3:9.2f} "
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


def main():
    global WARM_S
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--warm-s", type=float, default=WARM_S,
                    help="minimum seconds of untimed warm-up replays per measurement (default %(default)s)")
    ap.add_argument("--no-secondary", action="store_true", help="only the primary workload")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
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

    _log("primary: config 2 quantize")
    primary = bench_quant(torch, wl.quant_cfg2(), args.steps, args.warmup, dev)
    primary["roofline"]["traffic"] = _traffic_from_profiles("quantize_cfg2")
    _log(f"config 2: {primary['us_per_step']:.2f} us/step, {primary['GBps']:.0f} GB/s")

    secondary = {}
    if not args.no_secondary:
        _log("secondary: config 4 GEMM")
        secondary["gemm_cfg4"] = bench_gemm(torch, wl.gemm_cfg4(), args.steps, args.warmup, dev)
        secondary["gemm_cfg4"]["roofline"]["traffic"] = _traffic_from_profiles("gemm_cfg4")
        _log(f"config 4: {secondary['gemm_cfg4']['us_per_step']:.1f} us/step, "
             f"{secondary['gemm_cfg4']['TOPS']:.0f} TOPS")
        _log("secondary: config 3 quantize")
        secondary["quantize_cfg3"] = bench_quant(torch, wl.quant_cfg3(), args.steps, args.warmup, dev)
        secondary["quantize_cfg3"]["roofline"]["traffic"] = _traffic_from_profiles("quantize_cfg3")
        _log(f"config 3: {secondary['quantize_cfg3']['us_per_step']:.1f} us/step, "
             f"{secondary['quantize_cfg3']['GBps']:.0f} GB/s")
        for t in (16, 4096):
            _log(f"secondary: config 5 linear T={t}")
            secondary[f"linear_cfg5_T{t}"] = bench_linear(torch, t, args.steps, args.warmup, dev)
        _log("secondary: weight layout kernels (config 4 weight)")
        secondary["layout_cfg4_weight"] = bench_layout(torch, args.steps, args.warmup, dev)
        _log("secondary: dequantize (config 2 codes)")
        secondary["dequant_cfg2"] = bench_dequant(torch, args.steps, args.warmup, dev)

    cpu = None
    if not args.no_cpu:
        _log("cpu baseline (oracle on host cores)")
        cpu = cpu_baseline(torch)
        if not args.no_secondary:
            secondary["gemm_cfg4"]["cpu_baseline"] = cpu_baseline_gemm(torch)

    line = {
        "metric": METRIC,
        "value": primary["GBps"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": primary["us_per_step"] / 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic: seeded N(0,1) activations with 1% of channels x20, orthogonal transforms from QR "
                "of seeded Gaussians",
        "config": {
            "workload": "BASELINE config 2: flatquant_dynamic_quantize fp16 X[2048,4096], M=N=64, "
                        "clip_ratio=0.9, pack_int32=True (one step = one quantize call)",
            "tokens": 2048, "features": 4096, "M": 64, "N": 64,
        },
        "roofline": primary["roofline"],
        "cpu_baseline": cpu,
        "primary": primary,
        "secondary": secondary,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
