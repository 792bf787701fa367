"""Host-side behaviour of the drop-in API and the C ABI (no GPU needed)."""
import ctypes
import os
import re
import subprocess
import sys

import numpy as np
import pytest
import torch

import quant_ops_amd as qo
from quant_ops_amd import _loader, capi
from quant_ops_amd import workloads as wl
from oracle import fq_reference as ofq
from oracle import int4_reference as oi4

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_public_names_match_reference():
    # src/quant_ops/__init__.py:39-45
    assert set(qo.__all__) == {"flatquant_dynamic_quantize", "dequantize_int4", "int4_matmul",
                               "get_decompose_dim", "CUDA_AVAILABLE"}
    for name in ("flatquant_cuda", "flatquant_pytorch", "_FlatQuantCUDA", "int4_matmul_cuda",
                 "int4_matmul_pytorch", "pack_int4_to_int32", "unpack_int32_to_int4", "__version__"):
        assert hasattr(qo, name), name


def test_native_library_loaded_and_schemas_defined():
    assert _loader.KERNELS_AVAILABLE, _loader.LOAD_ERROR
    assert qo.CUDA_AVAILABLE
    ops = torch.ops.quant_ops
    assert str(ops.flatquant_dynamic_quantize.default._schema) == (
        "quant_ops::flatquant_dynamic_quantize(Tensor input, Tensor left_trans, Tensor right_trans, "
        "float clip_ratio=1., bool pack_int32=False) -> (Tensor, Tensor)")
    assert str(ops.int4_matmul.default._schema) == (
        "quant_ops::int4_matmul(Tensor a, Tensor b, Tensor scale_a, Tensor scale_b) -> Tensor")


def test_c_abi_exports_every_declared_symbol():
    header = open(os.path.join(ROOT, "include", "quant_ops_hip.h")).read()
    code = re.sub(r"/\*.*?\*/", "", header, flags=re.S)
    code = re.sub(r"//[^\n]*", "", code)
    declared = set(re.findall(r"\b(qo_[a-z0-9_]+)\s*\(", code))
    assert declared == set(capi.EXPORTED)
    out = subprocess.run(["nm", "-D", "--defined-only", _loader.HIP_LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert declared <= exported
    lib = capi.lib()
    for name in declared:
        assert getattr(lib, name) is not None


def test_c_abi_status_and_errors_without_gpu():
    lib = capi.lib()
    assert capi.version() == qo.__version__
    assert lib.qo_status_string(0) == b"ok"
    assert lib.qo_status_string(2) == b"invalid shape"
    # argument checks run before any device work, so they are testable here
    st = lib.qo_flatquant_quantize(None, 1, 4, 64, None, None, 8, 8, ctypes.c_float(1.0), 1, None, None, None)
    assert st == 1  # NULL pointer
    st = lib.qo_flatquant_quantize(None, 1, 4, 12, None, None, 3, 4, ctypes.c_float(1.0), 1, None, None, None)
    assert st == 2 and b"divisible by 8" in lib.qo_last_error()
    st = lib.qo_flatquant_quantize(None, 9, 4, 64, None, None, 8, 8, ctypes.c_float(1.0), 0, None, None, None)
    assert st in (1, 3)
    st = lib.qo_int4_gemm(None, 1, None, 1, 1, None, 0, None, 0, None, 1, 4, 4, 4, 12, None)
    assert st == 2 and b"multiple of 8" in lib.qo_last_error()
    st = lib.qo_int4_gemm(None, 1 << 18, None, 1, 1, None, 0, None, 0, None, 1, 4, 4, 4, 1 << 21, None)
    assert st == 2
    st = lib.qo_int4_gemm(None, 1, None, 1, 1, None, 7, None, 0, None, 1, 4, 4, 4, 8, None)
    assert st == 3
    st = lib.qo_dequantize_int4(None, 1, None, 0, 4, 12, None, None)
    assert st == 2
    # the linear layer's entry point: sizes, strides, dtypes, NULL pointers
    f = ctypes.c_float(1.0)
    st = lib.qo_w4a4_linear(None, 2, 4, 14336, None, None, 112, 128, f, None, 1792, 0, None, 0, None, None, None,
                            None, 4096, None)
    assert st == 2 and b"out_features" in lib.qo_last_error()
    st = lib.qo_w4a4_linear(None, 2, 4, 12, None, None, 3, 4, f, None, 2, 16, None, 0, None, None, None, None, 16,
                            None)
    assert st == 2 and b"divisible by 8" in lib.qo_last_error()
    st = lib.qo_w4a4_linear(None, 2, 4, 14336, None, None, 112, 128, f, None, 1000, 4096, None, 0, None, None, None,
                            None, 4096, None)
    assert st == 2 and b"row stride" in lib.qo_last_error()
    st = lib.qo_w4a4_linear(None, 7, 4, 14336, None, None, 112, 128, f, None, 1792, 4096, None, 0, None, None, None,
                            None, 4096, None)
    assert st == 3
    st = lib.qo_w4a4_linear(None, 2, 4, 14336, None, None, 112, 128, f, None, 1792, 4096, None, 9, None, None, None,
                            None, 4096, None)
    assert st == 3
    st = lib.qo_w4a4_linear(None, 2, 4, 14336, None, None, 112, 128, f, None, 1792, 4096, None, 0, None, None, None,
                            None, 4096, None)
    assert st == 1
    assert lib.qo_w4a4_linear(None, 2, 0, 14336, None, None, 112, 128, f, None, 1792, 4096, None, 0, None, None,
                              None, None, 4096, None) == 0
    # the no-allocation variant: the staging limit and the same argument checks,
    # all before any device call
    nl = lib.qo_w4a4_linear_noalloc
    assert capi.LINEAR_NOALLOC_MAX_BYTES == 32 * 1024 * 1024
    st = nl(None, 2, 5000, 14336, None, None, 112, 128, f, None, 1792, 4096, None, 0, None, None, 4096, None)
    assert st == 2 and b"staging" in lib.qo_last_error() and b"qo_w4a4_linear_noalloc" in lib.qo_last_error()
    st = nl(None, 2, 1 << 40, 14336, None, None, 112, 128, f, None, 1792, 4096, None, 0, None, None, 4096, None)
    assert st == 2 and b"staging" in lib.qo_last_error()
    st = nl(None, 2, 4, 12, None, None, 3, 4, f, None, 2, 16, None, 0, None, None, 16, None)
    assert st == 2 and b"divisible by 8" in lib.qo_last_error()
    st = nl(None, 2, -1, 14336, None, None, 112, 128, f, None, 1792, 4096, None, 0, None, None, 4096, None)
    assert st == 2 and b"invalid sizes" in lib.qo_last_error()
    assert nl(None, 2, 0, 14336, None, None, 112, 128, f, None, 1792, 4096, None, 0, None, None, 4096, None) == 0
    # empty problems are valid no-ops
    assert lib.qo_int4_gemm(None, 1, None, 1, 1, None, 0, None, 0, None, 1, 0, 0, 0, 8, None) == 0
    assert lib.qo_flatquant_quantize(None, 1, 0, 64, None, None, 8, 8, ctypes.c_float(1.0), 1, None, None,
                                     None) == 0


def _cfg(t=16, m=8, n=8, dtype=torch.float16, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(t, m * n, generator=g) * 2).to(dtype)
    L = torch.linalg.qr(torch.randn(m, m, generator=g))[0].to(dtype)
    R = torch.linalg.qr(torch.randn(n, n, generator=g))[0].to(dtype)
    return x, L, R


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("pack", [False, True])
def test_cpu_tensors_use_reference_fallback(dtype, pack):
    x, L, R = _cfg(dtype=dtype)
    q, s = qo.flatquant_dynamic_quantize(x, L, R, 0.9, pack)
    q2, s2 = qo.flatquant_dynamic_quantize(x, L, R, 0.9, pack, use_cuda=False)
    qr, sr = ofq.flatquant_pytorch(x, L, R, 0.9, pack)
    assert torch.equal(q, qr) and torch.equal(s, sr) and torch.equal(q2, qr) and torch.equal(s2, sr)
    assert s.dtype == dtype                      # fallback keeps the input dtype (flatquant/ops.py:113)
    assert q.dtype == (torch.int32 if pack else torch.int8)


def test_dequantize_cpu_matches_oracle():
    x, L, R = _cfg(t=5, m=8, n=16, dtype=torch.bfloat16)
    for pack in (False, True):
        q, s = qo.flatquant_dynamic_quantize(x, L, R, 1.0, pack)
        assert torch.equal(qo.dequantize_int4(q, s, pack), ofq.dequantize_int4(q, s, pack))


def test_pack_unpack_match_oracle():
    g = torch.Generator().manual_seed(3)
    q = torch.randint(-8, 8, (7, 40), generator=g, dtype=torch.int8)
    w = qo.pack_int4_to_int32(q)
    assert np.array_equal(w.numpy(), oi4.pack_int4_to_int32(q.numpy()))
    assert torch.equal(qo.unpack_int32_to_int4(w), q)


def test_transpose_packed_cpu():
    w = torch.arange(6 * 10, dtype=torch.int32).view(6, 10)
    t = qo.transpose_packed(w)
    assert t.is_contiguous() and torch.equal(t, w.t())
    # a [K/8, N] weight built as pack(b.T).T and the [N, K/8] packing of the same
    # codes are transposes of each other
    g = torch.Generator().manual_seed(8)
    codes = torch.randint(-8, 8, (12, 32), generator=g, dtype=torch.int8)   # [N, K]
    assert torch.equal(qo.transpose_packed(qo.pack_int4_to_int32(codes)),
                       qo.pack_int4_to_int32(codes).t().contiguous())


def test_prepare_weight_clamps_then_packs():
    w = torch.tensor([[-20, -8, -1, 0, 3, 7, 8, 100]], dtype=torch.int32)
    packed = qo.prepare_w4a4_weight(w)
    # clamp to [-8, 7] first (pack_int4_to_int32_manual): codes -8 -8 -1 0 3 7 7 7
    expect = sum((c + 8) << (4 * i) for i, c in enumerate([-8, -8, -1, 0, 3, 7, 7, 7]))
    assert packed.dtype == torch.int32 and int(packed[0, 0]) & 0xFFFFFFFF == expect


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_w4a4_linear_cpu_composes_quantize_and_gemm(dtype):
    """The linear equals quantize -> int4 GEMM on W.t() -> + bias, and, with
    orthogonal transforms, approximates x @ W_deqᵀ (a transposed weight or a
    transform applied on the wrong side fails the second check)."""
    g = torch.Generator().manual_seed(12)
    m, n, out_f, t = 4, 8, 16, 6
    x = torch.randn(2, t // 2, m * n, generator=g).to(dtype)
    L, R = wl.orthogonal(m, 31).to(dtype), wl.orthogonal(n, 32).to(dtype)
    wc = torch.randint(-8, 8, (out_f, m * n), generator=g, dtype=torch.int8)
    sw = (torch.rand(out_f, generator=g) * 0.1 + 0.01).float()
    bias = torch.randn(out_f, generator=g).to(dtype)
    wp = qo.prepare_w4a4_weight(wc)
    y = qo.w4a4_flatquant_linear(x, L, R, wp, sw.view(-1, 1), clip_ratio=1.0, bias=bias)
    assert y.shape == (2, t // 2, out_f) and y.dtype == dtype
    q, s = ofq.flatquant_pytorch(x.reshape(-1, m * n), L, R, 1.0, True)
    ref = oi4.int4_matmul_pytorch(q, wp.t(), s.float(), sw, out_dtype=dtype) + bias
    assert torch.equal(y.reshape(-1, out_f), ref)
    # Y = quantized (x·kron(L,R)); W acts on the transformed input, so compare
    # with (x·kron(L,R)) @ (W·diag)ᵀ in float64
    kron = torch.kron(L.double(), R.double())
    xt = x.reshape(-1, m * n).double() @ kron
    exact = xt @ (wc.double() * sw.double().view(-1, 1)).t() + bias.double()
    rel = (y.reshape(-1, out_f).double() - exact).norm() / exact.norm()
    assert rel < 0.15


def test_int4_matmul_cpu_matches_oracle():
    g = torch.Generator().manual_seed(4)
    qa = torch.randint(-8, 8, (9, 64), generator=g, dtype=torch.int8)
    qb = torch.randint(-8, 8, (64, 11), generator=g, dtype=torch.int8)
    a = qo.pack_int4_to_int32(qa)
    b = qo.pack_int4_to_int32(qb.T).T.contiguous()
    sa = torch.rand(9, generator=g).half()
    sb = torch.rand(11, generator=g).half()
    out = qo.int4_matmul(a, b, sa, sb)
    ref = oi4.int4_matmul_pytorch(a, b, sa, sb)
    assert out.dtype == torch.float16 and torch.equal(out, ref)
    assert qo.int4_matmul(a, b, sa, sb, out_dtype=torch.bfloat16).dtype == torch.bfloat16


def test_get_decompose_dim():
    assert qo.get_decompose_dim(4096) == (64, 64)
    assert qo.get_decompose_dim(2048) == (32, 64)
    assert qo.get_decompose_dim(14336) == (112, 128)
    assert qo.get_decompose_dim(0) == (0, 0)
    with pytest.raises(ValueError):
        qo.get_decompose_dim(6)


def test_gpu_entry_points_refuse_without_kernels(monkeypatch):
    monkeypatch.setattr(_loader, "KERNELS_AVAILABLE", False)
    monkeypatch.setattr(_loader, "LOAD_ERROR", "simulated")
    x, L, R = _cfg()
    with pytest.raises(RuntimeError, match="not available"):
        qo.flatquant_cuda(x, L, R)
    with pytest.raises(RuntimeError, match="not available"):
        qo.int4_matmul_cuda(torch.zeros(1, 1, dtype=torch.int32), torch.zeros(1, 1, dtype=torch.int32),
                            torch.ones(1), torch.ones(1))
    # the CPU path is unaffected
    qo.flatquant_dynamic_quantize(x, L, R)


def test_fake_kernels_give_reference_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        a = torch.empty(5, 16, dtype=torch.int32)
        b = torch.empty(16, 9, dtype=torch.int32)
        o = torch.ops.quant_ops.int4_matmul_bias(a, b, torch.empty(5), torch.empty(9), torch.empty(9),
                                                 torch.bfloat16)
        assert o.shape == (5, 9) and o.dtype == torch.bfloat16
        x = torch.empty(6, 64, dtype=torch.float16)
        L = torch.empty(8, 8, dtype=torch.float16)
        q, s = torch.ops.quant_ops.flatquant_dynamic_quantize(x, L, L, 0.9, True)
        assert q.shape == (6, 8) and q.dtype == torch.int32 and s.shape == (6,) and s.dtype == torch.float32
        q, s = torch.ops.quant_ops.flatquant_dynamic_quantize(x, L, L, 0.9, False)
        assert q.shape == (6, 64) and q.dtype == torch.int8
        a = torch.empty(5, 4, dtype=torch.int32)
        b = torch.empty(4, 7, dtype=torch.int32)
        o = torch.ops.quant_ops.int4_matmul(a, b, torch.empty(5), torch.empty(7))
        assert o.shape == (5, 7) and o.dtype == torch.float16
        o = torch.ops.quant_ops.int4_matmul_ex(a, b, torch.empty(5), torch.empty(7), torch.bfloat16)
        assert o.dtype == torch.bfloat16
        d = torch.ops.quant_ops.dequantize_int4(a, torch.empty(5), True)
        assert d.shape == (5, 32) and d.dtype == torch.float32
        w = torch.empty(24, 8, dtype=torch.int32)
        y = torch.ops.quant_ops.w4a4_linear(x, L, L, w, torch.empty(24, dtype=torch.bfloat16), 0.9, None)
        assert y.shape == (6, 24) and y.dtype == torch.float16


def test_workload_generators_are_seeded():
    from quant_ops_amd import workloads as wl

    c1, c2 = wl.quant_cfg2(tokens=8), wl.quant_cfg2(tokens=8)
    assert torch.equal(c1.x, c2.x) and torch.equal(c1.left, c2.left)
    assert c1.x.dtype == torch.float16 and c1.pack_int32 and c1.clip_ratio == 0.9
    full = wl.quant_cfg2()
    assert full.algorithmic_bytes() == 20_996_096      # X + packed codes + fp32 scales + L, R
    g = wl.gemm_case(32, 48, 64, b_transposed_view=True)
    assert g.b.shape == (8, 48) and g.b.stride() == (1, 8)
    assert wl.gemm_cfg4().ops() == 481_036_337_152


# ----------------------------------------------------------------- the reference's import surface

def test_reference_import_paths_resolve():
    """Every name the reference's examples and tests import resolves to this
    build's object (examples/basic_usage.py:13-14, examples/int4_matmul_benchmark.py:12-13,
    tests/test_accuracy.py:15-20, tests/test_performance.py:21-26)."""
    import quant_ops
    import quant_ops_amd
    from quant_ops import (CUDA_AVAILABLE, dequantize_int4, flatquant_dynamic_quantize, get_decompose_dim,
                           int4_matmul)
    from quant_ops.ops.quantization.flatquant.ops import flatquant_cuda, flatquant_pytorch
    from quant_ops.ops.quantization.flatquant.kernels import CUDA_KERNELS_AVAILABLE as FQ_AVAILABLE
    from quant_ops.ops.quantization.flatquant.kernels import cuda_quant_ops
    from quant_ops.ops.quantization.int4_matmul.ops import int4_matmul_cuda, int4_matmul_pytorch, pack_int4_to_int32
    from quant_ops.ops.quantization.int4_matmul.ops import unpack_int32_to_int4
    from quant_ops.ops.quantization.int4_matmul.kernels import CUDA_KERNELS_AVAILABLE as MM_AVAILABLE
    from quant_ops.ops.quantization.int4_matmul.kernels import cuda_int4_matmul_ops
    from quant_ops.ops.quantization.int4_matmul import int4_matmul as int4_matmul_pkg
    from quant_ops.ops.quantization.flatquant import flatquant_dynamic_quantize as fdq_pkg
    from quant_ops.utils.decompose import get_decompose_dim as gdd
    from quant_ops.utils import get_decompose_dim as gdd2
    import quant_ops.meta_ops  # noqa: F401

    assert quant_ops.__version__ == quant_ops_amd.__version__
    assert sorted(quant_ops.__all__) == sorted(["flatquant_dynamic_quantize", "dequantize_int4", "int4_matmul",
                                                "get_decompose_dim", "CUDA_AVAILABLE"])
    assert flatquant_dynamic_quantize is quant_ops_amd.flatquant_dynamic_quantize is fdq_pkg
    assert dequantize_int4 is quant_ops_amd.dequantize_int4
    assert int4_matmul is quant_ops_amd.int4_matmul is int4_matmul_pkg
    assert get_decompose_dim is gdd is gdd2 is quant_ops_amd.get_decompose_dim
    assert flatquant_cuda is quant_ops_amd.flatquant_cuda and flatquant_pytorch is quant_ops_amd.flatquant_pytorch
    assert int4_matmul_cuda is quant_ops_amd.int4_matmul_cuda
    assert int4_matmul_pytorch is quant_ops_amd.int4_matmul_pytorch
    assert pack_int4_to_int32 is quant_ops_amd.pack_int4_to_int32
    assert unpack_int32_to_int4 is quant_ops_amd.unpack_int32_to_int4
    assert CUDA_AVAILABLE == quant_ops_amd.CUDA_AVAILABLE == FQ_AVAILABLE == MM_AVAILABLE
    if CUDA_AVAILABLE:
        assert callable(cuda_quant_ops.cuda_kronecker_quant_int8)
        assert callable(cuda_int4_matmul_ops.cuda_int4_matmul)
    else:
        assert cuda_quant_ops is None and cuda_int4_matmul_ops is None
    # the reference's CPU path through the new import surface
    x = torch.randn(4, 4096, dtype=torch.float16)
    L = torch.eye(64, dtype=torch.float16)
    q, s = flatquant_dynamic_quantize(x, L, L, 1.0, True, use_cuda=False)
    assert q.shape == (4, 512) and s.shape == (4,)


def test_pybind_equivalents_check_arguments_like_the_reference():
    """cuda_int4_matmul rejects host tensors and non-float32 scales with the
    reference's messages (cuda_int4_matmul_kernel.cu:136-150)."""
    from quant_ops_amd import extension

    if not extension.CUDA_KERNELS_AVAILABLE:
        pytest.skip("HIP library not built")
    a = torch.zeros(2, 1, dtype=torch.int32)
    b = torch.zeros(1, 3, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="a_packed must be on CUDA"):
        extension.cuda_int4_matmul(a, b, torch.ones(2), torch.ones(3))


def test_bench_rotation_and_gpu_count(tmp_path):
    """bench.py gives every timed step its own buffer set while the sets fit,
    never fewer than 1.25 x the MALL's worth, and refuses more than one GPU."""
    import bench

    assert bench._nsets(155_226_112, 20) == 20                # config 4: one set per step
    assert bench._nsets(20_996_096, 5) == 16                 # few steps: still past the MALL
    assert bench._nsets(300_000_000, 1000) == bench.ROTATION_CAP_BYTES // 300_000_000
    proc = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                          capture_output=True, text=True)
    assert proc.returncode == 2 and "one GPU only" in proc.stderr


def test_kernel_routing_mask_round_trips():
    """qo_set_kernel_routing keeps only the QO_ROUTE_* bits and returns the previous mask."""
    prev = capi.set_kernel_routing(capi.route_mask("FQ_GENERIC", "GEMM_NO_DMA"))
    try:
        assert capi.set_kernel_routing(0xFFFFFFFF) == capi.route_mask("FQ_GENERIC", "GEMM_NO_DMA")
        assert capi.set_kernel_routing(0) == sum(capi.ROUTE.values())
        with capi.kernel_routing("FQ_NO_DUO"):
            assert capi.set_kernel_routing(capi.route_mask("FQ_NO_DUO")) == capi.route_mask("FQ_NO_DUO")
        assert capi.set_kernel_routing(0) == 0
    finally:
        capi.set_kernel_routing(prev)
