"""ctypes binding of the C ABI in ``include/quant_ops_hip.h``.

This is the FFI view of ``libquant_ops_hip.so``: plain device pointers, sizes,
strides and a stream handle, no torch types. Tests and the benchmark call the
kernels through it; torch tensors are only used here to own device memory and
to name the current stream. Every call raises ``QuantOpsError`` on a non-zero
status, with the library's message.
"""
import contextlib
import ctypes
import os

import torch

from ._loader import HIP_LIB_PATH

DTYPE_F32, DTYPE_F16, DTYPE_BF16, DTYPE_I8, DTYPE_I32 = 0, 1, 2, 3, 4
STATUS = {0: "QO_OK", 1: "QO_ERR_NULL_POINTER", 2: "QO_ERR_SHAPE", 3: "QO_ERR_DTYPE",
          4: "QO_ERR_ALIGNMENT", 5: "QO_ERR_UNSUPPORTED", 6: "QO_ERR_LAUNCH"}

# Every symbol the header declares; the CPU tests check they are all exported.
EXPORTED = ("qo_status_string", "qo_version", "qo_last_error", "qo_set_kernel_routing", "qo_flatquant_quantize",
            "qo_int4_gemm", "qo_int4_gemm_bias", "qo_int4_gemm_ws", "qo_int4_gemm_workspace_size", "qo_int4_gemm_f6_workspace_bytes",
            "qo_int4_gemm_f6_prepare", "qo_int4_gemm_f6_run", "qo_int4_gemm_f6_operand_bytes",
            "qo_int4_gemm_f6_convert", "qo_int4_gemm_f6_run2", "qo_w4a4_linear_f6w", "qo_w4a4_linear", "qo_w4a4_linear_ws", "qo_w4a4_linear_noalloc", "qo_dequantize_int4",
            "qo_pack_int4_to_int32", "qo_unpack_int32_to_int4", "qo_transpose_int32")

# QO_ROUTE_* bits of qo_set_kernel_routing (include/quant_ops_hip.h)
ROUTE = {"FQ_GENERIC": 1 << 0, "FQ_NO_WAVE": 1 << 1, "FQ_NO_DUO": 1 << 2, "FQ_NO_FEW": 1 << 3,
         "GEMM_GENERIC": 1 << 4, "GEMM_NO_DMA": 1 << 5, "GEMM_NO_SKINNY": 1 << 6,
         "LINEAR_NO_READ_AHEAD": 1 << 7, "GEMM_NO_F6": 1 << 8}

_TORCH_CODE = {torch.float32: DTYPE_F32, torch.float16: DTYPE_F16, torch.bfloat16: DTYPE_BF16}


class QuantOpsError(RuntimeError):
    def __init__(self, status, message):
        super().__init__(f"{STATUS.get(status, status)}: {message}")
        self.status = status


_lib = None


def lib():
    """Load (once) and return the ctypes handle with argument types set."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(HIP_LIB_PATH):
        raise QuantOpsError(5, f"{HIP_LIB_PATH} is not built")
    L = ctypes.CDLL(HIP_LIB_PATH)
    c_i64, c_int, c_vp, c_f = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_float
    L.qo_status_string.restype = ctypes.c_char_p
    L.qo_status_string.argtypes = [c_int]
    L.qo_version.restype = ctypes.c_char_p
    L.qo_version.argtypes = []
    L.qo_last_error.restype = ctypes.c_char_p
    L.qo_last_error.argtypes = []
    L.qo_set_kernel_routing.restype = ctypes.c_uint
    L.qo_set_kernel_routing.argtypes = [ctypes.c_uint]
    L.qo_flatquant_quantize.restype = c_int
    L.qo_flatquant_quantize.argtypes = [c_vp, c_int, c_i64, c_i64, c_vp, c_vp, c_int, c_int, c_f, c_int,
                                        c_vp, c_vp, c_vp]
    L.qo_int4_gemm.restype = c_int
    L.qo_int4_gemm.argtypes = [c_vp, c_i64, c_vp, c_i64, c_i64, c_vp, c_int, c_vp, c_int, c_vp, c_int, c_i64,
                               c_i64, c_i64, c_i64, c_vp]
    L.qo_int4_gemm_bias.restype = c_int
    L.qo_int4_gemm_bias.argtypes = [c_vp, c_i64, c_vp, c_i64, c_i64, c_vp, c_int, c_vp, c_int, c_vp, c_vp, c_int,
                                    c_i64, c_i64, c_i64, c_i64, c_vp]
    L.qo_int4_gemm_ws.restype = c_int
    L.qo_int4_gemm_ws.argtypes = [c_vp, c_i64, c_vp, c_i64, c_i64, c_vp, c_int, c_vp, c_int, c_vp, c_vp, c_int,
                                  c_i64, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp]
    L.qo_int4_gemm_workspace_size.restype = c_i64
    L.qo_int4_gemm_workspace_size.argtypes = [c_i64, c_i64, c_i64, c_int]
    L.qo_int4_gemm_f6_workspace_bytes.restype = c_i64
    L.qo_int4_gemm_f6_workspace_bytes.argtypes = [c_i64, c_i64, c_i64]
    L.qo_int4_gemm_f6_prepare.restype = c_int
    L.qo_int4_gemm_f6_prepare.argtypes = [c_vp, c_i64, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp]
    L.qo_int4_gemm_f6_run.restype = c_int
    L.qo_int4_gemm_f6_run.argtypes = [c_vp, c_int, c_vp, c_int, c_vp, c_vp, c_int, c_i64, c_i64, c_i64, c_i64, c_vp,
                                      c_i64, c_vp]
    L.qo_w4a4_linear.restype = c_int
    L.qo_w4a4_linear.argtypes = [c_vp, c_int, c_i64, c_i64, c_vp, c_vp, c_int, c_int, c_f, c_vp, c_i64, c_i64,
                                 c_vp, c_int, c_vp, c_vp, c_vp, c_vp, c_i64, c_vp]
    L.qo_w4a4_linear_ws.restype = c_int
    L.qo_w4a4_linear_ws.argtypes = [c_vp, c_int, c_i64, c_i64, c_vp, c_vp, c_int, c_int, c_f, c_vp, c_i64, c_i64,
                                    c_vp, c_int, c_vp, c_vp, c_vp, c_vp, c_i64, c_vp, c_i64, c_vp]
    L.qo_int4_gemm_f6_operand_bytes.restype = c_i64
    L.qo_int4_gemm_f6_operand_bytes.argtypes = [c_i64, c_i64]
    L.qo_int4_gemm_f6_convert.restype = c_int
    L.qo_int4_gemm_f6_convert.argtypes = [c_vp, c_i64, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp]
    L.qo_int4_gemm_f6_run2.restype = c_int
    L.qo_int4_gemm_f6_run2.argtypes = [c_vp, c_i64, c_vp, c_i64, c_vp, c_int, c_vp, c_int, c_vp, c_vp, c_int, c_i64,
                                       c_i64, c_i64, c_i64, c_vp]
    L.qo_w4a4_linear_f6w.restype = c_int
    L.qo_w4a4_linear_f6w.argtypes = [c_vp, c_int, c_i64, c_i64, c_vp, c_vp, c_int, c_int, c_f, c_vp, c_i64, c_i64,
                                     c_vp, c_int, c_vp, c_vp, c_vp, c_vp, c_i64, c_vp, c_i64, c_vp]
    L.qo_w4a4_linear_noalloc.restype = c_int
    L.qo_w4a4_linear_noalloc.argtypes = [c_vp, c_int, c_i64, c_i64, c_vp, c_vp, c_int, c_int, c_f, c_vp, c_i64,
                                         c_i64, c_vp, c_int, c_vp, c_vp, c_i64, c_vp]
    L.qo_dequantize_int4.restype = c_int
    L.qo_dequantize_int4.argtypes = [c_vp, c_int, c_vp, c_int, c_i64, c_i64, c_vp, c_vp]
    for name in ("qo_pack_int4_to_int32", "qo_unpack_int32_to_int4", "qo_transpose_int32"):
        fn = getattr(L, name)
        fn.restype = c_int
        fn.argtypes = [c_vp, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp]
    _lib = L
    return L


def _check(status):
    if status != 0:
        raise QuantOpsError(status, lib().qo_last_error().decode())


def _stream(stream):
    if stream is None:
        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if isinstance(stream, torch.cuda.Stream):
        return ctypes.c_void_p(stream.cuda_stream)
    return ctypes.c_void_p(stream)


def version() -> str:
    return lib().qo_version().decode()


def set_kernel_routing(mask: int) -> int:
    """Set the process-wide QO_ROUTE_* mask; returns the previous one."""
    return int(lib().qo_set_kernel_routing(mask))


def route_mask(*names) -> int:
    mask = 0
    for name in names:
        mask |= ROUTE[name]
    return mask


@contextlib.contextmanager
def kernel_routing(*names):
    """Add the named QO_ROUTE_* bits (``ROUTE`` keys) for the duration of the block."""
    prev = set_kernel_routing(0)
    set_kernel_routing(prev | route_mask(*names))
    try:
        yield
    finally:
        set_kernel_routing(prev)


def flatquant_quantize(x, left, right, clip_ratio=1.0, pack_int32=False, out_codes=None, out_scales=None,
                       stream=None):
    """Call ``qo_flatquant_quantize`` on device tensors; allocates outputs if not given.

    The C ABI reads L and R as row-major [M, M] / [N, N]; other layouts (e.g. the
    column-major Q that torch.linalg.qr returns) are made contiguous here.
    """
    t, f = x.shape
    if x.stride(1) != 1:
        x = x.contiguous()
    left, right = left.contiguous(), right.contiguous()
    m, n = left.shape[0], right.shape[0]
    if out_codes is None:
        out_codes = torch.empty((t, f // 8) if pack_int32 else (t, f),
                                dtype=torch.int32 if pack_int32 else torch.int8, device=x.device)
    if out_scales is None:
        out_scales = torch.empty((t,), dtype=torch.float32, device=x.device)
    _check(lib().qo_flatquant_quantize(
        ctypes.c_void_p(x.data_ptr()), _TORCH_CODE[x.dtype], t, x.stride(0) if t else f,
        ctypes.c_void_p(left.data_ptr()), ctypes.c_void_p(right.data_ptr()), m, n,
        float(clip_ratio), 1 if pack_int32 else 0,
        ctypes.c_void_p(out_codes.data_ptr()), ctypes.c_void_p(out_scales.data_ptr()), _stream(stream)))
    return out_codes, out_scales


def gemm_workspace_size(m, n, k, out_dtype=torch.float16):
    """``qo_int4_gemm_workspace_size``: bytes of the FP6 route's workspace (0: not taken)."""
    return int(lib().qo_int4_gemm_workspace_size(m, n, k, _TORCH_CODE[out_dtype]))


def int4_gemm(a, b, scale_a, scale_b, out_dtype=torch.float16, out=None, stream=None, bias=None,
              workspace=None):
    """Call ``qo_int4_gemm`` (``qo_int4_gemm_bias`` with ``bias``, converted to the
    output dtype); ``b`` may be row-major [K/8, N] or the ``W.t()`` view. With
    ``workspace`` (a uint8 device tensor, or True to allocate one of
    gemm_workspace_size bytes) the call goes to ``qo_int4_gemm_ws``."""
    m, kp = a.shape
    if a.stride(1) != 1:
        a = a.contiguous()
    if b.stride(0) != 1 and b.stride(1) != 1:
        b = b.contiguous()
    scale_a, scale_b = scale_a.contiguous(), scale_b.contiguous()
    n = b.shape[1]
    if out is None:
        out = torch.empty((m, n), dtype=out_dtype, device=a.device)
    head = (ctypes.c_void_p(a.data_ptr()), a.stride(0) if m else kp,
            ctypes.c_void_p(b.data_ptr()), b.stride(0), b.stride(1),
            ctypes.c_void_p(scale_a.data_ptr()), _TORCH_CODE[scale_a.dtype],
            ctypes.c_void_p(scale_b.data_ptr()), _TORCH_CODE[scale_b.dtype])
    tail = (ctypes.c_void_p(out.data_ptr()), _TORCH_CODE[out.dtype], out.stride(0) if m else n,
            m, n, kp * 8, _stream(stream))
    if bias is not None:
        bias = bias.to(out.dtype).contiguous()
    if workspace is not None:
        if workspace is True:
            workspace = torch.empty(max(1, gemm_workspace_size(m, n, kp * 8, out.dtype)), dtype=torch.uint8,
                                    device=a.device)
        _check(lib().qo_int4_gemm_ws(*head, ctypes.c_void_p(bias.data_ptr() if bias is not None else None),
                                     *tail[:-1], ctypes.c_void_p(workspace.data_ptr()), workspace.numel(),
                                     tail[-1]))
    elif bias is None:
        _check(lib().qo_int4_gemm(*head, *tail))
    else:
        _check(lib().qo_int4_gemm_bias(*head, ctypes.c_void_p(bias.data_ptr()), *tail))
    return out


def f6_workspace_bytes(m, n, k):
    """``qo_int4_gemm_f6_workspace_bytes``."""
    return int(lib().qo_int4_gemm_f6_workspace_bytes(m, n, k))


def f6_prepare(workspace, m, n, k, a=None, b=None, stream=None):
    """``qo_int4_gemm_f6_prepare``: convert A [M, K/8] and / or B ([K/8, N] or the
    ``W.t()`` view) into ``workspace`` (uint8 device tensor)."""
    if a is not None and a.stride(1) != 1:
        a = a.contiguous()
    if b is not None and b.stride(0) != 1 and b.stride(1) != 1:
        b = b.contiguous()
    _check(lib().qo_int4_gemm_f6_prepare(
        ctypes.c_void_p(a.data_ptr() if a is not None else None), a.stride(0) if a is not None else 0,
        ctypes.c_void_p(b.data_ptr() if b is not None else None), b.stride(0) if b is not None else 0,
        b.stride(1) if b is not None else 0, m, n, k, ctypes.c_void_p(workspace.data_ptr()), workspace.numel(),
        _stream(stream)))


def f6_run(workspace, m, n, k, scale_a, scale_b, out_dtype=torch.float16, out=None, bias=None, stream=None):
    """``qo_int4_gemm_f6_run`` on a prepared ``workspace``; returns out [M, N]."""
    scale_a, scale_b = scale_a.contiguous(), scale_b.contiguous()
    if out is None:
        out = torch.empty((m, n), dtype=out_dtype, device=workspace.device)
    if bias is not None:
        bias = bias.to(out.dtype).contiguous()
    _check(lib().qo_int4_gemm_f6_run(
        ctypes.c_void_p(scale_a.data_ptr()), _TORCH_CODE[scale_a.dtype], ctypes.c_void_p(scale_b.data_ptr()),
        _TORCH_CODE[scale_b.dtype], ctypes.c_void_p(bias.data_ptr() if bias is not None else None),
        ctypes.c_void_p(out.data_ptr()), _TORCH_CODE[out.dtype], out.stride(0), m, n, k,
        ctypes.c_void_p(workspace.data_ptr()), workspace.numel(), _stream(stream)))
    return out


def f6_operand_bytes(rows, k):
    """``qo_int4_gemm_f6_operand_bytes``."""
    return int(lib().qo_int4_gemm_f6_operand_bytes(rows, k))


def f6_convert(src, k, rows_are_columns=False, out=None, stream=None):
    """``qo_int4_gemm_f6_convert``: an operand in the FP6 layout. ``src`` int32
    [rows, K/8] (A, or a [N, K/8] weight whose W.t() is B), or with
    ``rows_are_columns`` a row-major [K/8, N] B. Returns the uint8 tensor."""
    if rows_are_columns:
        rows, rs, ws_ = src.shape[1], src.stride(1), src.stride(0)
    else:
        rows, rs, ws_ = src.shape[0], src.stride(0), src.stride(1)
    n = f6_operand_bytes(rows, k)
    if out is None:
        out = torch.empty(n, dtype=torch.uint8, device=src.device)
    _check(lib().qo_int4_gemm_f6_convert(ctypes.c_void_p(src.data_ptr()), rs, ws_, rows, k,
                                         ctypes.c_void_p(out.data_ptr()), out.numel(), _stream(stream)))
    return out


def w4a4_linear_f6w(x, left, right, weight_f6, out_features, weight_scale, clip_ratio=1.0, bias=None, out=None,
                    codes=None, scales=None, a_workspace=None, stream=None):
    """``qo_w4a4_linear_f6w`` against ``weight_f6`` (``f6_convert(weight, M*N)`` of
    the packed [out, M*N/8] weight). Returns (out, codes, scales)."""
    t, f = x.shape
    if x.stride(1) != 1:
        x = x.contiguous()
    left, right = left.contiguous(), right.contiguous()
    weight_scale = weight_scale.reshape(-1).contiguous()
    m, n = left.shape[0], right.shape[0]
    if codes is None:
        codes = torch.empty((t, f // 8), dtype=torch.int32, device=x.device)
    if scales is None:
        scales = torch.empty((t,), dtype=torch.float32, device=x.device)
    if out is None:
        out = torch.empty((t, out_features), dtype=x.dtype, device=x.device)
    if a_workspace is None:
        a_workspace = torch.empty(max(1, f6_operand_bytes(t, f)), dtype=torch.uint8, device=x.device)
    if bias is not None:
        bias = bias.to(x.dtype).contiguous()
    _check(lib().qo_w4a4_linear_f6w(
        ctypes.c_void_p(x.data_ptr()), _TORCH_CODE[x.dtype], t, x.stride(0) if t else f,
        ctypes.c_void_p(left.data_ptr()), ctypes.c_void_p(right.data_ptr()), m, n, float(clip_ratio),
        ctypes.c_void_p(weight_f6.data_ptr()), weight_f6.numel(), out_features,
        ctypes.c_void_p(weight_scale.data_ptr()), _TORCH_CODE[weight_scale.dtype],
        ctypes.c_void_p(bias.data_ptr() if bias is not None else None),
        ctypes.c_void_p(codes.data_ptr()), ctypes.c_void_p(scales.data_ptr()),
        ctypes.c_void_p(out.data_ptr()), out.stride(0) if t else out_features,
        ctypes.c_void_p(a_workspace.data_ptr()), a_workspace.numel(), _stream(stream)))
    return out, codes, scales


def w4a4_linear(x, left, right, weight, weight_scale, clip_ratio=1.0, bias=None, out=None, codes=None,
                scales=None, stream=None, workspace=None):
    """Call ``qo_w4a4_linear``: x [T, M*N] (float32 / float16 / bfloat16), the packed
    weight int32 [out, M*N/8] (rows may be strided), weight_scale [out], optional
    bias [out] (converted to x's dtype). Returns (out [T, out] in x's dtype, packed
    codes [T, M*N/8], float32 scales [T]). With ``workspace`` (a uint8 device
    tensor, or True to allocate gemm_workspace_size bytes) ``qo_w4a4_linear_ws``."""
    t, f = x.shape
    if x.stride(1) != 1:
        x = x.contiguous()
    left, right = left.contiguous(), right.contiguous()
    if weight.stride(1) != 1:
        weight = weight.contiguous()
    weight_scale = weight_scale.reshape(-1).contiguous()
    m, n = left.shape[0], right.shape[0]
    no = weight.shape[0]
    if codes is None:
        codes = torch.empty((t, f // 8), dtype=torch.int32, device=x.device)
    if scales is None:
        scales = torch.empty((t,), dtype=torch.float32, device=x.device)
    if out is None:
        out = torch.empty((t, no), dtype=x.dtype, device=x.device)
    if bias is not None:
        bias = bias.to(x.dtype).contiguous()
    args = (ctypes.c_void_p(x.data_ptr()), _TORCH_CODE[x.dtype], t, x.stride(0) if t else f,
            ctypes.c_void_p(left.data_ptr()), ctypes.c_void_p(right.data_ptr()), m, n, float(clip_ratio),
            ctypes.c_void_p(weight.data_ptr()), _ld(weight), no,
            ctypes.c_void_p(weight_scale.data_ptr()), _TORCH_CODE[weight_scale.dtype],
            ctypes.c_void_p(bias.data_ptr() if bias is not None else None),
            ctypes.c_void_p(codes.data_ptr()), ctypes.c_void_p(scales.data_ptr()),
            ctypes.c_void_p(out.data_ptr()), out.stride(0) if t else no)
    if workspace is None:
        _check(lib().qo_w4a4_linear(*args, _stream(stream)))
    else:
        if workspace is True:
            workspace = torch.empty(max(1, gemm_workspace_size(t, no, f, x.dtype)), dtype=torch.uint8,
                                    device=x.device)
        _check(lib().qo_w4a4_linear_ws(*args, ctypes.c_void_p(workspace.data_ptr()), workspace.numel(),
                                       _stream(stream)))
    return out, codes, scales


# Byte size of the staging array of qo_w4a4_linear_noalloc (its header's
# QO_LINEAR_NOALLOC_MAX_BYTES).
LINEAR_NOALLOC_MAX_BYTES = 32 * 1024 * 1024


def w4a4_linear_noalloc(x, left, right, weight, weight_scale, clip_ratio=1.0, bias=None, out=None, stream=None):
    """Call ``qo_w4a4_linear_noalloc``: as ``w4a4_linear``, with the activation
    codes and scales staged in the library's per-GPU array instead of caller
    buffers (nothing is allocated except ``out`` when it is not given). Returns
    out [T, out_features] in x's dtype."""
    t, f = x.shape
    if x.stride(1) != 1:
        x = x.contiguous()
    left, right = left.contiguous(), right.contiguous()
    if weight.stride(1) != 1:
        weight = weight.contiguous()
    weight_scale = weight_scale.reshape(-1).contiguous()
    m, n = left.shape[0], right.shape[0]
    no = weight.shape[0]
    if out is None:
        out = torch.empty((t, no), dtype=x.dtype, device=x.device)
    if bias is not None:
        bias = bias.to(x.dtype).contiguous()
    _check(lib().qo_w4a4_linear_noalloc(
        ctypes.c_void_p(x.data_ptr()), _TORCH_CODE[x.dtype], t, x.stride(0) if t else f,
        ctypes.c_void_p(left.data_ptr()), ctypes.c_void_p(right.data_ptr()), m, n, float(clip_ratio),
        ctypes.c_void_p(weight.data_ptr()), _ld(weight), no,
        ctypes.c_void_p(weight_scale.data_ptr()), _TORCH_CODE[weight_scale.dtype],
        ctypes.c_void_p(bias.data_ptr() if bias is not None else None),
        ctypes.c_void_p(out.data_ptr()), out.stride(0) if t else no, _stream(stream)))
    return out


def dequantize_int4(codes, scales, packed_int32=False, out=None, stream=None):
    """Call ``qo_dequantize_int4``; returns float32 [T, F]."""
    codes, scales = codes.contiguous(), scales.contiguous()
    t = codes.shape[0]
    f = codes.shape[1] * (8 if packed_int32 else 1)
    if out is None:
        out = torch.empty((t, f), dtype=torch.float32, device=codes.device)
    _check(lib().qo_dequantize_int4(
        ctypes.c_void_p(codes.data_ptr()), 1 if packed_int32 else 0,
        ctypes.c_void_p(scales.data_ptr()), _TORCH_CODE[scales.dtype], t, f,
        ctypes.c_void_p(out.data_ptr()), _stream(stream)))
    return out


def _ld(t):
    return t.stride(0) if t.dim() == 2 and t.shape[0] > 1 else t.shape[-1]


def pack_int4_to_int32(codes, out=None, stream=None):
    """Call ``qo_pack_int4_to_int32``: int8 [rows, F] -> int32 [rows, F/8] (rows may be strided)."""
    assert codes.dtype == torch.int8 and codes.dim() == 2 and codes.stride(1) == 1
    rows, feats = codes.shape
    if out is None:
        out = torch.empty((rows, feats // 8), dtype=torch.int32, device=codes.device)
    _check(lib().qo_pack_int4_to_int32(ctypes.c_void_p(codes.data_ptr()), _ld(codes), rows, feats,
                                       ctypes.c_void_p(out.data_ptr()), _ld(out), _stream(stream)))
    return out


def unpack_int32_to_int4(words, out=None, stream=None):
    """Call ``qo_unpack_int32_to_int4``: int32 [rows, W] -> int8 [rows, 8W] (rows may be strided)."""
    assert words.dtype == torch.int32 and words.dim() == 2 and words.stride(1) == 1
    rows, nw = words.shape
    if out is None:
        out = torch.empty((rows, 8 * nw), dtype=torch.int8, device=words.device)
    _check(lib().qo_unpack_int32_to_int4(ctypes.c_void_p(words.data_ptr()), _ld(words), rows, nw,
                                         ctypes.c_void_p(out.data_ptr()), _ld(out), _stream(stream)))
    return out


def transpose_int32(x, out=None, stream=None):
    """Call ``qo_transpose_int32``: int32 [R, C] -> contiguous int32 [C, R]."""
    assert x.dtype == torch.int32 and x.dim() == 2 and x.stride(1) == 1
    rows, cols = x.shape
    if out is None:
        out = torch.empty((cols, rows), dtype=torch.int32, device=x.device)
    _check(lib().qo_transpose_int32(ctypes.c_void_p(x.data_ptr()), _ld(x), rows, cols,
                                    ctypes.c_void_p(out.data_ptr()), _ld(out), _stream(stream)))
    return out
