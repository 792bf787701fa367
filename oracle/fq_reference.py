"""Oracle for the FlatQuant dynamic int4 quantize — test infrastructure only.

Restates the reference fallback ``flatquant_pytorch``
(``src/quant_ops/ops/quantization/flatquant/ops.py:78-130``) on CPU tensors with
the same torch operations in the same order, because the fallback's results are
defined by *where* it rounds to the input dtype D:

1. ``Z = rnd_D(X @ R)`` per token, X = row viewed as [M, N]   (ops.py:100-101)
2. ``Y = rnd_D(L^T @ Z)``                                      (ops.py:102)
3. ``xmax = amax(Y)``, ``xmin = amin(Y)`` per token            (ops.py:108-109)
4. ``a = max(|rnd_D(xmin * c)|, rnd_D(xmax * c))`` (c as float32)  (ops.py:112)
5. ``s = max(rnd_D(a / 7), rnd_D(1e-8))``                       (ops.py:113)
6. ``q = clamp(round_half_even(rnd_D(Y / s)), -8, 7)``          (ops.py:117)
7. int8 codes, or 8 codes per int32 word: ``sum_i (q_i + 8) << 4i``
                                                               (ops.py:119-130)

The scale is returned in D with shape [T] (the fallback's dtype; the GPU op
returns the same values as float32). ``dequantize_int4`` follows ops.py:156-178.
"""
import numpy as np
import torch

from .int4_reference import pack_int4_to_int32, unpack_int32_to_int4


def flatquant_pytorch(x, left, right, clip_ratio=1.0, pack_int32=False):
    """CPU restatement of ``flatquant_pytorch`` (flatquant/ops.py:78-130)."""
    tokens, feats = x.shape
    m, n = left.shape[0], right.shape[0]
    blocks = x.reshape(-1, m, n)
    z = torch.matmul(blocks, right)          # rounding point 1
    y = torch.matmul(left.T, z)              # rounding point 2
    y = y.reshape(tokens, feats)

    hi = y.amax(dim=1, keepdim=True)
    lo = y.amin(dim=1, keepdim=True)
    bound = torch.maximum((lo * clip_ratio).abs(), hi * clip_ratio)
    scale = (bound / 7.0).clamp(min=1e-8).squeeze(1)

    codes = torch.round(y / scale.view(-1, 1).expand_as(y)).clamp(-8, 7)
    if not pack_int32:
        return codes.to(torch.int8), scale
    offs = (codes + 8).to(torch.uint8).view(tokens, feats // 8, 8)
    word = torch.zeros(tokens, feats // 8, dtype=torch.int32, device=x.device)
    for i in range(8):
        word += offs[:, :, i].to(torch.int32) << (4 * i)
    return word, scale


def dequantize_int4(quantized, scales, packed_int32=False):
    """CPU restatement of ``dequantize_int4`` (flatquant/ops.py:156-178).

    Returns float32 ``float(q) * scale[token]``; with ``packed_int32`` the codes
    are first unpacked (nibble i of word p -> column 8p+i, value nibble-8).
    """
    q = quantized
    if packed_int32:
        q = torch.from_numpy(unpack_int32_to_int4(quantized.cpu().numpy()))
    return q.float() * scales.view(-1, 1).expand_as(q)


def flatquant_sequential(x, left, right, clip_ratio=1.0, pack_int32=False):
    """The fallback with its two GEMMs pinned to sequential float32 accumulation.

    ``flatquant_pytorch`` inherits the host BLAS's summation order: torch's CPU
    half/bfloat16 GEMM accumulates k = 0, 1, 2, ... in float32 on the Intel
    AVX-512 host this suite is developed on (bit-identical to this function),
    while on an AMD EPYC host the first product uses four interleaved float32
    accumulators (k mod 4). This variant fixes the order (products of D values
    are exact in float32, so each step is one float32 rounding) and then applies
    the fallback's scale/quantize steps unchanged, giving a host-independent
    reference for the kernels' rounding points.
    """
    tokens, feats = x.shape
    m, n = left.shape[0], right.shape[0]
    dt = x.dtype
    xb = x.reshape(-1, m, n).float()
    rf, lf = right.float(), left.float()
    acc = torch.zeros(xb.shape[0], m, n, dtype=torch.float32)
    for k in range(n):
        acc = acc + xb[:, :, k:k + 1] * rf[k:k + 1, :]
    z = acc.to(dt).float()
    acc = torch.zeros_like(acc)
    for k in range(m):
        acc = acc + lf[k].view(1, m, 1) * z[:, k:k + 1, :]
    y = acc.to(dt).reshape(tokens, feats)
    hi = y.amax(dim=1, keepdim=True)
    lo = y.amin(dim=1, keepdim=True)
    scale = (torch.maximum((lo * clip_ratio).abs(), hi * clip_ratio) / 7.0).clamp(min=1e-8).squeeze(1)
    codes = torch.round(y / scale.view(-1, 1).expand_as(y)).clamp(-8, 7)
    if not pack_int32:
        return codes.to(torch.int8), scale
    return torch.from_numpy(pack_int4_to_int32(codes.to(torch.int8).numpy())), scale


# ---------------------------------------------------------------------------
# Independent restatements used to PIN the oracle (never the thing measured).
# ---------------------------------------------------------------------------

def kron_transform_f64(x, left, right) -> np.ndarray:
    """Brute force ``y_row = x_row @ kron(L, R)`` in float64.

    With X = row viewed as [M, N] (f = m*N + n): ``(L^T X R)[i, j] =
    sum_{m, n} L[m, i] X[m, n] R[n, j]`` = ``x @ kron(L, R)`` column ``i*N + j``.
    """
    xd = np.asarray(x, dtype=np.float64)
    return xd @ np.kron(np.asarray(left, dtype=np.float64), np.asarray(right, dtype=np.float64))


def _rnd(v, dtype):
    """Round float64/float32 numpy values to ``dtype`` (RNE) and back to float64."""
    t = torch.from_numpy(np.asarray(v, dtype=np.float32))
    return t.to(dtype).double().numpy()


def quantize_rows_closed_form(y_d: np.ndarray, dtype, clip_ratio: float):
    """Scale + codes from already D-rounded rows ``y_d`` (float64 holding D values).

    Closed form of steps 3-6 with every rounding written out: products and the
    quotient in float32, each result rounded to D, ``round`` half to even.
    Returns (scale as float64 D values [T], codes int64 [T, F]).
    """
    c32 = np.float32(clip_ratio)
    hi = y_d.max(axis=1).astype(np.float32)
    lo = y_d.min(axis=1).astype(np.float32)
    t_lo = _rnd(lo * c32, dtype)
    t_hi = _rnd(hi * c32, dtype)
    bound = np.maximum(np.abs(t_lo), t_hi).astype(np.float32)
    s = _rnd(bound / np.float32(7.0), dtype)
    floor = _rnd(np.float32(1e-8), dtype)
    s = np.maximum(s, floor)
    with np.errstate(divide="ignore", invalid="ignore"):
        quo = _rnd(y_d.astype(np.float32) / s.astype(np.float32)[:, None], dtype)
    q = np.clip(np.round(quo), -8, 7)       # numpy rounds half to even
    return s, q
