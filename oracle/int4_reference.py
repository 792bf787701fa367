"""Oracle for int4 packing and the W4A4 GEMM — test infrastructure only.

Integer work is done in numpy (exact), float work with the same torch CPU ops
as the reference fallback so that rounding is the fallback's rounding.

* pack / unpack: ``src/quant_ops/ops/quantization/int4_matmul/ops.py:23-66``
  (same format as ``flatquant/ops.py:119-128`` and ``:164-172``): word ``p`` of a
  row holds the codes of columns ``8p .. 8p+7``, code ``i`` in bits ``4i .. 4i+3``
  as the offset value ``q + 8`` (0..15); the 32-bit sum wraps to int32.
* GEMM: ``int4_matmul_pytorch`` (``int4_matmul/ops.py:69-103``): unpack, float32
  matmul (exact for integer sums below 2**24), multiply by ``scale_a[m]``, then by
  ``scale_b[n]`` (both promoted to float32), and round to float16.
"""
import numpy as np
import torch


def pack_int4_to_int32(codes) -> np.ndarray:
    """Pack int8 codes of shape [rows, F] (F % 8 == 0) to int32 [rows, F/8].

    Reference: ``int4_matmul/ops.py:23-45``: ``(tensor + 8).to(torch.uint8)``
    keeps the low 8 bits of code + 8 (the int8 add wraps, the cast takes the
    value mod 256), and the shifted int32 sum wraps mod 2^32. For codes in
    [-8, 7] that is code + 8 in nibble i of the word.
    """
    q = np.asarray(codes).astype(np.int64)
    rows, feats = q.shape
    if feats % 8:
        raise ValueError(f"features ({feats}) must be divisible by 8")
    u = ((q + 8) & 0xFF).astype(np.uint64).reshape(rows, feats // 8, 8)
    shifts = (np.arange(8, dtype=np.uint64) * np.uint64(4))
    word = (u << shifts).sum(axis=2) & np.uint64(0xFFFFFFFF)
    return word.astype(np.uint32).view(np.int32)


def unpack_int32_to_int4(packed) -> np.ndarray:
    """Inverse of :func:`pack_int4_to_int32`: int32 [rows, W] -> int8 [rows, 8W].

    Reference: ``int4_matmul/ops.py:48-66`` (nibble ``i`` of word ``p`` is column
    ``8p + i``, value ``nibble - 8``).
    """
    w = np.asarray(packed).astype(np.int32).view(np.uint32).astype(np.uint64)
    rows, words = w.shape
    shifts = (np.arange(8, dtype=np.uint64) * np.uint64(4))
    nib = (w[:, :, None] >> shifts) & np.uint64(0xF)
    return (nib.astype(np.int16) - 8).astype(np.int8).reshape(rows, words * 8)


def int4_gemm_int64(a_packed, b_packed) -> np.ndarray:
    """Exact int64 accumulators ``sum_k qa[m,k] * qb[k,n]``.

    ``a_packed`` is int32 [M, K/8] (K-packed rows); ``b_packed`` is int32
    [K/8, N] where word ``(p, n)`` holds ``k = 8p .. 8p+7`` of column ``n``
    (``examples/int4_matmul_benchmark.py:21-22`` packs it as ``pack(b.T).T``).
    Brute force for small shapes; used to pin :func:`int4_matmul_pytorch`.
    """
    qa = unpack_int32_to_int4(a_packed).astype(np.int64)
    qb = unpack_int32_to_int4(np.ascontiguousarray(np.asarray(b_packed).T)).astype(np.int64).T
    return qa @ qb


def int4_matmul_pytorch(a_packed, b_packed, scale_a, scale_b, out_dtype=torch.float16):
    """The reference fallback GEMM on CPU tensors (``int4_matmul/ops.py:69-103``).

    Returns ``half((float32(acc) * scale_a[m]) * scale_b[n])``; the scale
    tensors keep their dtype and are promoted by torch exactly as in the
    reference. ``out_dtype`` other than float16 is this build's documented
    extension (the reference always returns float16).
    """
    a = torch.as_tensor(a_packed).cpu()
    b = torch.as_tensor(b_packed).cpu()
    m, kp = a.shape
    n = b.shape[1]
    qa = torch.from_numpy(unpack_int32_to_int4(a.numpy())).float()
    qb = torch.from_numpy(unpack_int32_to_int4(b.T.contiguous().numpy())).T.float()
    acc = torch.matmul(qa.view(m, kp * 8), qb.reshape(kp * 8, n))
    out = acc * scale_a.cpu().view(m, 1) * scale_b.cpu().view(1, n)
    return out.to(out_dtype)


def int4_matmul_int32(a_packed, b_packed) -> torch.Tensor:
    """Integer accumulators as the fallback forms them (float32 matmul -> int32)."""
    a = torch.as_tensor(a_packed).cpu()
    b = torch.as_tensor(b_packed).cpu()
    m, kp = a.shape
    n = b.shape[1]
    qa = torch.from_numpy(unpack_int32_to_int4(a.numpy())).float()
    qb = torch.from_numpy(unpack_int32_to_int4(b.T.contiguous().numpy())).T.float()
    return torch.matmul(qa.view(m, kp * 8), qb.reshape(kp * 8, n)).to(torch.int32)
