"""Seeded synthetic inputs for the benchmark configurations of this hot path.

Everything is generated on the CPU with ``torch.Generator().manual_seed`` so a
kernel and its CPU checker see identical bits; callers move tensors to the GPU.

Configurations (shapes of the reference's own usage: hidden 4096 with 64 x 64
transforms, Llama-3-8B FFN width 14336 with 112 x 128):

* ``quant_cfg1`` fp32 X [128, 4096], M = N = 64, clip 1.0, int8 codes
* ``quant_cfg2`` fp16 X [2048, 4096], 1 % of channels x20, M = N = 64, clip 0.9, packed
* ``quant_cfg3`` bf16 X [8192, 14336], 0.5 % of channels x30, M = 112, N = 128, clip 1.0, packed
* ``gemm_cfg4``  A [4096, 4096/8], B [4096/8, 14336] uniform codes, fp16 scales
* ``linear_cfg5`` bf16 X [T, 14336] -> quantize (112 x 128, clip 0.9) -> GEMM
  against W [4096, 14336] packed and passed as ``W.t()``, bf16 out.
"""
from dataclasses import dataclass
from typing import Optional

import torch


def orthogonal(n: int, seed: int, dtype=torch.float32) -> torch.Tensor:
    """Q of the QR factorisation of a seeded N(0, 1) n x n matrix, cast to ``dtype``.

    The factorisation runs in float64: LAPACK builds on different host CPUs
    return float32 Q factors that differ in the last bits, which after the cast
    to fp16 changed 26 of 4096 entries of a 64 x 64 Q between this container
    and a GPU box host. In float64 those differences are far below the rounding
    of the cast, so every host builds the same transforms.
    """
    g = torch.Generator().manual_seed(seed)
    a = torch.randn(n, n, generator=g, dtype=torch.float32).double()
    q, _ = torch.linalg.qr(a)
    return q.to(dtype).contiguous()      # QR returns Q column-major


def gaussian_transforms(m: int, n: int, dtype, seed: int):
    """Non-orthogonal N(0, 1) transforms L [m, m] and R [n, n] in ``dtype``, as the
    reference's own tests build them (tests/test_performance.py:28-37,
    tests/test_accuracy.py:38-40)."""
    g = torch.Generator().manual_seed(seed)
    left = torch.randn(m, m, generator=g, dtype=torch.float32).to(dtype)
    right = torch.randn(n, n, generator=g, dtype=torch.float32).to(dtype)
    return left, right


def activations(tokens: int, features: int, dtype, seed: int, outlier_frac: float = 0.0,
                outlier_scale: float = 1.0) -> torch.Tensor:
    """N(0, 1) rows with a seeded ``ceil(frac * F)`` channels scaled by ``outlier_scale``."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(tokens, features, generator=g, dtype=torch.float32)
    if outlier_frac > 0:
        k = int(-(-outlier_frac * features // 1))
        idx = torch.randperm(features, generator=g)[:k]
        x[:, idx] *= outlier_scale
    return x.to(dtype)


def random_packed(rows: int, words: int, seed: int) -> torch.Tensor:
    """int32 [rows, words] with every nibble uniform in 0..15 (codes uniform in [-8, 7])."""
    g = torch.Generator().manual_seed(seed)
    w = torch.randint(0, 2**32, (rows, words), generator=g, dtype=torch.int64)
    return torch.where(w >= 2**31, w - 2**32, w).to(torch.int32)


def uniform(n: int, lo: float, hi: float, seed: int, dtype=torch.float16) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return (lo + (hi - lo) * torch.rand(n, generator=g, dtype=torch.float32)).to(dtype)


@dataclass
class QuantCase:
    name: str
    x: torch.Tensor
    left: torch.Tensor
    right: torch.Tensor
    clip_ratio: float
    pack_int32: bool

    @property
    def tokens(self):
        return self.x.shape[0]

    @property
    def features(self):
        return self.x.shape[1]

    def algorithmic_bytes(self, scale_bytes: int = 4) -> int:
        """HBM bytes one call must move: X in, codes out, scales out, L and R in."""
        t, f = self.x.shape
        es = self.x.element_size()
        codes = t * f // 2 if self.pack_int32 else t * f
        return t * f * es + codes + t * scale_bytes + (self.left.numel() + self.right.numel()) * es

    def flops(self) -> int:
        m, n = self.left.shape[0], self.right.shape[0]
        return 2 * self.tokens * m * n * (m + n)


def quant_case(name: str, tokens: int, m: int, n: int, dtype, clip: float, pack: bool, seed: int = 0,
               outlier_frac: float = 0.0, outlier_scale: float = 1.0) -> QuantCase:
    x = activations(tokens, m * n, dtype, seed, outlier_frac, outlier_scale)
    return QuantCase(name, x, orthogonal(m, seed + 1, dtype), orthogonal(n, seed + 2, dtype), clip, pack)


def reference_test_case(tokens: int, features: int, dtype, clip: float = 1.0, pack: bool = False,
                        seed: int = 42) -> QuantCase:
    """The reference tests' inputs: X ~ N(0, 1) [tokens, features] in ``dtype``, the
    Kronecker dims from ``get_decompose_dim`` and N(0, 1) (non-orthogonal) L and R
    in ``dtype`` (tests/test_performance.py:28-37,215-251)."""
    from .decompose import get_decompose_dim

    m, n = get_decompose_dim(features)
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(tokens, features, generator=g, dtype=torch.float32).to(dtype)
    left, right = gaussian_transforms(m, n, dtype, seed + 1)
    return QuantCase(f"ref_{tokens}x{features}_{str(dtype)[6:]}_{m}x{n}", x, left, right, clip, pack)


def quant_cfg1(tokens: int = 128, seed: int = 0) -> QuantCase:
    return quant_case("cfg1_fp32_128x4096_64x64", tokens, 64, 64, torch.float32, 1.0, False, seed)


def quant_cfg2(tokens: int = 2048, seed: int = 0) -> QuantCase:
    return quant_case("cfg2_fp16_2048x4096_64x64", tokens, 64, 64, torch.float16, 0.9, True, seed, 0.01, 20.0)


def quant_cfg3(tokens: int = 8192, seed: int = 0) -> QuantCase:
    return quant_case("cfg3_bf16_8192x14336_112x128", tokens, 112, 128, torch.bfloat16, 1.0, True, seed,
                      0.005, 30.0)


@dataclass
class GemmCase:
    name: str
    a: torch.Tensor        # int32 [M, K/8]
    b: torch.Tensor        # int32 [K/8, N] (row-major, or the W.t() view)
    scale_a: torch.Tensor  # [M]
    scale_b: torch.Tensor  # [N]
    out_dtype: torch.dtype = torch.float16

    @property
    def mnk(self):
        return self.a.shape[0], self.b.shape[1], self.a.shape[1] * 8

    def ops(self) -> int:
        m, n, k = self.mnk
        return 2 * m * n * k

    def algorithmic_bytes(self) -> int:
        m, n, k = self.mnk
        osz = torch.empty((), dtype=self.out_dtype).element_size()
        return (m * k + k * n) // 2 + m * self.scale_a.element_size() + n * self.scale_b.element_size() + m * n * osz


def gemm_case(m: int, n: int, k: int, seed: int = 0, b_transposed_view: bool = False,
              out_dtype=torch.float16, name: Optional[str] = None) -> GemmCase:
    a = random_packed(m, k // 8, seed)
    if b_transposed_view:
        b = random_packed(n, k // 8, seed + 1).t()          # W.t() of a [N, K/8] weight
    else:
        b = random_packed(k // 8, n, seed + 1)              # row-major [K/8, N]
    sa = uniform(m, 0.01, 0.1, seed + 2)
    sb = uniform(n, 0.001, 0.01, seed + 3)
    return GemmCase(name or f"gemm_{m}x{n}x{k}", a, b, sa, sb, out_dtype)


def gemm_cfg4(seed: int = 0) -> GemmCase:
    return gemm_case(4096, 14336, 4096, seed, name="cfg4_gemm_4096x14336x4096")
