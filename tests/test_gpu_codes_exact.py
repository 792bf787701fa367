"""Codes at rounding ties, bit-exact: with permutation matrices as L and R
(orthogonal, each product a single term times 1.0) the transformed Y is an
exact permutation of X, so every rounding the kernels do before the codes is
exact and their codes and scales must equal the oracle's
(flatquant/ops.py:78-130) bit for bit, with no flip budget.

Each token holds one element of magnitude 7 (its absmax, so at clip 1.0 the
bf16 scale is exactly 1 and each quotient is the element itself) and draws
the rest from the values the code step must get right: every half-integer
tie in [-7, 7] (round half to even), their bf16 neighbours on both sides,
integers, zeros of both signs and tiny values. At clip 0.9 the same tokens
take the clamped bf16 code form (quotients up to 7 / 0.9), at clip 1.0 the
unclamped one; fp16 tokens at clip 1.0 take the fp16 form. The 64 x 64
shape runs the one-wave kernel, 112 x 128 and 64 x 128 the few-token kernel
(packed and int8 codes), at 300 tokens (one per workgroup) and 1200 (several
per workgroup: the staged code copies).
"""
import pytest
import torch

from quant_ops_amd import capi
from oracle import fq_reference as ofq

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-codes-exact] {msg}", flush=True)


def _tie_values(dtype):
    """Values of ``dtype`` in [-7, 7] around every rounding decision of the code step."""
    vals = []
    for k in range(-7, 7):
        h = torch.tensor(k + 0.5, dtype=dtype)
        bits = h.view(torch.int32 if dtype == torch.float32 else torch.int16)
        up = (bits + 1).view(dtype) if float(h) > 0 else (bits - 1).view(dtype)
        down = (bits - 1).view(dtype) if float(h) > 0 else (bits + 1).view(dtype)
        vals += [float(h), float(up), float(down), float(k)]
    tiny = 1e-7 if dtype == torch.float16 else 1e-30
    vals += [0.0, -0.0, 7.0, -7.0, tiny, -tiny, 6.96875, -6.96875]
    return torch.tensor(vals, dtype=torch.float32)


def _permutation(n, seed):
    g = torch.Generator().manual_seed(seed)
    p = torch.randperm(n, generator=g)
    return torch.eye(n)[p]


def _tokens(tokens, m, n, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    vals = _tie_values(dtype)
    idx = torch.randint(0, vals.numel(), (tokens, m * n), generator=g)
    x = vals[idx]
    # one element of magnitude 7 per token (either sign) fixes its absmax
    pos = torch.randint(0, m * n, (tokens,), generator=g)
    sign = torch.where(torch.rand(tokens, generator=g) < 0.5, -7.0, 7.0)
    x[torch.arange(tokens), pos] = sign
    if dtype == torch.bfloat16:
        x[tokens // 2].zero_()                  # an all-zero token (scale at its floor)
    return x.to(dtype)


@pytest.mark.parametrize("m,n,tokens,clip,pack", [
    (112, 128, 300, 1.0, True), (112, 128, 1200, 1.0, True), (112, 128, 300, 0.9, True),
    (112, 128, 1200, 0.9, True), (112, 128, 300, 0.9, False), (64, 128, 600, 1.0, True),
    (64, 128, 600, 0.9, True), (64, 64, 500, 1.0, True), (64, 64, 500, 0.9, True),
])
def test_codes_at_ties_bit_exact(gpu, m, n, tokens, clip, pack):
    _say(f"{tokens} x {m}x{n} bf16 clip={clip} pack={pack}")
    x = _tokens(tokens, m, n, seed=31 * m + n + tokens)
    left = _permutation(m, seed=m).to(torch.bfloat16)
    right = _permutation(n, seed=n + 1).to(torch.bfloat16)
    q, s = capi.flatquant_quantize(x.to(gpu), left.to(gpu), right.to(gpu), clip, pack)
    torch.cuda.synchronize()
    q_ref, s_ref = ofq.flatquant_pytorch(x, left, right, clip, pack)
    assert torch.equal(s.cpu(), s_ref.float()), "scales"
    if pack:
        assert torch.equal(q.cpu(), q_ref), "packed codes"
    else:
        assert torch.equal(q.cpu(), q_ref.to(q.dtype)), "int8 codes"


@pytest.mark.parametrize("m,n,tokens", [(64, 64, 2048), (112, 128, 300), (64, 128, 600)])
def test_fp16_codes_at_ties_bit_exact(gpu, m, n, tokens):
    """The fp16 code form (a packed add of 1536 + 8 rounds each quotient) at
    clip 1.0, where the fp16 scale of an absmax of 7 is exactly 1; config 2's
    shape and token count first. (The all-zero token is left out: its fp16
    scale floor rounds to 0, a case the other tests cover.)"""
    _say(f"{tokens} x {m}x{n} fp16 clip=1.0")
    x = _tokens(tokens, m, n, seed=17 * m + n + tokens, dtype=torch.float16)
    left = _permutation(m, seed=m + 5).to(torch.float16)
    right = _permutation(n, seed=n + 6).to(torch.float16)
    q, s = capi.flatquant_quantize(x.to(gpu), left.to(gpu), right.to(gpu), 1.0, True)
    torch.cuda.synchronize()
    q_ref, s_ref = ofq.flatquant_pytorch(x, left, right, 1.0, True)
    assert torch.equal(s.cpu(), s_ref.float()), "scales"
    assert torch.equal(q.cpu(), q_ref), "packed codes"


def test_fp32_int8_codes_at_ties_bit_exact(gpu):
    """fp32 inputs with int8 codes (config 1's dtype, layout and shape), clip 1.0."""
    m, n, tokens = 64, 64, 128
    _say(f"{tokens} x {m}x{n} fp32 clip=1.0 int8 codes")
    x = _tokens(tokens, m, n, seed=77, dtype=torch.float32)
    left, right = _permutation(m, seed=3), _permutation(n, seed=4)
    q, s = capi.flatquant_quantize(x.to(gpu), left.to(gpu), right.to(gpu), 1.0, False)
    torch.cuda.synchronize()
    q_ref, s_ref = ofq.flatquant_pytorch(x, left, right, 1.0, False)
    assert torch.equal(s.cpu(), s_ref.float()), "scales"
    assert torch.equal(q.cpu(), q_ref.to(q.dtype)), "int8 codes"
