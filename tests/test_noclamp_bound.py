"""CPU check of the bound behind the quantize kernels' unclamped bf16 code form.

fq_few2_kernel skips the upper clamp of bf16 codes when clip >= 0.95
(kNoClampClip in quant_ops_amd/csrc/flatquant_quant.hip): no quotient
y * (1 / s) can then round to bf16 7.5 or above, so round-half-even of it is
at most 7. The kernel's arithmetic for the largest |y| of a token (amax, a
bf16 value) is: bound = rnd(amax * clip), s = max(rnd(bound / 7), rnd(1e-8)),
rcp = fl(1 / s), u = fl(amax * rcp), all float32 with rnd() to bf16. Every
other |y| gives a smaller u. This test runs that arithmetic for every positive
finite bf16 amax at clip ratios from 0.95 up, and shows that at clip 0.93 the
bound fails (so the check can fail).
"""
import torch


def _bf16(x):
    return x.to(torch.bfloat16).to(torch.float32)


def _all_positive_bf16():
    bits = torch.arange(1, 0x7F80, dtype=torch.int32)            # +denormals .. largest finite
    return (bits << 16).view(torch.float32)


def _largest_rounded_quotient(amax, clip):
    c = torch.tensor(clip, dtype=torch.float32)
    bound = _bf16(amax * c)
    s = torch.maximum(_bf16(bound / torch.tensor(7.0)), _bf16(torch.tensor(1e-8)))
    rcp = torch.tensor(1.0, dtype=torch.float32) / s
    return _bf16(amax * rcp)


def test_every_bf16_amax_stays_below_7_5_from_clip_0_95():
    amax = _all_positive_bf16()
    for clip in (0.95, 0.951, 0.97, 0.99, 1.0, 1.25, 2.0, 10.0):
        t = _largest_rounded_quotient(amax, clip)
        assert torch.isfinite(t).all()
        assert float(t.max()) < 7.5, f"clip {clip}: {float(t.max())}"


def test_the_check_fails_below_the_bound():
    amax = _all_positive_bf16()
    t = _largest_rounded_quotient(amax, 0.93)
    assert float(t.max()) >= 7.5
