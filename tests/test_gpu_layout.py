"""GPU parity of the layout kernels (pack / unpack of int4 codes, the packed
word transpose) and of the W4A4 linear layer, through the C ABI, against the
CPU oracle. Byte and word work, so the bar is bit-exact."""
import numpy as np
import pytest
import torch

import quant_ops_amd as qo
from quant_ops_amd import capi
from quant_ops_amd import workloads as wl
from oracle import fq_reference as ofq
from oracle import int4_reference as oi4

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-layout] {msg}", flush=True)


def _codes(rows, feats, seed, full_range=False):
    g = torch.Generator().manual_seed(seed)
    lo, hi = (-128, 128) if full_range else (-8, 8)
    return torch.randint(lo, hi, (rows, feats), generator=g, dtype=torch.int8)


def _words(rows, nwords, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(-2**31, 2**31, (rows, nwords), generator=g, dtype=torch.int64).to(torch.int32)


@pytest.mark.parametrize("rows,feats", [(1, 8), (3, 24), (5, 16), (64, 4096), (1024, 14336)])
@pytest.mark.parametrize("full_range", [False, True])
def test_pack_bit_exact(gpu, rows, feats, full_range):
    q = _codes(rows, feats, rows + feats, full_range)
    _say(f"pack {rows}x{feats} full_range={full_range}")
    w = capi.pack_int4_to_int32(q.to(gpu))
    torch.cuda.synchronize()
    assert w.dtype == torch.int32 and w.shape == (rows, feats // 8)
    assert np.array_equal(w.cpu().numpy(), oi4.pack_int4_to_int32(q.numpy()))


@pytest.mark.parametrize("offset", [0, 1, 16])
def test_pack_strided_and_misaligned_rows(gpu, offset):
    """Rows inside a wider buffer (row stride 4112 bytes), starting 0, 1 or 16
    bytes in: the 1-byte offset takes the byte-load path."""
    q = _codes(37, 4096, 5, True)
    big = torch.zeros(37, 4096 + 16, dtype=torch.int8)
    big[:, offset:offset + 4096] = q
    view = big.to(gpu)[:, offset:offset + 4096]
    out_big = torch.full((37, 600), 7, dtype=torch.int32, device=gpu)
    out = out_big[:, 3:3 + 512]
    _say(f"pack strided offset={offset}")
    capi.pack_int4_to_int32(view, out=out)
    torch.cuda.synchronize()
    ob = out_big.cpu()
    assert np.array_equal(ob[:, 3:515].numpy(), oi4.pack_int4_to_int32(q.numpy()))
    assert bool((ob[:, :3] == 7).all()) and bool((ob[:, 515:] == 7).all())   # nothing outside the view


@pytest.mark.parametrize("rows,nwords", [(1, 1), (3, 3), (7, 10), (64, 512), (2048, 1792)])
def test_unpack_bit_exact(gpu, rows, nwords):
    w = _words(rows, nwords, rows * 31 + nwords)
    _say(f"unpack {rows}x{nwords}")
    q = capi.unpack_int32_to_int4(w.to(gpu))
    torch.cuda.synchronize()
    assert q.dtype == torch.int8 and q.shape == (rows, 8 * nwords)
    assert np.array_equal(q.cpu().numpy(), oi4.unpack_int32_to_int4(w.numpy()))


def test_unpack_misaligned_output_and_round_trips(gpu):
    w = _words(9, 130, 77)
    out_big = torch.full((9, 8 * 130 + 40), 5, dtype=torch.int8, device=gpu)
    out = out_big[:, 3:3 + 8 * 130]
    _say("unpack misaligned output")
    capi.unpack_int32_to_int4(w.to(gpu)[:, :], out=out)
    torch.cuda.synchronize()
    ob = out_big.cpu()
    assert np.array_equal(ob[:, 3:3 + 1040].numpy(), oi4.unpack_int32_to_int4(w.numpy()))
    assert bool((ob[:, :3] == 5).all()) and bool((ob[:, 1043:] == 5).all())
    # pack(unpack(w)) == w for any word; unpack(pack(q)) == q for codes in [-8, 7]
    wg = w.to(gpu)
    assert torch.equal(capi.pack_int4_to_int32(capi.unpack_int32_to_int4(wg)), wg)
    q = _codes(33, 2048, 78).to(gpu)
    assert torch.equal(capi.unpack_int32_to_int4(capi.pack_int4_to_int32(q)), q)


@pytest.mark.parametrize("rows,cols", [(1, 1), (1, 100), (100, 1), (63, 65), (64, 64), (130, 257), (512, 14336)])
def test_transpose_bit_exact(gpu, rows, cols):
    w = _words(rows, cols, rows * 7 + cols)
    _say(f"transpose {rows}x{cols}")
    t = capi.transpose_int32(w.to(gpu))
    torch.cuda.synchronize()
    assert t.shape == (cols, rows) and torch.equal(t.cpu(), w.t().contiguous())


def test_transpose_strided_input_and_layout_conversion(gpu):
    w = _words(100, 300, 9)
    view = w.to(gpu)[:, 17:17 + 250]
    _say("transpose strided")
    t = capi.transpose_int32(view)
    assert torch.equal(t.cpu(), w[:, 17:267].t().contiguous())
    # [N, K/8] packing of W and the [K/8, N] packing of the same codes
    codes = _codes(300, 512, 10)                      # W [N, K]
    nk = qo.pack_int4_to_int32(codes.to(gpu))         # HIP pack, [N, K/8]
    kn = qo.transpose_packed(nk)                      # HIP transpose, [K/8, N]
    ref_kn = torch.from_numpy(oi4.pack_int4_to_int32(codes.numpy())).t().contiguous()
    assert torch.equal(kn.cpu(), ref_kn)
    assert torch.equal(qo.transpose_packed(kn), nk)
    assert torch.equal(qo.unpack_int32_to_int4(nk).cpu(), codes)


def test_layout_entry_points_reject_bad_sizes(gpu):
    q = torch.zeros(4, 12, dtype=torch.int8, device=gpu)
    with pytest.raises(capi.QuantOpsError, match="QO_ERR_SHAPE"):
        capi.pack_int4_to_int32(q, out=torch.empty(4, 2, dtype=torch.int32, device=gpu))


@pytest.mark.parametrize("tokens", [16, 300])
def test_w4a4_linear_gpu(gpu, tokens):
    """The linear on the GPU: quantize parity as for the kernel alone, GEMM and
    bias stage bit-exact given the kernel's own codes and scales."""
    m, n, out_f = 64, 64, 1024
    x = wl.activations(tokens, m * n, torch.bfloat16, seed=41, outlier_frac=0.01, outlier_scale=20.0)
    L, R = wl.orthogonal(m, 42, torch.bfloat16), wl.orthogonal(n, 43, torch.bfloat16)
    g = torch.Generator().manual_seed(44)
    wc = torch.randint(-8, 8, (out_f, m * n), generator=g, dtype=torch.int8)
    sw = wl.uniform(out_f, 0.001, 0.01, 45, torch.float32)
    bias = torch.randn(out_f, generator=g).to(torch.bfloat16)
    _say(f"w4a4 linear T={tokens}")
    wp = qo.prepare_w4a4_weight(wc.to(gpu))
    assert np.array_equal(wp.cpu().numpy(), oi4.pack_int4_to_int32(wc.numpy()))
    y = qo.w4a4_flatquant_linear(x.to(gpu), L.to(gpu), R.to(gpu), wp, sw.to(gpu), 0.9, bias.to(gpu))
    q, s = qo.flatquant_dynamic_quantize(x.to(gpu), L.to(gpu), R.to(gpu), 0.9, True)
    torch.cuda.synchronize()
    assert y.shape == (tokens, out_f) and y.dtype == torch.bfloat16
    q_ref, s_ref = ofq.flatquant_pytorch(x, L, R, 0.9, True)
    d = (torch.from_numpy(oi4.unpack_int32_to_int4(q.cpu().numpy())).int()
         - torch.from_numpy(oi4.unpack_int32_to_int4(q_ref.numpy())).int()).abs()
    assert int(d.max()) <= 1 and float((d != 0).float().mean()) <= 1e-3
    ref = oi4.int4_matmul_pytorch(q.cpu(), wp.cpu().t(), s.cpu(), sw, out_dtype=torch.bfloat16) + bias
    assert torch.equal(y.cpu(), ref)
