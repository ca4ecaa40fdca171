"""GPU parity of the reference operator set (norm, gate, split, pack,
silu_mul, epilogue, ordered_softmax) against textbook torch / oracle math.

Case matrices follow the reference's tests: sizes around wave / tile
boundaries, empty and singleton inputs, address offsets, strided masks, a
whole masked triangle slice, and a non-default stream
(tests/test_pair_transition.py:38-51,68-78; tests/test_triangle_softmax.py:25-47).
"""

import pytest
import torch
import torch.nn.functional as F

from boltz_lumi_amd import ops

pytestmark = pytest.mark.gpu


def rel(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).abs().max() / b.abs().max().clamp_min(1e-30)).item()


def bits_close(a, b, max_ulp_frac=1e-3):
    """bf16 results: fraction of elements that differ by more than one bf16 ulp."""
    a, b = a.float().cpu(), b.float().cpu()
    if b.numel() == 0:
        return a.numel() == 0
    ulp = b.abs().clamp_min(1e-30) * 2.0**-7
    return ((a - b).abs() > ulp * 1.01).float().mean().item() <= max_ulp_frac


@pytest.mark.parametrize("rows", [0, 1, 7, 129, 4096])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("channel_first", [False, True])
@pytest.mark.parametrize("bf16_output", [False, True])
def test_norm(gpu, rows, dtype, channel_first, bf16_output):
    g = torch.Generator().manual_seed(rows)
    x = (torch.randn(rows, 128, generator=g) * 2 + 0.5).to(dtype)
    w = torch.randn(128, generator=g) * 0.1 + 1
    b = torch.randn(128, generator=g) * 0.1
    want = F.layer_norm(x.float(), (128,), w, b, 1e-5)
    xin = (x.t().contiguous() if channel_first else x).to(gpu)
    with torch.inference_mode():
        got = ops.norm(xin, w.to(gpu), b.to(gpu), 1e-5, channel_first, bf16_output=bf16_output)
    assert got.shape == (rows, 128)
    assert got.dtype == (torch.bfloat16 if bf16_output else torch.float32)
    if rows:
        tol = 1e-2 if bf16_output else 1e-5
        assert rel(got, want) < tol


def test_norm_rejects_grad_mode(gpu):
    x = torch.randn(4, 128, device=gpu)
    w, b = torch.ones(128, device=gpu), torch.zeros(128, device=gpu)
    with torch.enable_grad(), pytest.raises(RuntimeError, match="Inference only"):
        ops.norm(x, w, b, 1e-5)


@pytest.mark.parametrize("size", [0, 1, 17, 257, 512, 513, 117 * 512, 312 * 512])  # the reference's sizes
@pytest.mark.parametrize("offset", [0, 1])
def test_silu_mul_and_gate(gpu, size, offset):
    g = torch.Generator().manual_seed(81 + size)
    a = (torch.randn(size + 2, generator=g) * 20).to(torch.bfloat16).to(gpu)
    b = torch.randn(size + 2, generator=g).to(torch.bfloat16).to(gpu)
    a_s, b_s = a[offset:offset + size], b[offset:offset + size]
    with torch.inference_mode():
        got = ops.silu_mul(a_s, b_s)
        want = F.silu(a_s) * b_s  # torch's bf16 ops round silu, then the product
        assert bits_close(got, want)
        got_g = ops.gate(a_s, b_s)
        want_g = a_s * torch.sigmoid(b_s)
        assert bits_close(got_g, want_g)


def test_silu_mul_non_default_stream(gpu):
    stream = torch.cuda.Stream()
    with torch.inference_mode(), torch.cuda.stream(stream):
        a = torch.randn(513, device=gpu, dtype=torch.bfloat16)
        b = torch.randn_like(a)
        want = F.silu(a) * b
        got = ops.silu_mul(a, b)
    stream.synchronize()
    assert bits_close(got, want)


@pytest.mark.parametrize("n", [7, 117, 130, 136])  # 136: 16-byte segment stores, then a ragged tail
@pytest.mark.parametrize("joint", [False, True])
def test_split_and_pack(gpu, n, joint):
    g = torch.Generator().manual_seed(n)
    width = 512 if joint else 256
    pg = (torch.randn(1, n, n, width, generator=g)).to(torch.bfloat16).to(gpu)
    gg = (torch.randn(1, n, n, width, generator=g)).to(torch.bfloat16).to(gpu)
    p, gt = pg[..., :256], gg[..., :256]
    mask = torch.rand(1, n, n, generator=g).to(gpu)
    with torch.inference_mode():
        h = (p * torch.sigmoid(gt)) * mask[..., None]
        a_ref, b_ref = h[..., :128].to(torch.bfloat16), h[..., 128:].to(torch.bfloat16)
        a, b = ops.split(p, gt, mask)
        assert bits_close(a, a_ref) and bits_close(b, b_ref)
        for outgoing in (True, False):
            left, right = ops.pack(p, gt, mask, outgoing)
            if outgoing:
                want_l, want_r = a_ref.permute(0, 3, 1, 2), b_ref.permute(0, 3, 2, 1)
            else:
                want_l, want_r = a_ref.permute(0, 3, 2, 1), b_ref.permute(0, 3, 1, 2)
            assert torch.equal(left, want_l.reshape(128, n, n))
            assert torch.equal(right, want_r.reshape(128, n, n))


@pytest.mark.parametrize("outgoing", [True, False])
def test_pack_into_unaligned_operands(gpu, outgoing):
    """The ABI asks 16-byte alignment of p and g only: operands that start one
    element into a buffer (2-byte aligned) take element stores and hold the
    same values as 16-byte-aligned ones (n = 136 would take 16-byte segment
    stores)."""
    from boltz_lumi_amd import _native as N

    n = 136
    g = torch.Generator().manual_seed(11)
    p = torch.randn(1, n, n, 256, generator=g).to(torch.bfloat16).to(gpu)
    gt = torch.randn(1, n, n, 256, generator=g).to(torch.bfloat16).to(gpu)
    mask = torch.rand(1, n, n, generator=g).to(gpu)
    with torch.inference_mode():
        want_a, want_b = ops.pack(p, gt, mask, outgoing)
        buf = torch.full((2, 128 * n * n + 8), -7.0, device=gpu, dtype=torch.bfloat16)
        a, b = buf[0, 1:1 + 128 * n * n], buf[1, 1:1 + 128 * n * n]
        assert a.data_ptr() % 16 == 2 and b.data_ptr() % 16 == 2
        N.call("bmx_trimul_pack", p.data_ptr(), gt.data_ptr(), mask.data_ptr(), a.data_ptr(), b.data_ptr(), n, 256,
               int(outgoing), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(a.view(128, n, n), want_a) and torch.equal(b.view(128, n, n), want_b)
    assert (buf[:, 0] == -7.0).all() and (buf[:, 1 + 128 * n * n:] == -7.0).all()  # nothing written outside


@pytest.mark.parametrize("kind", [ops.MODULATION, ops.GATE, ops.GATED_SWIGLU])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_epilogue(gpu, kind, dtype):
    g = torch.Generator().manual_seed(kind)
    rows, cols = 37, 768
    a = torch.randn(rows, 2 * cols if kind == ops.GATED_SWIGLU else cols, generator=g)
    b = torch.randn(rows, cols, generator=g)
    c = torch.randn(rows, cols, generator=g)
    if kind == ops.MODULATION:
        want = torch.sigmoid(b) * a + c
    elif kind == ops.GATE:
        want = torch.sigmoid(a) * b
    else:
        want = F.silu(a[:, cols:]) * a[:, :cols] * b
    with torch.inference_mode():
        got = ops.epilogue(a.to(dtype).to(gpu), b.to(dtype).to(gpu), c.to(dtype).to(gpu), kind)
    assert rel(got, want) < (1e-5 if dtype == torch.float32 else 2e-2)


_SOFTMAX_KEYS = [117, 129, 257, 312, 512, 513, 576, 1023, 1024, 1134, 1734, 2511]


@pytest.mark.parametrize("n,dtype", [(n, torch.bfloat16) for n in _SOFTMAX_KEYS]
                         + [(n, torch.float32) for n in _SOFTMAX_KEYS if n <= 1024])
def test_ordered_softmax(gpu, n, dtype):
    """The reference's recipe: s += mask; s += bias; softmax (fp32 inside), at
    the reference test's key counts (fp32 up to 1024, as there)."""
    g = torch.Generator().manual_seed(46 + n)
    scores = (torch.randn(1, 3, 4, n, n, generator=g) * 5).to(dtype).to(gpu)
    bias = (torch.randn(1, 1, 4, n, n, generator=g) * 2).to(dtype).to(gpu)
    mask = torch.zeros(1, n, 1, 1, 3, device=gpu).transpose(1, 4)  # strided mask
    mask[..., -3:] = -1e9
    mask[:, 1] = -1e9  # a whole triangle slice
    with torch.inference_mode():
        ref = scores.clone()
        ref += mask
        ref += bias
        want = torch.softmax(ref.float(), -1)
        got = ops.ordered_softmax(scores, bias, mask)
    assert got.dtype == dtype
    assert rel(got, want) < (1e-5 if dtype == torch.float32 else 1e-2)
    assert torch.isfinite(got).all()
