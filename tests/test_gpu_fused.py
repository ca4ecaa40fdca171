"""GPU parity of the fused hot-path kernels against the fp32 CPU oracle.

Tolerance (north star): max|a-b| / max|b| <= 2e-2 for the bf16 kernels,
with relative L2 reported beside it.  Cases mirror the reference's matrices
(tests/test_operator_additions.py:60-68,77-81,117-124): sizes around tile
boundaries, masks zero / ones / partial / fractional, both directions.
"""

import copy

import pytest
import torch
import torch.nn.functional as F

from boltz_lumi_amd import ops
from oracle import boltz_ref as R

pytestmark = pytest.mark.gpu

TOL = 2e-2


def errors(got, want):
    got, want = got.double().cpu(), want.double().cpu()
    d = got - want
    return {
        "max_rel": (d.abs().max() / want.abs().max().clamp_min(1e-30)).item(),
        "rel_l2": (d.norm() / want.norm().clamp_min(1e-30)).item(),
        "max_abs": d.abs().max().item(),
    }


def make_mask(kind, n, g):
    mask = torch.ones(1, n, n)
    if kind == "zero":
        mask.zero_()
    elif kind == "partial":
        mask[:, -3:, :] = 0
        mask[:, :, -3:] = 0
    elif kind == "fractional":
        mask = torch.rand(1, n, n, generator=g)
    elif kind == "tokens":
        keep = (torch.rand(n, generator=g) > 0.1).float()
        mask = (keep[:, None] * keep[None, :])[None]
    return mask


@pytest.mark.parametrize("outgoing", [True, False])
@pytest.mark.parametrize("n,kind", [(7, "ones"), (117, "partial"), (130, "fractional"), (256, "tokens"),
                                    (64, "zero")])
def test_trimul_matches_oracle(gpu, outgoing, n, kind):
    g = torch.Generator().manual_seed(732991 + n)
    cls = R.TriangleMultiplicationOutgoing if outgoing else R.TriangleMultiplicationIncoming
    m = R.randomize(cls(128), generator=g)
    x = torch.randn(1, n, n, 128, generator=g)
    mask = make_mask(kind, n, g)
    with torch.no_grad():
        want = m(x, mask)[0]
    md = m.to(gpu)
    with torch.inference_mode():
        got = ops.trimul(md, x[0].to(gpu), mask[0].to(gpu), outgoing)
        got32 = ops.trimul(md, x[0].to(gpu), mask[0].to(gpu), outgoing, out_mode=ops.OUT_F32)
        z = x[0].to(gpu).clone()
        ops.trimul(md, z, mask[0].to(gpu), outgoing, out_mode=ops.OUT_ACCUMULATE, out=z)
    e = errors(got, want)
    assert got.dtype == torch.bfloat16 and e["max_rel"] < TOL, e
    assert errors(got32, want)["max_rel"] < TOL
    assert errors(z, x[0] + got.float().cpu())["max_abs"] < 1e-5  # residual adds the bf16-rounded output


@pytest.mark.parametrize("starting", [True, False])
@pytest.mark.parametrize("n,kind", [(7, "ones"), (64, "partial"), (130, "tokens"), (200, "fractional"),
                                    (256, "ones")])
def test_triattn_matches_oracle(gpu, starting, n, kind):
    g = torch.Generator().manual_seed(17 + n)
    cls = R.TriangleAttention if starting else R.TriangleAttentionEndingNode
    m = R.randomize(cls(128, 32, 4), generator=g)
    x = torch.randn(1, n, n, 128, generator=g)
    mask = make_mask(kind, n, g)
    with torch.no_grad():
        want = m(x, mask)[0]
    md = m.to(gpu)
    with torch.inference_mode():
        got = ops.triattn(md, x[0].to(gpu), mask[0].to(gpu), starting)
        z = x[0].to(gpu).clone()
        ops.triattn(md, z, mask[0].to(gpu), starting, out_mode=ops.OUT_ACCUMULATE, out=z)
    e = errors(got, want)
    assert e["max_rel"] < TOL, e
    assert errors(z, x[0] + got.float().cpu())["max_abs"] < 1e-5


def test_triattn_fully_masked_rows_are_uniform(gpu):
    g = torch.Generator().manual_seed(5)
    m = R.randomize(R.TriangleAttention(128, 32, 4), generator=g)
    n = 96
    x = torch.randn(1, n, n, 128, generator=g) * 0.3
    mask = torch.ones(1, n, n)
    mask[:, -5:, :] = 0  # rows fully masked
    with torch.no_grad():
        want = m(x, mask)[0]
    with torch.inference_mode():
        got = ops.triattn(m.to(gpu), x[0].to(gpu), mask[0].to(gpu), True)
    assert torch.isfinite(got).all()
    assert errors(got, want)["max_rel"] < TOL


@pytest.mark.parametrize("rows", [1, 117, 128 * 5 + 3])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_pair_transition_matches_oracle(gpu, rows, dtype):
    g = torch.Generator().manual_seed(81 + rows)
    t = R.randomize(R.Transition(128, 512), std=0.05, generator=g)
    x = torch.randn(rows, 128, generator=g).to(dtype)
    with torch.no_grad():
        want = t(x.float())
    td = t.to(gpu)
    with torch.inference_mode():
        got = ops.pair_transition(td, x.to(gpu))
    e = errors(got, want)
    assert want.abs().max() > 0 and e["max_rel"] < TOL, e


@pytest.mark.parametrize("rows,mode", [(1, ops.OUT_RESIDUAL), (117, ops.OUT_ACCUMULATE),
                                       (128 * 5 + 3, ops.OUT_RESIDUAL), (128 * 8, ops.OUT_F32)])
def test_pair_transition_with_pair_bias(gpu, rows, mode):
    """The fused epilogue's pair bias equals the oracle's proj_z applied to
    the kernel's own fp32 output (LN + 128 -> 16 in fp32), and equals the
    stand-alone pair-bias kernel on that output; the transition output is
    bitwise the plain entry point's."""
    g = torch.Generator().manual_seed(17 + rows)
    t = R.randomize(R.Transition(128, 512), std=0.05, generator=g)
    apb = R.randomize(R.AttentionPairBias(384, 128, 16), generator=g)
    norm, lin = apb.proj_z[0], apb.proj_z[1]
    x = torch.randn(rows, 128, generator=g)
    td, nd, ld = t.to(gpu), copy.deepcopy(norm).to(gpu), copy.deepcopy(lin).to(gpu)
    xd = x.to(gpu)
    with torch.inference_mode():
        plain_out = xd.clone()
        plain = ops.pair_transition(td, plain_out if mode == ops.OUT_ACCUMULATE else xd, mode,
                                    plain_out if mode == ops.OUT_ACCUMULATE else None)
        out = xd.clone() if mode == ops.OUT_ACCUMULATE else torch.empty_like(xd)
        bias = torch.empty(16, rows, device=gpu)
        got = ops.pair_transition(td, out if mode == ops.OUT_ACCUMULATE else xd, mode, out, pair_bias=(nd, ld, bias))
        alone = ops.pair_bias(nd, ld, got.view(rows, 1, 128)).view(16, rows)
    assert torch.equal(got, plain)
    with torch.no_grad():
        want = lin(norm(got.cpu())).t()  # oracle proj_z on the kernel's output, [16, rows]
    assert (bias.cpu() - want).abs().max() / want.abs().max() < 1e-5  # fp32 epilogue
    assert (bias - alone).abs().max() / alone.abs().max() < 1e-5


@pytest.mark.parametrize("rows,cols", [(32, 16), (1024, 128), (128, 512)])
def test_pack_mfma_weights_layout(gpu, rows, cols):
    """Element (r, c) of the packed copy sits at ((r/32 * cols/16 + c/16) * 64
    + 32 * ((c%16)/8) + r%32) * 8 + c%8: checked by placing every element by
    that formula on the CPU."""
    w = torch.arange(rows * cols, dtype=torch.float32).reshape(rows, cols) % 251
    want = torch.empty(rows * cols)
    r = torch.arange(rows)[:, None].expand(rows, cols)
    c = torch.arange(cols)[None, :].expand(rows, cols)
    lane = 32 * ((c % 16) // 8) + r % 32
    want[(((r // 32) * (cols // 16) + c // 16) * 64 + lane) * 8 + c % 8] = w
    got = ops.pack_mfma_weights(w.to(gpu)).float().cpu().flatten()
    assert torch.equal(got, want)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_adaln_modulate_matches_oracle(gpu, dtype):
    g = torch.Generator().manual_seed(3)
    m = R.randomize(R.AdaLN(768, 768), generator=g)
    a = torch.randn(2, 300, 768, generator=g)
    s = torch.randn(2, 300, 768, generator=g)
    with torch.no_grad():
        want = m(a, s)
        sn = m.s_norm(s)
        scale, shift = m.s_scale(sn), m.s_bias(sn)
    with torch.inference_mode():
        got = ops.adaln_modulate(a.to(dtype).to(gpu), scale.to(dtype).to(gpu), shift.to(dtype).to(gpu), 1e-5)
    assert errors(got, want)["max_rel"] < (1e-5 if dtype == torch.float32 else TOL)


@pytest.mark.parametrize("dim", [4, 100, 128, 132, 256, 1024])
def test_adaln_modulate_widths_and_ragged_rows(gpu, dim):
    """Both row layouts of bmx_adaln (a half-wave per row up to 128 channels,
    a wave per row above) at widths that leave lanes or whole chunks idle,
    with a row count that ends inside a block; fp32 against the eager
    expression sigmoid(scale) * LN(a) + shift."""
    g = torch.Generator().manual_seed(dim)
    rows = 37
    a, scale, shift = (torch.randn(rows, dim, generator=g) for _ in range(3))
    want = torch.sigmoid(scale) * F.layer_norm(a, (dim,), eps=1e-5) + shift
    with torch.inference_mode():
        got = ops.adaln_modulate(a.to(gpu), scale.to(gpu), shift.to(gpu), 1e-5)
    assert errors(got, want)["max_rel"] < 1e-5


@pytest.mark.parametrize("m,k,n,bias", [(37, 768, 3072, False), (1024, 384, 1536, True), (41, 128, 256, True),
                                        (5, 1536, 768, False)])
def test_linear_x3_is_near_fp32(gpu, m, k, n, bias):
    """One bf16 GEMM of the split activation [xh | xh | xl] against the split
    weight [Wh | Wl | Wh] (fp32 accumulation) against the fp64 product: the
    dropped xl Wl term and the residues below the low parts leave about 2^-16
    relative per product, far inside the fp32-mode tolerance of 1e-4."""
    g = torch.Generator().manual_seed(m + k)
    lin = torch.nn.Linear(k, n, bias=bias)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(n, k, generator=g) * 0.05)
        if bias:
            lin.bias.copy_(torch.randn(n, generator=g))
    x = torch.randn(2, m, k, generator=g)
    want = torch.nn.functional.linear(x.double(), lin.weight.double(), None if not bias else lin.bias.double())
    lin = lin.to(gpu)
    with torch.inference_mode():
        got = ops.linear_x3(x.to(gpu), lin)
        split = ops.split3(x[0].to(gpu).contiguous())
    assert got.dtype == torch.float32 and got.shape == want.shape
    assert errors(got, want)["max_rel"] < 2e-5
    hi = x[0].bfloat16()
    split = split.cpu()
    assert split.shape == (m, 3 * k + 64)
    assert torch.equal(split[:, :k], hi) and torch.equal(split[:, k:2 * k], hi)
    assert torch.equal(split[:, 2 * k:3 * k], (x[0] - hi.float()).bfloat16())
    assert (split[:, 3 * k:3 * k + 2] == 1).all() and (split[:, 3 * k + 2:] == 0).all()
