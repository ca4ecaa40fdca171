"""Split-bf16 operand writers and the strided modulation kernels of the
diffusion transformer's near-fp32 linears.

Each writer is checked bit for bit against the fp32 kernel that computes the
same value (bmx_adaln, the GATED_SWIGLU / MODULATION epilogues) split by torch
into hi = bf16(v), lo = bf16(v - hi); the LayerNorm writer, which has no fp32
twin, against float64 LayerNorm.  The GEMM of an operand against a split
weight with its bias folded in is checked against the float64 linear.  Row
counts end inside a block; modulation operands are column slices of one wider
projection (rows at a stride), as the diffusion transformer's conditioning
precompute hands them over."""

import pytest
import torch
import torch.nn.functional as F

from boltz_lumi_amd import ops

pytestmark = pytest.mark.gpu


def split_of(v):
    v = v.float().cpu()
    hi = v.bfloat16()
    return hi, (v - hi.float()).bfloat16()


def check_operand(op, v):
    """``op`` [rows, 3 k + 64] holds [hi | hi | lo | 1 1 0 ...] of fp32 ``v``."""
    op = op.cpu()
    k = v.shape[-1]
    hi, lo = split_of(v)
    assert op.shape == v.shape[:-1] + (3 * k + 64,)
    assert torch.equal(op[..., :k], hi) and torch.equal(op[..., k:2 * k], hi)
    assert torch.equal(op[..., 2 * k:3 * k], lo)
    assert (op[..., 3 * k:3 * k + 2] == 1).all() and (op[..., 3 * k + 2:] == 0).all()


def wide(g, rows, cols, width, offset, gpu):
    """[rows, cols] column slice at ``offset`` of a [rows, width] projection."""
    full = torch.randn(rows, width, generator=g).to(gpu)
    return full[:, offset:offset + cols]


@pytest.mark.parametrize("rows,dim", [(37, 768), (5, 1024), (9, 384), (3, 4)])
def test_adaln_split3_matches_adaln(gpu, rows, dim):
    g = torch.Generator().manual_seed(rows + dim)
    a = torch.randn(rows, dim, generator=g).to(gpu)
    scale, shift = wide(g, rows, dim, 4 * dim, dim, gpu), wide(g, rows, dim, 4 * dim, 3 * dim, gpu)
    with torch.inference_mode():
        dense = ops.adaln_modulate(a, scale.contiguous(), shift.contiguous(), 1e-5)
        strided = ops.adaln_modulate(a, scale, shift, 1e-5)
        op = ops.adaln_split3(a, scale, shift, 1e-5)
    want = torch.sigmoid(scale.double()) * F.layer_norm(a.double(), (dim,), eps=1e-5) + shift.double()
    assert ((dense.double() - want).abs().max() / want.abs().max()).item() < 1e-5
    assert torch.equal(strided, dense)
    check_operand(op, dense)


@pytest.mark.parametrize("rows,dim", [(37, 768), (6, 1024), (3, 128)])
def test_layernorm_split3_matches_fp64(gpu, rows, dim):
    g = torch.Generator().manual_seed(dim)
    x = (torch.randn(rows, dim, generator=g) * 3 + 1).to(gpu)
    with torch.inference_mode():
        op = ops.layernorm_split3(x, 1e-5).cpu()
    want = F.layer_norm(x.double().cpu(), (dim,), eps=1e-5)
    got = op[:, :dim].double() + op[:, 2 * dim:3 * dim].double()
    # hi + lo keeps LN(x) to the bf16 precision of lo: 2^-17 relative, plus fp32 rounding
    assert ((got - want).abs() <= want.abs() * 2.0 ** -16 + 1e-6).all()
    assert torch.equal(op[:, dim:2 * dim], op[:, :dim])
    assert (op[:, 3 * dim:3 * dim + 2] == 1).all() and (op[:, 3 * dim + 2:] == 0).all()


@pytest.mark.parametrize("n,dim", [(1, 128), (37, 128), (130, 128), (9, 768)])
def test_layernorm_split3_t_is_the_operand_of_the_transposed_frame(gpu, n, dim):
    """The ending-node fp32 projection operand: rows of x.transpose(0, 1) read in
    place, bit for bit the operand of the transposed copy."""
    g = torch.Generator().manual_seed(n + dim)
    x = (torch.randn(n, n, dim, generator=g) * 2 - 1).to(gpu)
    with torch.inference_mode():
        got = ops.layernorm_split3_t(x, 1e-5)
        want = ops.layernorm_split3(x.transpose(0, 1).contiguous().view(-1, dim), 1e-5)
    assert got.shape == (n, n, 3 * dim + 64)
    assert torch.equal(got.view(-1, 3 * dim + 64), want)


@pytest.mark.parametrize("rows,cols", [(37, 1536), (5, 4), (3, 260)])
def test_swiglu_split3_matches_gated_swiglu(gpu, rows, cols):
    g = torch.Generator().manual_seed(cols)
    u = torch.randn(rows, 3 * cols, generator=g).to(gpu)
    with torch.inference_mode():
        want = ops.epilogue(u[:, :2 * cols].contiguous(), u[:, 2 * cols:].contiguous(), None, ops.GATED_SWIGLU)
        op = ops.swiglu_split3(u, cols)
    eager = F.silu(u[:, cols:2 * cols].double()) * u[:, :cols].double() * u[:, 2 * cols:].double()
    assert ((want.double() - eager).abs().max() / eager.abs().max()).item() < 1e-5
    check_operand(op, want)


@pytest.mark.parametrize("rows,cols", [(37, 768), (5, 128)])
def test_gated_residual_matches_modulation(gpu, rows, cols):
    g = torch.Generator().manual_seed(rows)
    a, c = (torch.randn(rows, cols, generator=g).to(gpu) for _ in range(2))
    gate = wide(g, rows, cols, 6 * cols, 2 * cols, gpu)
    with torch.inference_mode():
        want = ops.epilogue(a, gate.contiguous(), c, ops.MODULATION)
        got = ops.gated_residual(a, gate, c)
        c2 = c.clone()
        ops.gated_residual(a, gate, c2, out=c2)
    assert torch.equal(got, want) and torch.equal(c2, want)
    eager = c.double() + torch.sigmoid(gate.double()) * a.double()
    assert ((want.double() - eager).abs().max() / eager.abs().max()).item() < 1e-6


@pytest.mark.parametrize("rows,dim", [(37, 768), (5, 128), (3, 1024)])
def test_gated_residual_adaln_split3_matches_the_two_kernels(gpu, rows, dim):
    """One pass of the residual update and the next AdaLN operand gives the bits
    of gated_residual followed by adaln_split3; in place (out = c) too."""
    g = torch.Generator().manual_seed(rows * dim)
    y, c = (torch.randn(rows, dim, generator=g).to(gpu) for _ in range(2))
    proj = torch.randn(rows, 3 * dim, generator=g).to(gpu)  # gate | scale | shift of one projection
    gate, scale, shift = proj.split(dim, dim=-1)
    with torch.inference_mode():
        r_want = ops.gated_residual(y, gate, c)
        op_want = ops.adaln_split3(r_want, scale, shift, 1e-5)
        r_got, op_got = ops.gated_residual_adaln_split3(y, gate, c, scale, shift, 1e-5)
        c2 = c.clone()
        r_in, op_in = ops.gated_residual_adaln_split3(y, gate, c2, scale, shift, 1e-5, out=c2)
    assert torch.equal(r_got, r_want) and torch.equal(op_got, op_want)
    assert r_in.data_ptr() == c2.data_ptr() and torch.equal(c2, r_want) and torch.equal(op_in, op_want)


@pytest.mark.parametrize("m,k,n", [(37, 768, 4608), (5, 512, 8), (130, 1536, 768)])
def test_split_gemm_with_folded_bias_is_near_fp32(gpu, m, k, n):
    """mm_split of a strided operand source against x3_weight of two stacked
    linears, one with a bias (folded into the GEMM) and one without."""
    g = torch.Generator().manual_seed(m + n)
    lins = [torch.nn.Linear(k, n // 2, bias=True), torch.nn.Linear(k, n - n // 2, bias=False)]
    with torch.no_grad():
        for lin in lins:
            lin.weight.copy_(torch.randn(lin.weight.shape, generator=g) * 0.05)
        lins[0].bias.copy_(torch.randn(n // 2, generator=g) * 3)
    x = wide(g, m, k, 2 * k, k, gpu)
    w = torch.cat([lin.weight for lin in lins]).double()
    b = torch.cat([lins[0].bias, torch.zeros(n - n // 2)]).double()
    want = x.double().cpu() @ w.t() + b
    host = torch.nn.Module()
    lins = [lin.to(gpu) for lin in lins]
    with torch.inference_mode():
        w3 = ops.x3_weight(host, "w", [lin.weight for lin in lins], [lin.bias for lin in lins])
        got = ops.mm_split(ops.split3(x), w3).cpu()
        again = ops.mm_split(ops.split3(x), ops.x3_weight(host, "w", [lin.weight for lin in lins],
                                                           [lin.bias for lin in lins]))
    assert w3.shape == (n, 3 * k + 64)
    assert ((got.double() - want).abs().max() / want.abs().max()).item() < 2e-5
    assert torch.equal(again.cpu(), got)
