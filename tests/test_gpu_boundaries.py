"""GPU parity at the kernels' tile boundaries.

The kernels tile queries by 16, keys by 64 per stage, pairs by 64 per
projection/output tile and pad rows to a multiple of 256 (triangle
attention) or of the contraction tile (multiplication); sizes on either
side of those edges exercise the ragged-tile paths.  Each case compares the
native op with the fp32 oracle (run on the GPU) on seeded inputs with a
seeded token mask, at the north star's bf16 tolerance 2e-2
(max|a - b| / max|b|)."""

import pytest
import torch

from boltz_lumi_amd import ops
from oracle import boltz_ref as R

pytestmark = pytest.mark.gpu

TOL = 2e-2
SIZES = [1, 2, 15, 16, 17, 63, 65, 127, 129, 255, 257]


def case(n, gpu):
    g = torch.Generator().manual_seed(1000 + n)
    x = torch.randn(n, n, 128, generator=g)
    tok = (torch.rand(n, generator=g) > 0.15).float()
    tok[0] = 1.0
    return g, x.to(gpu), (tok[:, None] * tok[None, :]).to(gpu)


def max_rel(got, want):
    got, want = got.double(), want.double()
    return ((got - want).abs().max() / want.abs().max()).item()


@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("starting", [True, False])
def test_triattn_tile_edges(gpu, n, starting):
    g, x, mask = case(n, gpu)
    m = R.randomize(R.TriangleAttention(128, 32, 4, starting=starting), generator=g).to(gpu).eval()
    with torch.inference_mode():
        want = m(x[None], mask[None])[0]
        got = ops.triattn(m, x, mask, starting)
    assert torch.isfinite(got).all()
    assert max_rel(got, want) < TOL


@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("outgoing", [True, False])
def test_trimul_tile_edges(gpu, n, outgoing):
    g, x, mask = case(n, gpu)
    cls = R.TriangleMultiplicationOutgoing if outgoing else R.TriangleMultiplicationIncoming
    m = R.randomize(cls(128), generator=g).to(gpu).eval()
    with torch.inference_mode():
        want = m(x[None], mask[None])[0]
        got = ops.trimul(m, x, mask, outgoing)
    assert torch.isfinite(got).all()
    assert max_rel(got, want) < TOL


@pytest.mark.parametrize("n", SIZES)
def test_pair_transition_tile_edges(gpu, n):
    g, x, _ = case(n, gpu)
    m = R.randomize(R.Transition(128, 512), generator=g).to(gpu).eval()
    with torch.inference_mode():
        want = m(x)
        got = ops.pair_transition(m, x)
        acc = x.clone()
        ops.pair_transition(m, acc, ops.OUT_ACCUMULATE, out=acc)
    assert max_rel(got, want) < TOL
    assert max_rel(acc - x, want) < TOL


@pytest.mark.parametrize("n", [17, 65, 130])
@pytest.mark.parametrize("starting", [True, False])
def test_triattn_bf16_input(gpu, n, starting):
    """bf16 x (the kernels' second input type) against the oracle on the same
    bf16-rounded values, and the fp32 result modes on that input."""
    g, x, mask = case(n, gpu)
    xb = x.bfloat16()
    m = R.randomize(R.TriangleAttention(128, 32, 4, starting=starting), generator=g).to(gpu).eval()
    with torch.inference_mode():
        want = m(xb.float()[None], mask[None])[0]
        got = ops.triattn(m, xb, mask, starting)
        got32 = ops.triattn(m, xb, mask, starting, ops.OUT_F32)
    assert got.dtype == torch.bfloat16 and got32.dtype == torch.float32
    assert max_rel(got, want) < TOL
    assert max_rel(got32, want) < TOL
    assert torch.equal(got32.bfloat16(), got)


@pytest.mark.parametrize("n", [65, 129])
@pytest.mark.parametrize("op", ["trimul_out", "trimul_in", "triattn_start", "triattn_end", "transition"])
def test_output_modes_are_exact_compositions(gpu, n, op):
    """Every result mode of an op is its fp32 result y composed with fp32 adds:
    bf16 = bf16(y) (y already holds bf16 values), residual out = x + y,
    accumulate into another buffer out += y, accumulate in place x += y."""
    g, x, mask = case(n, gpu)
    if op.startswith("trimul"):
        outgoing = op == "trimul_out"
        cls = R.TriangleMultiplicationOutgoing if outgoing else R.TriangleMultiplicationIncoming
        m = R.randomize(cls(128), generator=g).to(gpu).eval()

        def run(xx, mode, out=None):
            return ops.trimul(m, xx, mask, outgoing, mode, out)
    elif op.startswith("triattn"):
        starting = op == "triattn_start"
        m = R.randomize(R.TriangleAttention(128, 32, 4, starting=starting), generator=g).to(gpu).eval()

        def run(xx, mode, out=None):
            return ops.triattn(m, xx, mask, starting, mode, out)
    else:
        m = R.randomize(R.Transition(128, 512), generator=g).to(gpu).eval()

        def run(xx, mode, out=None):
            return ops.pair_transition(m, xx, mode, out)

    with torch.inference_mode():
        y = run(x, ops.OUT_F32)
        assert torch.equal(run(x, ops.OUT_BF16), y.bfloat16())
        assert torch.equal(y.bfloat16().float(), y)
        assert torch.equal(run(x, ops.OUT_RESIDUAL, torch.empty_like(x)), x + y)
        other = torch.randn(x.shape, generator=g).to(gpu)
        want = other + y
        run(x, ops.OUT_ACCUMULATE, other)
        assert torch.equal(other, want)
        xi = x.clone()
        run(xi, ops.OUT_ACCUMULATE, xi)
        assert torch.equal(xi, x + y)


def test_empty_inputs_return_empty_outputs(gpu):
    """N = 0 (and zero transition rows): every fused op returns an empty result
    of the right shape and dtype without launching a kernel."""
    g = torch.Generator().manual_seed(0)
    x = torch.empty(0, 0, 128, device=gpu)
    mask = torch.empty(0, 0, device=gpu)
    att = R.randomize(R.TriangleAttention(128, 32, 4), generator=g).to(gpu).eval()
    mul = R.randomize(R.TriangleMultiplicationOutgoing(128), generator=g).to(gpu).eval()
    tr = R.randomize(R.Transition(128, 512), generator=g).to(gpu).eval()
    with torch.inference_mode():
        outs = [ops.triattn(att, x, mask, True), ops.trimul(mul, x, mask, True),
                ops.pair_transition(tr, torch.empty(0, 128, device=gpu))]
    torch.cuda.synchronize()
    assert [tuple(o.shape) for o in outs] == [(0, 0, 128), (0, 0, 128), (0, 128)]
    assert all(o.dtype == torch.bfloat16 for o in outs)

