"""GPU checks at the largest sizes the entry points accept.

Triangle attention accepts n <= 8192.  Triangle multiplication accepts
n <= 16384, but at 16384 x, the output and its 3 x 128 x n^2 bf16 workspace
need about 320 GB, beyond one MI355X; 8192 is the largest size checked here.
The kernels address the operand planes with 64-bit offsets and the triangle
bias (4 x np^2 elements) with 32-bit ones, so these sizes exercise the
widest offsets and grids they form.

The whole-tensor oracle does not fit a test at these sizes, so sampled output
rows (first, masked, interior, last unmasked, last) are compared with the
fp32 oracle evaluated for those rows only (``forward_rows``, pinned against
the full forward in tests/test_oracle_pins.py), run on the GPU in chunks that
keep every torch intermediate at or under 1 GiB: evaluated whole at
n >= 6144 (19 to 32 GiB LayerNorm / linear inputs, a 3 GB score tensor), the
same fp32 torch ops returned wrong values on this stack, rows with zero
variation among them, while at n = 4096 (1.3 GB) they agreed with the kernel
to 5e-3.  Inputs: z ~ N(0, 1), the
last 37 tokens and token n // 3 masked, plus n = 4000 for ragged tiles.
Tolerance (north star, bf16): max|a - b| / max|b| <= 2e-2 over the rows.
"""

import pytest
import torch

from boltz_lumi_amd import ops
from oracle import boltz_ref as R

pytestmark = pytest.mark.gpu

TOL = 2e-2


def inputs(n, gpu):
    torch.manual_seed(n)
    x = torch.randn(n, n, 128, device=gpu)
    tok = torch.ones(n, device=gpu)
    tok[-37:] = 0
    tok[n // 3] = 0
    return x, tok[:, None] * tok[None, :], [0, n // 3, n // 2 + 5, n - 38, n - 1]


def finite(t, step=256):
    return all(bool(torch.isfinite(t[s:s + step]).all()) for s in range(0, t.shape[0], step))


def pick(out, rows, starting=True):
    """Rows (pairs (i, :)) or columns (pairs (:, i)) through views, stacked."""
    return torch.stack([(out[i] if starting else out[:, i]).float() for i in rows], 0 if starting else 1)


def max_rel(got, want):
    got, want = got.double(), want.double()
    return ((got - want).abs().max() / want.abs().max()).item()


@pytest.mark.parametrize("n,starting", [(4000, True), (4000, False), (8192, True)])
def test_triattn_largest_sizes(gpu, n, starting):
    print(f"triattn n={n} starting={starting}", flush=True)
    cls = R.TriangleAttention if starting else R.TriangleAttentionEndingNode
    torch.manual_seed(1)
    m = R.randomize(cls(128, 32, 4)).to(gpu).eval()
    x, mask, rows = inputs(n, gpu)
    with torch.inference_mode():
        out = ops.triattn(m, x, mask, starting)
        got = pick(out, rows, starting)
        ok = finite(out)
        del out
        torch.cuda.empty_cache()
        want = m.forward_rows(x[None], mask[None], rows)[0]
    assert ok
    assert max_rel(got, want) < TOL


@pytest.mark.parametrize("n,outgoing", [(4000, True), (4000, False), (8192, True)])
def test_trimul_largest_sizes(gpu, n, outgoing):
    print(f"trimul n={n} outgoing={outgoing}", flush=True)
    cls = R.TriangleMultiplicationOutgoing if outgoing else R.TriangleMultiplicationIncoming
    torch.manual_seed(2)
    m = R.randomize(cls(128)).to(gpu).eval()
    x, mask, rows = inputs(n, gpu)
    with torch.inference_mode():
        out = ops.trimul(m, x, mask, outgoing)
        got = pick(out, rows)
        ok = finite(out)
        del out
        torch.cuda.empty_cache()
        want = m.forward_rows(x[None], mask[None], rows, chunk=64)[0]
    assert ok
    assert max_rel(got, want) < TOL


def test_pair_transition_largest_size(gpu):
    """N = 8191: 67,092,481 pair rows, the last 64-row tile holding one row.
    The transition is per pair, so the oracle on the sampled rows alone is the
    oracle's output there; the in-place fp32 accumulate mode is checked on the
    same rows."""
    n = 8191
    print(f"pair_transition n={n}", flush=True)
    torch.manual_seed(3)
    m = R.randomize(R.Transition(128, 512)).to(gpu).eval()
    x, _, rows = inputs(n, gpu)
    with torch.inference_mode():
        want = torch.stack([m(x[i]) for i in rows])
        out = ops.pair_transition(m, x)
        got = pick(out, rows)
        ok = finite(out)
        del out
        torch.cuda.empty_cache()
        base = pick(x, rows)
        ops.pair_transition(m, x, ops.OUT_ACCUMULATE, out=x)  # x += transition(x), in place
        res = pick(x, rows)
    assert ok
    assert max_rel(got, want) < TOL
    assert max_rel(res - base, want) < TOL


@pytest.mark.parametrize("starting", [True, False])
def test_fp32_triattn_row_blocks_at_large_n(gpu, starting, monkeypatch):
    """fp32-mode triangle attention at N = 6144, where one pass does not fit
    (4.6 KB per pair, 174 GB): the installed forward runs blocks of frame rows
    and the sampled rows meet the fp32-mode bar (1e-4) against the fp32
    oracle's rows."""
    from boltz_lumi_amd import triangle

    n = 6144
    total = torch.cuda.get_device_properties(gpu).total_memory
    rows_per_block = triangle.fp32_block_rows(n, total)
    print(f"fp32 triattn n={n} starting={starting}: blocks of {rows_per_block} rows", flush=True)
    assert 0 < rows_per_block < n
    seen = []
    original = ops.triattn_fp32
    monkeypatch.setattr(ops, "triattn_fp32", lambda *a, **k: seen.append(k.get("block_rows")) or original(*a, **k))
    cls = R.TriangleAttention if starting else R.TriangleAttentionEndingNode
    torch.manual_seed(2)
    m = R.randomize(cls(128, 32, 4)).to(gpu).eval()
    x, mask, rows = inputs(n, gpu)
    with torch.inference_mode():
        out = triangle.triangle_attention_forward(m, x[None], mask[None])[0]
        assert seen == [rows_per_block] and out.dtype == torch.float32
        got = pick(out, rows, starting)
        ok = finite(out)
        del out
        torch.cuda.empty_cache()
        want = m.forward_rows(x[None], mask[None], rows)[0]
    assert ok
    err = max_rel(got, want)
    print(f"fp32 triattn n={n} starting={starting}: sampled rows max_rel {err:.2e}", flush=True)
    assert err < 1e-4
