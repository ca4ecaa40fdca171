"""fp32-mode triangle attention (autocast off, fp32 x; reference
triangle.py:38-52): the installed forward (ops.triattn_fp32: the projection as
one split-bf16 GEMM with the LayerNorm affine folded in, the fused split-bf16
attention, an fp32 output linear) must meet the north star's fp32-mode bar,
max relative error <= 1e-4 against the fp32 CPU oracle, for both nodes at
N = 117, 512 and 1024, with padded tokens."""

import copy

import pytest
import torch

from boltz_lumi_amd import ops
from boltz_lumi_amd.triangle import triangle_attention_forward
from oracle import boltz_ref as R

pytestmark = pytest.mark.gpu


def max_rel(got, want):
    got, want = got.double().cpu(), want.double().cpu()
    return ((got - want).abs().max() / want.abs().max()).item()


@pytest.mark.parametrize("n,exact", [(117, False), (512, False), (1024, False), (117, True), (512, True)])
@pytest.mark.parametrize("starting", [True, False])
def test_fp32_triangle_attention_matches_oracle(gpu, n, exact, starting):
    """``exact``: BMX_EXACT_FP32_LINEARS mode (fp32 LayerNorm, fp32 GEMMs and
    the fp32-MFMA attention)."""
    g = torch.Generator().manual_seed(n + starting)
    cls = R.TriangleAttention if starting else R.TriangleAttentionEndingNode
    ref = R.randomize(cls(128, 32, 4), generator=g).eval()
    x = torch.randn(1, n, n, 128, generator=g)
    tok = torch.ones(n)
    tok[-(n // 10):] = 0
    mask = (tok[:, None] * tok[None, :])[None]
    print(f"fp32 triangle attention n={n} exact={exact} starting={starting}: CPU oracle", flush=True)
    with torch.no_grad():
        want = ref(x, mask, chunk_size=64)
    mine = copy.deepcopy(ref).to(gpu)
    calls = []
    original = ops.triattn_fp32
    before = ops.exact_fp32_linears(exact)
    try:
        ops.triattn_fp32 = lambda *a, **k: calls.append(1) or original(*a, **k)
        with torch.inference_mode():
            got = triangle_attention_forward(mine, x.to(gpu), mask.to(gpu))
    finally:
        ops.triattn_fp32 = original
        ops.exact_fp32_linears(before)
    torch.cuda.synchronize()
    assert calls == [1] and got.dtype == torch.float32 and got.shape == want.shape
    err = max_rel(got, want)
    print(f"fp32 triangle attention n={n} exact={exact} starting={starting}: max_rel {err:.2e}", flush=True)
    assert err < 1e-4


def test_fp32_triangle_attention_falls_back_under_grad(gpu):
    ref = R.randomize(R.TriangleAttention(128, 32, 4), generator=torch.Generator().manual_seed(1)).to(gpu).eval()
    x = torch.randn(1, 20, 20, 128, device=gpu, requires_grad=True)
    mask = torch.ones(1, 20, 20, device=gpu)
    got = triangle_attention_forward(ref, x, mask)
    want = type(ref).forward(ref, x, mask)
    assert torch.equal(got, want) and got.requires_grad


@pytest.mark.parametrize("exact", [False, True])
@pytest.mark.parametrize("starting", [True, False])
def test_fp32_working_set_within_the_native_bound(gpu, starting, exact):
    """The one-pass fp32 path holds every row at once and runs while
    ``FP32_BYTES_PER_PAIR`` * N^2 fits the device (``fp32_native_fits``; row
    blocks above): the memory one call allocates on top of its input, output
    included, must stay within that per-pair figure."""
    from boltz_lumi_amd.triangle import FP32_BYTES_PER_PAIR

    n = 1024
    cls = R.TriangleAttention if starting else R.TriangleAttentionEndingNode
    layer = R.randomize(cls(128, 32, 4), generator=torch.Generator().manual_seed(3)).to(gpu).eval()
    x = torch.randn(1, n, n, 128, device=gpu)
    tok = torch.ones(n, device=gpu)
    tok[-50:] = 0
    mask = (tok[:, None] * tok[None, :])[None]
    before = ops.exact_fp32_linears(exact)
    try:
        with torch.inference_mode():
            triangle_attention_forward(layer, x, mask)  # weight packs and library state built here
            torch.cuda.synchronize()
            torch.cuda.reset_peak_memory_stats(gpu)
            base = torch.cuda.memory_allocated(gpu)
            out = triangle_attention_forward(layer, x, mask)
            torch.cuda.synchronize()
            peak = torch.cuda.max_memory_allocated(gpu) - base
    finally:
        ops.exact_fp32_linears(before)
    assert out.dtype == torch.float32
    per_pair = peak / (n * n)
    print(f"fp32 triangle attention n={n} starting={starting} exact={exact}: {per_pair:.0f} bytes per pair at peak",
          flush=True)
    assert per_pair <= FP32_BYTES_PER_PAIR


@pytest.mark.parametrize("n,rows", [(117, 40), (300, 128)])
@pytest.mark.parametrize("exact", [False, True])
@pytest.mark.parametrize("starting", [True, False])
def test_fp32_row_blocks_match_one_pass(gpu, n, rows, exact, starting):
    """Above the one-pass fit, fp32 mode runs in blocks of frame rows (x's rows
    for the starting node, its columns for the ending node), the triangle bias
    first for every row: the same products as one pass, block by block."""
    g = torch.Generator().manual_seed(n + 7 * starting)
    cls = R.TriangleAttention if starting else R.TriangleAttentionEndingNode
    layer = R.randomize(cls(128, 32, 4), generator=g).to(gpu).eval()
    x = torch.randn(n, n, 128, generator=g).to(gpu)
    tok = torch.ones(n)
    tok[-(n // 10):] = 0
    mask = (tok[:, None] * tok[None, :]).to(gpu)
    before = ops.exact_fp32_linears(exact)
    try:
        with torch.inference_mode():
            one = ops.triattn_fp32(layer, x, mask, starting)
            blocked = ops.triattn_fp32(layer, x, mask, starting, block_rows=rows)
    finally:
        ops.exact_fp32_linears(before)
    torch.cuda.synchronize()
    assert blocked.shape == one.shape and blocked.dtype == torch.float32
    err = max_rel(blocked, one)
    print(f"fp32 row blocks n={n} rows={rows} exact={exact} starting={starting}: max_rel {err:.2e} against one pass",
          flush=True)
    assert err < 1e-6


@pytest.mark.parametrize("starting", [True, False])
def test_installed_fp32_forward_takes_row_blocks_where_one_pass_does_not_fit(gpu, monkeypatch, starting):
    """With the memory share shrunk so that one pass does not fit at N = 300,
    the installed forward runs row blocks and still meets the 1e-4 bar
    against the fp32 oracle."""
    from boltz_lumi_amd import triangle

    n = 300
    total = torch.cuda.get_device_properties(gpu).total_memory
    share = (triangle.FP32_FRAME_BYTES_PER_PAIR * n * n + triangle.FP32_BYTES_PER_PAIR * 100 * n) / total
    monkeypatch.setattr(triangle, "FP32_MEMORY_SHARE", share)
    rows = triangle.fp32_block_rows(n, total)
    assert 90 <= rows < n
    g = torch.Generator().manual_seed(31 + starting)
    cls = R.TriangleAttention if starting else R.TriangleAttentionEndingNode
    ref = R.randomize(cls(128, 32, 4), generator=g).eval()
    x = torch.randn(1, n, n, 128, generator=g)
    tok = torch.ones(n)
    tok[-30:] = 0
    mask = (tok[:, None] * tok[None, :])[None]
    with torch.no_grad():
        want = ref(x, mask, chunk_size=64)
    mine = copy.deepcopy(ref).to(gpu)
    seen = []
    original = ops.triattn_fp32
    monkeypatch.setattr(ops, "triattn_fp32", lambda *a, **k: seen.append(k.get("block_rows")) or original(*a, **k))
    with torch.inference_mode():
        got = triangle_attention_forward(mine, x.to(gpu), mask.to(gpu))
    torch.cuda.synchronize()
    assert seen == [rows]
    err = max_rel(got, want)
    print(f"installed fp32 row blocks n={n} rows={rows} starting={starting}: max_rel {err:.2e}", flush=True)
    assert err < 1e-4


@pytest.mark.parametrize("starting", [True, False])
def test_fp32_row_block_working_set(gpu, starting):
    """Row blocks hold the output frame, the triangle bias and the mask for
    the whole frame and the rest for one block: within
    FP32_FRAME_BYTES_PER_PAIR + FP32_BYTES_PER_PAIR * rows / N per pair."""
    from boltz_lumi_amd.triangle import FP32_BYTES_PER_PAIR, FP32_FRAME_BYTES_PER_PAIR

    n, rows = 1024, 256
    cls = R.TriangleAttention if starting else R.TriangleAttentionEndingNode
    layer = R.randomize(cls(128, 32, 4), generator=torch.Generator().manual_seed(5)).to(gpu).eval()
    x = torch.randn(n, n, 128, device=gpu)
    mask = torch.ones(n, n, device=gpu)
    with torch.inference_mode():
        ops.triattn_fp32(layer, x, mask, starting, block_rows=rows)  # weight packs built here
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats(gpu)
        base = torch.cuda.memory_allocated(gpu)
        out = ops.triattn_fp32(layer, x, mask, starting, block_rows=rows)
        torch.cuda.synchronize()
        peak = torch.cuda.max_memory_allocated(gpu) - base
    assert out.shape == (n, n, 128)
    per_pair = peak / (n * n)
    bound = FP32_FRAME_BYTES_PER_PAIR + FP32_BYTES_PER_PAIR * rows / n
    print(f"fp32 row blocks n={n} rows={rows} starting={starting}: {per_pair:.0f} bytes per pair at peak "
          f"(bound {bound:.0f})", flush=True)
    assert per_pair <= bound
