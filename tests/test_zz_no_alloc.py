"""The allocation-free triangle multiplication entry point
(bmx_trimul_fwd_noalloc, operand planes in the library's static scratch)
against bmx_trimul_fwd with a caller-owned workspace: the same kernels, so
the results must be bit-identical.  Two calls in a row, the second with a
smaller input (the scratch keeps the first call's planes), both directions
and two result modes; sizes above the scratch's limit are rejected before
any launch."""

import pytest
import torch

from boltz_lumi_amd import _native as N
from boltz_lumi_amd import ops
from oracle import boltz_ref as R

pytestmark = pytest.mark.gpu

NOALLOC_MAX_N = 256


def noalloc_fn():
    return N.lib().bmx_trimul_fwd_noalloc  # argument types from the binding table (include/bmx.h)


def call_noalloc(module, x, mask, outgoing, out_mode, out):
    """The C entry point with the same weight packs ops.trimul passes."""
    w_in = ops.cached_weight(module, "w_in", (module.p_in.weight, module.g_in.weight), ops._bf16)
    w_pout = ops.cached_weight(module, "w_pout", (module.p_out.weight,), ops._bf16)
    w_gout = ops.cached_weight(module, "w_gout", (module.g_out.weight,), ops._bf16)
    ni, no = module.norm_in, module.norm_out
    return noalloc_fn()(x.data_ptr(), mask.data_ptr(), x.shape[0], int(outgoing), ni.weight.data_ptr(),
                        ni.bias.data_ptr(), ni.eps, w_in.data_ptr(), no.weight.data_ptr(), no.bias.data_ptr(), no.eps,
                        w_pout.data_ptr(), w_gout.data_ptr(), out.data_ptr(), out_mode,
                        torch.cuda.current_stream().cuda_stream)


def inputs(n, gpu, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, n, 128, generator=g)
    tokens = (torch.rand(n, generator=g) > 0.1).float()
    mask = tokens[:, None] * tokens[None, :]
    return x.to(gpu), mask.to(gpu)


@pytest.mark.parametrize("outgoing", [True, False])
def test_noalloc_matches_workspace_entry_point(gpu, outgoing):
    torch.manual_seed(0)
    cls = R.TriangleMultiplicationOutgoing if outgoing else R.TriangleMultiplicationIncoming
    module = R.randomize(cls(128), generator=torch.Generator().manual_seed(1)).to(gpu).eval()
    with torch.inference_mode():
        for n, seed in ((200, 3), (77, 4)):  # second call smaller: the scratch still holds the first call's planes
            print(f"noalloc trimul outgoing={outgoing} n={n}", flush=True)
            x, mask = inputs(n, gpu, seed)
            for mode in (ops.OUT_BF16, ops.OUT_RESIDUAL):
                want = ops.trimul(module, x, mask, outgoing, mode)
                got = torch.full_like(want, float("nan"))
                rc = call_noalloc(module, x, mask, outgoing, mode, got)
                assert rc == N.BMX_OK, N.last_error()
                torch.cuda.synchronize()
                assert torch.equal(got, want), (n, mode, (got.float() - want.float()).abs().max().item())


def test_noalloc_rejects_sizes_beyond_its_scratch(gpu):
    module = R.randomize(R.TriangleMultiplicationOutgoing(128)).to(gpu).eval()
    n = NOALLOC_MAX_N + 1
    x, mask = inputs(n, gpu, 5)
    out = torch.zeros(n, n, 128, device=gpu, dtype=torch.bfloat16)
    with torch.inference_mode():
        rc = call_noalloc(module, x, mask, True, ops.OUT_BF16, out)
    torch.cuda.synchronize()
    assert rc == N.BMX_EINVAL
    assert "[0, 256]" in N.last_error()
    assert not out.any()  # nothing was launched
