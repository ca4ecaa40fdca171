"""GPU checks at the BASELINE.json workload sizes.

configs[1] (triangle attention, N=512, last 51 tokens padded), configs[2]
(triangle multiplication, N=768, 5% of tokens masked) and configs[3]'s layer
(one PairformerLayer at N=1024) are compared with the fp32 oracle directly:
the oracle runs them in seconds on the host cores.  Size-independent
properties back them up: determinism, the ending-node / starting-node
transpose identity, masked tokens contributing nothing, and token-permutation
equivariance.  Tolerance (north star): max|a-b| / max|b| <= 2e-2 in bf16; the
oracle comparisons also print the relative L2 error, max absolute error and
the count of elements past the bar.
"""

import pytest
import torch

from boltz_lumi_amd import layers, ops
from oracle import boltz_ref as R

pytestmark = pytest.mark.gpu

TOL = 2e-2


def max_rel(got, want, name=None):
    """max |a - b| / max |b|.  With a name, also prints the relative L2 error,
    the max absolute error and the number of elements past the bar
    (|a - b| > TOL * max |b|), the fields the reference's own comparison
    reports (tests/test_operator_additions.py:25-39)."""
    got, want = got.double().cpu(), want.double().cpu()
    err = got - want
    scale = want.abs().max().clamp_min(1e-30)
    rel = (err.abs().max() / scale).item()
    if name is not None:
        l2 = (err.norm() / want.norm().clamp_min(1e-30)).item()
        failing = int((err.abs() > TOL * scale).sum())
        print(f"{name}: max_rel {rel:.3e}  rel_l2 {l2:.3e}  max_abs {err.abs().max().item():.3e}  "
              f"failing {failing} of {err.numel()} (bar {TOL})", flush=True)
    return rel


def cfg2_inputs():
    """z ~ N(0,1) [1,512,512,128]; token mask = 461 ones then 51 zeros."""
    g = torch.Generator().manual_seed(0)
    n = 512
    x = torch.randn(1, n, n, 128, generator=g)
    tok = torch.ones(n)
    tok[-51:] = 0
    return g, x, (tok[:, None] * tok[None, :])[None]


@pytest.mark.parametrize("starting", [True, False])
def test_triattn_config2_matches_oracle(gpu, starting):
    g, x, mask = cfg2_inputs()
    cls = R.TriangleAttention if starting else R.TriangleAttentionEndingNode
    m = R.randomize(cls(128, 32, 4), generator=g)
    with torch.no_grad():
        want = m(x, mask, chunk_size=64)[0]
    with torch.inference_mode():
        got = ops.triattn(m.to(gpu), x[0].to(gpu), mask[0].to(gpu), starting)
    assert torch.isfinite(got).all()
    assert max_rel(got, want, f"configs[1] triattn {'starting' if starting else 'ending'}") < TOL


def test_triattn_config2_ending_is_transposed_starting(gpu):
    """Ending node on (z, mask) is the starting node on (z^T, mask^T), transposed
    back; the kernels read the transposed frame in place, so the results match
    bit for bit."""
    g, x, mask = cfg2_inputs()
    mask = mask.clone()
    mask[0, 3, 7] = 0  # break the mask's symmetry
    m = R.randomize(R.TriangleAttention(128, 32, 4), generator=g).to(gpu)
    xd, md = x[0].to(gpu), mask[0].to(gpu)
    with torch.inference_mode():
        end = ops.triattn(m, xd, md, False)
        start_t = ops.triattn(m, xd.transpose(0, 1).contiguous(), md.t().contiguous(), True)
    assert torch.equal(end, start_t.transpose(0, 1))


def cfg3_inputs():
    """z ~ N(0,1) [1,768,768,128]; 38 random tokens (5%) masked."""
    g = torch.Generator().manual_seed(0)
    n = 768
    x = torch.randn(1, n, n, 128, generator=g)
    tok = torch.ones(n)
    tok[torch.randperm(n, generator=torch.Generator().manual_seed(0))[:38]] = 0
    return g, x, (tok[:, None] * tok[None, :])[None]


@pytest.mark.parametrize("outgoing", [True, False])
def test_trimul_config3_matches_oracle(gpu, outgoing):
    g, x, mask = cfg3_inputs()
    cls = R.TriangleMultiplicationOutgoing if outgoing else R.TriangleMultiplicationIncoming
    m = R.randomize(cls(128), generator=g)
    with torch.no_grad():
        want = m(x, mask)[0]
    with torch.inference_mode():
        got = ops.trimul(m.to(gpu), x[0].to(gpu), mask[0].to(gpu), outgoing)
    assert torch.isfinite(got).all()
    assert max_rel(got, want, f"configs[2] trimul {'outgoing' if outgoing else 'incoming'}") < TOL


def test_trimul_config3_masked_tokens_contribute_nothing(gpu):
    """Masked tokens' a/b rows are exactly zero, so changing z on a masked
    token k changes no output pair (i, j) with i, j unmasked."""
    g, x, mask = cfg3_inputs()
    m = R.randomize(R.TriangleMultiplicationOutgoing(128), generator=g).to(gpu)
    tok = mask[0].diagonal()
    k = int((tok == 0).nonzero()[0])
    x2 = x.clone()
    x2[0, :, k] += 3.0  # pairs (i, k): token k's column only
    keep = tok.bool()
    keep[k] = False
    with torch.inference_mode():
        a = ops.trimul(m, x[0].to(gpu), mask[0].to(gpu), True)
        b = ops.trimul(m, x2[0].to(gpu), mask[0].to(gpu), True)
    sel = keep.to(gpu)
    assert torch.equal(a[sel][:, sel], b[sel][:, sel])


def layer_n1024(gpu, seed=0):
    g = torch.Generator().manual_seed(seed)
    ref = R.randomize(R.PairformerLayer(), generator=g)
    mine = layers.PairformerLayer()
    mine.load_state_dict(ref.state_dict())
    return g, mine.to(gpu).eval()


def test_pairformer_layer_config4_matches_oracle(gpu):
    """configs[3]'s layer at full size against the fp32 oracle (about 15 s of
    CPU time on the GPU box's host cores)."""
    g = torch.Generator().manual_seed(0)
    ref = R.randomize(R.PairformerLayer(), generator=g).eval()
    mine = layers.PairformerLayer()
    mine.load_state_dict(ref.state_dict())
    mine = mine.to(gpu).eval()
    n = 1024
    z = torch.randn(1, n, n, 128, generator=g)
    s = torch.randn(1, n, 384, generator=g)
    mask = torch.ones(1, n)
    pm = mask[:, :, None] * mask[:, None, :]
    with torch.no_grad():
        s_ref, z_ref = ref(s, z, mask, pm, chunk_size_tri_attn=64)
    with torch.inference_mode():
        s_got, z_got = mine(s.to(gpu), z.to(gpu), mask.to(gpu), pm.to(gpu))
    e_dz = max_rel(z_got.cpu() - z, z_ref - z, "configs[3] layer z update")
    assert e_dz < TOL
    assert max_rel(z_got, z_ref, "configs[3] layer z") < TOL
    assert max_rel(s_got, s_ref, "configs[3] layer s") < TOL


def test_pairformer_layer_config4_deterministic_and_finite(gpu):
    g, layer = layer_n1024(gpu)
    n = 1024
    z = torch.randn(1, n, n, 128, generator=g).to(gpu)
    s = torch.randn(1, n, 384, generator=g).to(gpu)
    mask = torch.ones(1, n, device=gpu)
    pm = mask[:, :, None] * mask[:, None, :]
    with torch.inference_mode():
        s1, z1 = layer(s, z, mask, pm)
        s2, z2 = layer(s, z, mask, pm)
    assert torch.isfinite(z1).all() and torch.isfinite(s1).all()
    assert torch.equal(z1, z2) and torch.equal(s1, s2)


def test_pairformer_layer_config4_permutation_equivariant(gpu):
    """Relabelling the tokens permutes the layer's outputs the same way (every
    pair op is equivariant under a joint permutation of i and j).  Reduction
    orders over keys / k change, so the match is to the bf16 tolerance."""
    g, layer = layer_n1024(gpu, seed=1)
    n = 1024
    z = torch.randn(1, n, n, 128, generator=g).to(gpu)
    s = torch.randn(1, n, 384, generator=g).to(gpu)
    mask = torch.ones(1, n, device=gpu)
    mask[:, -40:] = 0
    pm = mask[:, :, None] * mask[:, None, :]
    perm = torch.randperm(n, generator=torch.Generator().manual_seed(2)).to(gpu)
    with torch.inference_mode():
        s1, z1 = layer(s, z, mask, pm)
        zp = z[:, perm][:, :, perm].contiguous()
        s2, z2 = layer(s[:, perm].contiguous(), zp, mask[:, perm].contiguous(), pm[:, perm][:, :, perm].contiguous())
        dz1 = (z1 - z)[:, perm][:, :, perm]
        dz2 = z2 - zp
    assert max_rel(dz2, dz1) < TOL
    assert max_rel(s2, s1[:, perm]) < TOL
