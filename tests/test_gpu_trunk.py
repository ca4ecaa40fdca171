"""BASELINE configs[3] in full on the GPU: the 64-block Pairformer trunk at
N=1024 (the north star's target configuration).  Properties that hold at
any depth: every output finite, the trunk deterministic, the ping-pong pair
buffers equal to layer-by-layer calls bit for bit; and the first two blocks
against the fp32 CPU oracle (about 30 s of host time on the GPU box)."""

import pytest
import torch

from boltz_lumi_amd import layers
from oracle import boltz_ref as R

pytestmark = pytest.mark.gpu

N, BLOCKS, TOL = 1024, 64, 2e-2


def max_rel(got, want):
    got, want = got.double().cpu(), want.double().cpu()
    return ((got - want).abs().max() / want.abs().max()).item()


@pytest.fixture(scope="module")
def trunk_and_refs(gpu):
    refs = [R.randomize(R.PairformerLayer(), generator=torch.Generator().manual_seed(seed)).eval()
            for seed in range(BLOCKS)]
    trunk = layers.PairformerModule(num_blocks=BLOCKS)
    for mine, ref in zip(trunk.layers, refs):
        mine.load_state_dict(ref.state_dict())
    return trunk.to(gpu).eval(), refs[:2]


def inputs(seed=11, padded=24):
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(1, N, N, 128, generator=g)
    s = torch.randn(1, N, 384, generator=g)
    mask = torch.ones(1, N)
    mask[:, -padded:] = 0
    return s, z, mask, mask[:, :, None] * mask[:, None, :]


def test_trunk_64_blocks_finite_deterministic_and_ping_pong(trunk_and_refs, gpu):
    trunk, _ = trunk_and_refs
    s, z, mask, pm = (t.to(gpu) for t in inputs())
    print(f"64-block trunk N={N}", flush=True)
    with torch.inference_mode():
        s1, z1 = trunk(s, z, mask, pm)
        s2, z2 = trunk(s, z, mask, pm)
        s3, z3 = s, z
        for layer in trunk.layers:  # a fresh output buffer per layer
            s3, z3 = layer(s3, z3, mask, pm)
    torch.cuda.synchronize()
    assert torch.isfinite(z1).all() and torch.isfinite(s1).all()
    assert torch.equal(z1, z2) and torch.equal(s1, s2)
    assert torch.equal(z1, z3) and torch.equal(s1, s3)
    print(f"64-block trunk: max |z| {z1.abs().max().item():.1f}, max |s| {s1.abs().max().item():.1f}", flush=True)


def test_trunk_first_two_blocks_match_oracle(trunk_and_refs, gpu):
    trunk, refs = trunk_and_refs
    s, z, mask, pm = inputs()
    print("trunk blocks 1-2: CPU oracle", flush=True)
    with torch.no_grad():
        s_ref, z_ref = s, z
        want = []
        for ref in refs:
            s_ref, z_ref = ref(s_ref, z_ref, mask, pm, chunk_size_tri_attn=64)
            want.append((s_ref, z_ref))
    with torch.inference_mode():
        s_got, z_got = s.to(gpu), z.to(gpu)
        for depth, (layer, (sw, zw)) in enumerate(zip(trunk.layers[:2], want), start=1):
            s_got, z_got = layer(s_got, z_got, mask.to(gpu), pm.to(gpu))
            ez, es = max_rel(z_got, zw), max_rel(s_got, sw)
            print(f"trunk block {depth}: z max_rel {ez:.3e}, s max_rel {es:.3e}", flush=True)
            assert ez < TOL and es < TOL
