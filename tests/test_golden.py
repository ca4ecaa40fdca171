"""The CPU oracle against the frozen self-fixtures of tests/golden (written by
tests/golden/make_golden.py from the fp64 explicit loops of oracle/brute.py):
the five pair modules and one PairformerLayer at production width, N = 6, a
token masked in the middle.  A refactor of the oracle or of the loops that
changes any result fails here.

Attention outputs are compared on the open pairs (and the sequence stack on
the open tokens): the masked token's query row has every key masked, where
fp32 and bf16 round S - 1e9 to -1e9 for every key (a uniform softmax, the mean
of v) while the fp64 loops keep softmax(S).  Masked keys carry exactly zero
weight at every precision, so the difference stays in that row and column."""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import boltz_ref as R

GOLDEN = Path(__file__).resolve().parent / "golden" / "pair_modules_n6.npz"

MODULES = {
    "tri_mul_out": lambda: R.TriangleMultiplicationOutgoing(128),
    "tri_mul_in": lambda: R.TriangleMultiplicationIncoming(128),
    "tri_att_start": lambda: R.TriangleAttention(128, 32, 4),
    "tri_att_end": lambda: R.TriangleAttentionEndingNode(128, 32, 4),
    "transition_z": lambda: R.Transition(128, 512),
}


@pytest.fixture(scope="module")
def golden():
    with np.load(GOLDEN, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def build(ctor, golden, name):
    module = R.randomize(ctor(), generator=torch.Generator().manual_seed(int(golden[f"{name}/seed"]))).eval()
    flat = torch.cat([p.detach().double().flatten() for p in module.parameters()])
    stats = np.array([flat.sum().item(), (flat * flat).sum().item()])
    # the fixture's weights are regenerated from the seed: the checksum says they are the same weights
    np.testing.assert_allclose(stats, golden[f"{name}/weight_stats"], rtol=1e-12, atol=1e-9)
    return module


def max_rel(got, want):
    got, want = torch.as_tensor(got).double(), torch.as_tensor(want).double()
    return ((got - want).abs().max() / want.abs().max()).item()


def call(name, module, z, pm):
    if name.startswith("tri_att"):
        return module(z, pm, chunk_size=None)
    if name.startswith("tri_mul"):
        return module(z, pm)
    return module(z)


def compared(name, golden):
    """Pairs compared for this output: all, or the open pairs for attention."""
    pm = golden["pair_mask"].astype(bool)
    return pm if name.startswith(("tri_att", "pairformer")) else np.ones_like(pm)


@pytest.mark.parametrize("name", list(MODULES))
def test_pair_module_matches_frozen_loops(golden, name):
    module = build(MODULES[name], golden, name)
    z, pm = torch.from_numpy(golden["z"])[None], torch.from_numpy(golden["pair_mask"])[None]
    want, keep = golden[f"{name}/out"], compared(name, golden)
    with torch.no_grad():
        got64 = call(name, module.double(), z.double(), pm.double())[0].numpy()
        got32 = call(name, module.float(), z, pm)[0].numpy()
    assert max_rel(got64[keep], want[keep]) < 1e-6  # the fixture is the fp64 result rounded to fp32
    assert max_rel(got32[keep], want[keep]) < 1e-5
    if name.startswith("tri_att"):  # the masked row in fp64: softmax(S), as stored
        assert max_rel(got64, want) < 1e-6


def test_pairformer_layer_matches_frozen_loops(golden):
    layer = build(R.PairformerLayer, golden, "pairformer_layer").double()
    z, s = torch.from_numpy(golden["z"]).double()[None], torch.from_numpy(golden["s"]).double()[None]
    tok, pm = torch.from_numpy(golden["token_mask"]).double()[None], torch.from_numpy(golden["pair_mask"]).double()[None]
    keep, open_tok = compared("pairformer_layer", golden), golden["token_mask"].astype(bool)
    dz_want = golden["pairformer_layer/z_out"].astype(np.float64) - golden["z"]
    for dtype in (torch.float64, torch.float32):
        lay = layer.to(dtype)
        with torch.no_grad():
            s_out, z_out = lay(s.to(dtype), z.to(dtype), tok.to(dtype), pm.to(dtype))
        dz = (z_out[0].double() - z[0]).numpy()
        bar = 1e-6 if dtype == torch.float64 else 1e-5
        assert max_rel(dz[keep], dz_want[keep]) < bar, dtype
        assert max_rel(s_out[0].double().numpy()[open_tok], golden["pairformer_layer/s_out"][open_tok]) < bar, dtype
    # the layer's update differs from any single branch's: the fixture covers the whole composition
    assert max_rel(dz[keep], golden["transition_z/out"][keep]) > 0.5


# ---------------------------------------------------------------- diffusion blocks

DIFFUSION = Path(__file__).resolve().parent / "golden" / "diffusion_blocks_n6.npz"
DIFFUSION_MODULES = {
    "adaln": lambda: R.AdaLN(768, 768),
    "conditioned_transition": lambda: R.ConditionedTransitionBlock(768, 768),
    "attention_pair_bias": lambda: R.AttentionPairBias(768, num_heads=16, compute_pair_bias=False),
}


@pytest.fixture(scope="module")
def golden_diffusion():
    with np.load(DIFFUSION, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def call_diffusion(name, module, t, dtype):
    a, s, bias, mask = (torch.from_numpy(t[k]).to(dtype) for k in ("a", "s", "bias", "mask"))
    if name == "attention_pair_bias":
        return module(s, bias, mask, s, multiplicity=int(t["multiplicity"]))
    return module(a, s)


@pytest.mark.parametrize("name", list(DIFFUSION_MODULES))
def test_diffusion_block_matches_frozen_loops(golden_diffusion, name):
    """The token transformer's blocks at width 768 (2 samples of 6 tokens;
    the attention with a given bias shared by the samples, one key masked)."""
    module = build(DIFFUSION_MODULES[name], golden_diffusion, name)
    want = golden_diffusion[f"{name}/out"]
    with torch.no_grad():
        got64 = call_diffusion(name, module.double(), golden_diffusion, torch.float64)
        got32 = call_diffusion(name, module.float(), golden_diffusion, torch.float32)
    assert max_rel(got64, want) < 1e-6
    assert max_rel(got32, want) < 1e-5
