"""The installed HIP path against the frozen self-fixtures of tests/golden
(fp64 explicit loops, production width, N = 6, a token masked in the middle):
the five pair modules and one PairformerLayer, each patched by ``install`` at
Boltz's module path and run as Boltz runs them (inference, bf16 autocast),
within the north star's bf16 bar; and the score model's width-768 blocks
(tests/golden/diffusion_blocks_n6.npz) in fp32 at the fp32 bar.  Attention
outputs are compared on the open pairs, the sequence stack on the open tokens
(the masked token's fully masked query row is a uniform softmax in fp32 /
bf16, softmax(S) in the fp64 loops; tests/test_golden.py)."""

from pathlib import Path

import numpy as np
import pytest
import torch
from torch import nn

from boltz_lumi_amd import adapters, ops
from oracle import boltz_ref as R

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "pair_modules_n6.npz"
TOL = 2e-2

MODULES = {
    "tri_mul_out": lambda: R.TriangleMultiplicationOutgoing(128),
    "tri_mul_in": lambda: R.TriangleMultiplicationIncoming(128),
    "tri_att_start": lambda: R.TriangleAttention(128, 32, 4),
    "tri_att_end": lambda: R.TriangleAttentionEndingNode(128, 32, 4),
    "transition_z": lambda: R.Transition(128, 512),
}


class Boltz2(nn.Module):
    """Stand-in with the trunk's module path for one PairformerLayer."""

    def __init__(self, layer):
        super().__init__()
        self.pairformer_module = nn.Module()
        self.pairformer_module.layers = nn.ModuleList([layer])


@pytest.fixture(scope="module")
def golden():
    with np.load(GOLDEN, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


@pytest.fixture()
def native_calls(monkeypatch):
    counts = {}
    for name in ("trimul", "triattn", "pair_transition"):
        original = getattr(ops, name)

        def counted(*args, _name=name, _original=original, **kwargs):
            counts[_name] = counts.get(_name, 0) + 1
            return _original(*args, **kwargs)

        monkeypatch.setattr(ops, name, counted)
    return counts


def seeded(ctor, golden, name):
    module = R.randomize(ctor(), generator=torch.Generator().manual_seed(int(golden[f"{name}/seed"])))
    flat = torch.cat([p.detach().double().flatten() for p in module.parameters()])
    np.testing.assert_allclose([flat.sum().item(), (flat * flat).sum().item()], golden[f"{name}/weight_stats"],
                               rtol=1e-12, atol=1e-9)
    return module.eval()


def max_rel(got, want):
    got, want = np.asarray(got, dtype=np.float64), np.asarray(want, dtype=np.float64)
    return float(np.abs(got - want).max() / np.abs(want).max())


def test_installed_pair_modules_match_frozen_loops(golden, gpu, native_calls):
    layer = R.PairformerLayer()
    for name, ctor in MODULES.items():
        setattr(layer, name, seeded(ctor, golden, name))
    model = Boltz2(layer).to(gpu).eval()
    adapters.install(model)
    try:
        z = torch.from_numpy(golden["z"]).to(gpu)[None]
        pm = torch.from_numpy(golden["pair_mask"]).to(gpu)[None]
        keep_attn = golden["pair_mask"].astype(bool)
        with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
            for name in MODULES:
                mod = getattr(layer, name)
                if name.startswith("tri_att"):
                    got = mod(z, pm, chunk_size=None)
                elif name.startswith("tri_mul"):
                    got = mod(z, pm)
                else:
                    got = mod(z)
                got = got[0].float().cpu().numpy()
                want = golden[f"{name}/out"]
                keep = keep_attn if name.startswith("tri_att") else np.ones_like(keep_attn)
                err = max_rel(got[keep], want[keep])
                print(f"golden {name}: max_rel {err:.2e}", flush=True)
                assert err < TOL, name
    finally:
        adapters.uninstall(model)
    assert native_calls == {"trimul": 2, "triattn": 2, "pair_transition": 1}


def test_installed_pairformer_layer_matches_frozen_loops(golden, gpu, native_calls):
    layer = seeded(R.PairformerLayer, golden, "pairformer_layer")
    model = Boltz2(layer).to(gpu).eval()
    adapters.install(model)
    try:
        z = torch.from_numpy(golden["z"]).to(gpu)[None]
        s = torch.from_numpy(golden["s"]).to(gpu)[None]
        tok = torch.from_numpy(golden["token_mask"]).to(gpu)[None]
        pm = torch.from_numpy(golden["pair_mask"]).to(gpu)[None]
        with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
            s_out, z_out = layer(s, z, tok, pm)
    finally:
        adapters.uninstall(model)
    assert native_calls == {"trimul": 2, "triattn": 2, "pair_transition": 1}
    keep, open_tok = golden["pair_mask"].astype(bool), golden["token_mask"].astype(bool)
    dz = z_out[0].double().cpu().numpy() - golden["z"]
    dz_want = golden["pairformer_layer/z_out"].astype(np.float64) - golden["z"]
    err_z = max_rel(dz[keep], dz_want[keep])
    err_s = max_rel(s_out[0].double().cpu().numpy()[open_tok], golden["pairformer_layer/s_out"][open_tok])
    print(f"golden pairformer_layer: z update max_rel {err_z:.2e}, s max_rel {err_s:.2e}", flush=True)
    assert err_z < TOL and err_s < TOL


DIFFUSION = Path(__file__).resolve().parent / "golden" / "diffusion_blocks_n6.npz"


def test_installed_diffusion_blocks_match_frozen_loops(gpu, monkeypatch):
    """The score model's token-transformer blocks at width 768 through the
    installed forwards in fp32 (autocast off, as the reference runs the score
    model): AdaLN and ConditionedTransitionBlock patched by ``install`` at
    ``structure_module.score_model``, the attention through
    ``pair_bias.prepared_forward`` (its patched forward); the fp32-mode bar
    1e-4 against the frozen fp64 loops."""
    from boltz_lumi_amd.pair_bias import prepared_forward

    with np.load(DIFFUSION, allow_pickle=False) as f:
        t = {k: f[k] for k in f.files}
    counts = {}
    for name in ("adaln_modulate", "epilogue", "seq_attention_batched"):
        original = getattr(ops, name)

        def counted(*args, _name=name, _original=original, **kwargs):
            counts[_name] = counts.get(_name, 0) + 1
            return _original(*args, **kwargs)

        monkeypatch.setattr(ops, name, counted)
    host = nn.Module()
    host.structure_module = nn.Module()
    host.structure_module.score_model = sm = nn.Module()
    sm.adaln = seeded(lambda: R.AdaLN(768, 768), t, "adaln")
    sm.transition = seeded(lambda: R.ConditionedTransitionBlock(768, 768), t, "conditioned_transition")
    apb = seeded(lambda: R.AttentionPairBias(768, num_heads=16, compute_pair_bias=False), t, "attention_pair_bias")
    host = host.to(gpu).eval()
    apb = apb.to(gpu)
    a, s, bias, mask = (torch.from_numpy(t[k]).to(gpu) for k in ("a", "s", "bias", "mask"))
    adapters.install(host, require_boltz2=False)
    try:
        assert "forward" in vars(sm.adaln) and "forward" in vars(sm.transition)
        with torch.inference_mode():
            got = {"adaln": sm.adaln(a, s), "conditioned_transition": sm.transition(a, s),
                   "attention_pair_bias": prepared_forward(apb, s, bias, mask, s, int(t["multiplicity"]))}
    finally:
        adapters.uninstall(host)
    assert counts.get("adaln_modulate", 0) >= 2 and counts.get("epilogue", 0) >= 2
    assert counts.get("seq_attention_batched", 0) == 1
    for name, out in got.items():
        err = max_rel(out.float().cpu().numpy(), t[f"{name}/out"])
        print(f"golden {name}: max_rel {err:.2e}", flush=True)
        assert err < 1e-4, name
