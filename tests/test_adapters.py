"""CPU tests of the drop-in boundary: install gating, idempotency, fallback to
the upstream forward (values and gradients), uninstall, and the conditioning
cache's restore-on-exception (reference tests/test_operator_additions.py:97-105,
139-147 and tests/test_atom_conditioning.py:106-111)."""

from types import SimpleNamespace

import pytest
import torch
from torch import nn

import boltz_lumi_amd
from boltz_lumi_amd import adapters
from boltz_lumi_amd.atom_conditioning import atom_conditioning_cache
from oracle import boltz_ref as R


class Boltz2(nn.Module):
    """Stand-in with the module paths adapters.install walks."""

    def __init__(self):
        super().__init__()
        self.pairformer_module = nn.Module()
        self.pairformer_module.layers = nn.ModuleList([R.PairformerLayer(token_s=32, token_z=128, num_heads=4)])
        self.structure_module = nn.Module()
        self.structure_module.score_model = nn.Module()
        self.structure_module.score_model.block = R.ConditionedTransitionBlock(16, 8)


def test_version_pin():
    assert boltz_lumi_amd.SUPPORTED_BOLTZ_VERSION == "2.2.1"
    assert boltz_lumi_amd.__version__.startswith("2.2.1.")


def test_install_requires_boltz2_and_gfx950():
    assert adapters.install(nn.Linear(2, 2)) == 0
    model = Boltz2()
    if not torch.cuda.is_available():
        assert adapters.install(model) == 0  # no gfx950 device: no-op
        assert not getattr(model, adapters.FLAG, False)


def test_install_patches_by_class_and_path_and_is_idempotent():
    model = Boltz2()
    n = adapters.install(model, require_device=False)
    # tri_mul_out, tri_mul_in, tri_att_start, tri_att_end, transition_z, AdaLN, CTB
    assert n == 7
    layer = model.pairformer_module.layers[0]
    assert "forward" in vars(layer.tri_att_start) and "forward" in vars(layer.tri_att_start.layer_norm)
    assert "forward" in vars(layer.transition_z) and "forward" not in vars(layer.transition_s)
    assert adapters.install(model, require_device=False) == 0
    assert adapters.uninstall(model) >= 7
    assert "forward" not in vars(layer.tri_att_start)


def test_cpu_tensors_fall_back_to_upstream_exactly():
    torch.manual_seed(0)
    model = Boltz2()
    R.randomize(model)
    layer = model.pairformer_module.layers[0]
    n = 6
    z = torch.randn(1, n, n, 128)
    s = torch.randn(1, n, 32)
    mask = torch.ones(1, n)
    mask[:, -1] = 0
    pm = mask[:, :, None] * mask[:, None, :]
    with torch.no_grad():
        want = layer(s, z, mask, pm)
    adapters.install(model, require_device=False)
    with torch.no_grad():
        got = layer(s, z, mask, pm)
    assert all(torch.equal(a, b) for a, b in zip(got, want))


def test_grad_mode_falls_back_with_equal_gradients():
    torch.manual_seed(1)
    tm = R.randomize(R.TriangleMultiplicationOutgoing(128))
    x = torch.randn(1, 3, 3, 128, requires_grad=True)
    mask = torch.ones(1, 3, 3)
    want = tm(x, mask)
    gw = torch.autograd.grad(want.sum(), x)[0]
    from boltz_lumi_amd.multiplication import normalized_forward

    got = normalized_forward(tm, x, mask)
    gg = torch.autograd.grad(got.sum(), x)[0]
    assert torch.equal(got, want) and torch.equal(gg, gw)


def test_conditioning_cache_restores_forwards_after_exception():
    layers = [R.DiffusionTransformerLayer(2, 16, 8) for _ in range(2)]
    score = SimpleNamespace(
        atom_attention_encoder=SimpleNamespace(atom_encoder=SimpleNamespace(
            diffusion_transformer=SimpleNamespace(layers=layers[:1]))),
        atom_attention_decoder=SimpleNamespace(atom_decoder=SimpleNamespace(
            diffusion_transformer=SimpleNamespace(layers=layers[1:]))),
    )
    before = [vars(m).get("forward") for m in (layers[0].adaln.s_norm, layers[1].transition.output_projection[0])]
    with pytest.raises(RuntimeError, match="boom"):
        with atom_conditioning_cache(score):
            assert "forward" in vars(layers[0].adaln.s_norm)
            raise RuntimeError("boom")
    after = [vars(m).get("forward") for m in (layers[0].adaln.s_norm, layers[1].transition.output_projection[0])]
    assert before == after == [None, None]


def test_conditioning_cache_is_inert_on_cpu():
    layer = R.DiffusionTransformerLayer(2, 16, 8)
    score = SimpleNamespace(
        atom_attention_encoder=SimpleNamespace(atom_encoder=SimpleNamespace(
            diffusion_transformer=SimpleNamespace(layers=[layer]))),
        atom_attention_decoder=SimpleNamespace(atom_decoder=SimpleNamespace(
            diffusion_transformer=SimpleNamespace(layers=[]))),
    )
    calls = []
    original = layer.adaln.s_norm.forward

    def counting(x):
        calls.append(1)
        return original(x)

    layer.adaln.s_norm.forward = counting
    s = torch.randn(3, 8)
    with torch.no_grad(), atom_conditioning_cache(score):
        layer.adaln.s_norm(s)
        layer.adaln.s_norm(s)
    assert len(calls) == 2  # CPU inputs are never cached
    assert layer.adaln.s_norm.forward is counting
