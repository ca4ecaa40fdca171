"""GPU tests of the pair stacks outside the trunk: the MSA module's and the
template module's ``PairformerNoSeqLayer`` and the confidence module's
``PairformerLayer``.  ``install`` patches them by class name and by the
``.transition_z`` suffix, as the reference does (adapters.py:24-45), so the
128-channel stacks (MSA, confidence) run the fused kernels; the template
stack (64 channels, one batch element per template) keeps the upstream
triangle forwards, whose guards need 128 channels in the reference too
(multiplication.py:57, triangle.py:35-75), and runs its 64 -> 256 -> 64
transition through the reference's composition with the native SiLU-product
kernel (pair_transition.py:20-28).  Outputs are compared with the upstream
fp32 math at the north star's bf16 tolerance, on the residual update so that
the unchanged part of z does not hide errors.  The sizes are small; the
kernels' full-size cases are covered by the trunk tests."""

import pytest
import torch
from torch import nn

from boltz_lumi_amd import adapters, ops
from oracle import boltz_ref as R

pytestmark = pytest.mark.gpu

TOL = 2e-2


class Boltz2(nn.Module):
    """Stand-in with upstream Boltz-2's module paths for the three stacks."""

    def __init__(self):
        super().__init__()
        self.msa_module = nn.Module()
        msa_layer = nn.Module()
        msa_layer.pairformer_layer = R.PairformerNoSeqLayer(128)
        msa_layer.msa_transition = R.Transition(64, 256)  # not a pair transition: left alone
        self.msa_module.layers = nn.ModuleList([msa_layer])
        self.template_module = nn.Module()
        self.template_module.pairformer = nn.Module()
        self.template_module.pairformer.layers = nn.ModuleList([R.PairformerNoSeqLayer(64)])
        self.confidence_module = nn.Module()
        self.confidence_module.pairformer_stack = nn.Module()
        self.confidence_module.pairformer_stack.layers = nn.ModuleList([R.PairformerLayer()])


def rel(got, want, base):
    """max |(got - base) - (want - base)| / max |want - base|"""
    d_got, d_want = got.double() - base.double(), want.double() - base.double()
    return ((d_got - d_want).abs().max() / d_want.abs().max()).item()


@pytest.fixture()
def model(gpu):
    torch.manual_seed(20260)
    m = R.randomize(Boltz2()).to(gpu).eval()
    yield m
    adapters.uninstall(m)


@pytest.fixture()
def calls(monkeypatch):
    """Counts the native entry points the patched forwards reach."""
    counts = {}
    for name in ("trimul", "triattn", "pair_transition", "silu_mul"):
        original = getattr(ops, name)

        def counted(*args, _name=name, _original=original, **kwargs):
            counts[_name] = counts.get(_name, 0) + 1
            return _original(*args, **kwargs)

        monkeypatch.setattr(ops, name, counted)
    return counts


def pair_mask(b, n, masked, gpu):
    m = torch.ones(b, n, device=gpu)
    if masked:
        m[:, -masked:] = 0
    return m[:, :, None] * m[:, None, :], m


def test_install_patches_every_pair_stack(model):
    assert adapters.install(model) == 18  # each of the three stacks: the layer and its 5 pair modules
    layer = model.msa_module.layers[0]
    assert "forward" in vars(layer.pairformer_layer)
    assert "forward" in vars(model.confidence_module.pairformer_stack.layers[0])
    assert "forward" in vars(layer.pairformer_layer.transition_z)
    assert "forward" not in vars(layer.msa_transition)
    assert "forward" in vars(model.template_module.pairformer.layers[0].tri_att_start)


def test_msa_stack_runs_native(model, gpu, calls):
    layer = model.msa_module.layers[0].pairformer_layer
    n = 96
    z = torch.randn(1, n, n, 128, device=gpu) * 0.5
    pm, _ = pair_mask(1, n, 5, gpu)
    with torch.inference_mode():
        want = layer(z, pm)
    adapters.install(model)
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
        got = layer(z, pm)
    assert calls == {"trimul": 2, "triattn": 2, "pair_transition": 1}
    assert torch.isfinite(got).all()
    assert rel(got, want, z) < TOL


def test_template_stack_transition_native_triangles_upstream(model, gpu, calls):
    layer = model.template_module.pairformer.layers[0]
    templates, n = 2, 80
    z = torch.randn(templates, n, n, 64, device=gpu) * 0.5
    pm, _ = pair_mask(templates, n, 3, gpu)
    with torch.inference_mode():
        want = layer(z, pm)
        want_t = layer.transition_z(z)
    adapters.install(model)
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
        got = layer(z, pm)
        got_t = layer.transition_z(z)
    assert calls == {"silu_mul": 2}
    assert got_t.dtype == torch.bfloat16
    assert ((got_t.double() - want_t.double()).abs().max() / want_t.double().abs().max()).item() < TOL
    assert torch.isfinite(got).all()
    assert rel(got, want, z) < TOL


def test_confidence_stack_runs_native(model, gpu, calls):
    layer = model.confidence_module.pairformer_stack.layers[0]
    n = 64
    s = torch.randn(1, n, 384, device=gpu)
    z = torch.randn(1, n, n, 128, device=gpu) * 0.5
    pm, mask = pair_mask(1, n, 4, gpu)
    with torch.inference_mode():
        want_s, want_z = layer(s, z, mask, pm)
    adapters.install(model)
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
        got_s, got_z = layer(s, z, mask, pm)
    assert calls == {"trimul": 2, "triattn": 2, "pair_transition": 1}
    assert rel(got_z, want_z, z) < TOL
    # The installed layer runs the sequence stack in fp32 with autocast off, as
    # upstream does (the pair bias from the transition's epilogue, the fused
    # attention): its update of s is checked against the fp32 oracle's.
    assert got_s.dtype == torch.float32
    assert rel(got_s, want_s, s) < TOL


def test_batched_pair_modules_match_per_element_calls(model, gpu):
    """Batch of two with different masks: every patched pair module loops over
    the batch with one shared workspace, so element b of the batched call must
    equal the call on element b alone, bit for bit, and both match upstream."""
    layer = model.msa_module.layers[0].pairformer_layer
    n = 72
    z = torch.randn(2, n, n, 128, device=gpu) * 0.5
    m = torch.ones(2, n, device=gpu)
    m[0, -7:] = 0
    m[1, :3] = 0
    m[1, 40:45] = 0
    pm = m[:, :, None] * m[:, None, :]
    calls = {
        "tri_mul_out": lambda mod, x, p: mod(x, p),
        "tri_mul_in": lambda mod, x, p: mod(x, p),
        "tri_att_start": lambda mod, x, p: mod(x, p, chunk_size=None),
        "tri_att_end": lambda mod, x, p: mod(x, p, chunk_size=None),
        "transition_z": lambda mod, x, p: mod(x),
    }
    with torch.inference_mode():
        want = {k: f(getattr(layer, k), z, pm) for k, f in calls.items()}
    adapters.install(model)
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
        for k, f in calls.items():
            mod = getattr(layer, k)
            got = f(mod, z, pm)
            assert got.dtype == torch.bfloat16, k
            for b in range(2):
                alone = f(mod, z[b:b + 1].contiguous(), pm[b:b + 1].contiguous())
                assert torch.equal(got[b], alone[0]), (k, b)
                w = want[k][b].double()
                assert ((got[b].double() - w).abs().max() / w.abs().max()).item() < TOL, (k, b)


def test_batched_installed_layers_match_per_element_calls(model, gpu, calls):
    """The installed whole-layer forwards on a batch of two with different
    token masks: element b equals the call on element b alone, bit for bit
    (one workspace shared by the batch loop, per-element masks and dropout
    row scales), and both layers match upstream's fp32 forward."""
    n = 80
    m = torch.ones(2, n, device=gpu)
    m[0, -6:] = 0
    m[1, 10:14] = 0
    pm = m[:, :, None] * m[:, None, :]
    s = torch.randn(2, n, 384, device=gpu)
    z = torch.randn(2, n, n, 128, device=gpu) * 0.5
    conf = model.confidence_module.pairformer_stack.layers[0]
    msa = model.msa_module.layers[0].pairformer_layer
    with torch.inference_mode():
        want_s, want_z = conf(s, z, m, pm)
        want_msa = msa(z, pm)
    adapters.install(model)
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
        got_s, got_z = conf(s, z, m, pm)
        got_msa = msa(z, pm)
        # the native pair stack ran for both elements of both layers
        assert calls == {"trimul": 8, "triattn": 8, "pair_transition": 4}
        for b in range(2):
            one = slice(b, b + 1)
            alone_s, alone_z = conf(s[one].contiguous(), z[one].contiguous(), m[one].contiguous(),
                                    pm[one].contiguous())
            assert torch.equal(got_z[b], alone_z[0]) and torch.equal(got_s[b], alone_s[0]), b
            assert torch.equal(got_msa[b], msa(z[one].contiguous(), pm[one].contiguous())[0]), b
    for b in range(2):
        assert rel(got_z[b], want_z[b], z[b]) < TOL, b
        assert rel(got_s[b], want_s[b], s[b]) < TOL, b
        assert rel(got_msa[b], want_msa[b], z[b]) < TOL, b
