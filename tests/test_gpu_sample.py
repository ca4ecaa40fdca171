"""``diffusion.optimized_sample`` is the class ``sample`` (reference
tests/test_atom_conditioning.py:131-164): on a stand-in sampler whose loop
draws its noise from torch's generators and whose score model runs atom
encoder / decoder DiffusionTransformerLayers on the fixed conditioning, the
wrapper returns bit-identical coordinates and leaves the CPU and GPU
generator states where the class ``sample`` leaves them.  With one sample of
one structure the atom conditioning cache is active during the call (each
conditioning projection computed once); with several samples it is not;
with grad enabled the wrapper passes the call through untouched."""

import pytest
import torch
from torch import nn

from boltz_lumi_amd.diffusion import optimized_sample
from oracle import boltz_ref as R

pytestmark = pytest.mark.gpu

ATOMS, DIM, HEADS, DEPTH = 24, 32, 4, 2


class ScoreModel(nn.Module):
    def __init__(self):
        super().__init__()
        self.embed = nn.Linear(3, DIM, bias=False)
        self.atom_attention_encoder = nn.Module()
        self.atom_attention_encoder.atom_encoder = nn.Module()
        self.atom_attention_encoder.atom_encoder.diffusion_transformer = nn.Module()
        self.atom_attention_encoder.atom_encoder.diffusion_transformer.layers = nn.ModuleList(
            [R.DiffusionTransformerLayer(HEADS, DIM, DIM) for _ in range(DEPTH)])
        self.atom_attention_decoder = nn.Module()
        self.atom_attention_decoder.atom_decoder = nn.Module()
        self.atom_attention_decoder.atom_decoder.diffusion_transformer = nn.Module()
        self.atom_attention_decoder.atom_decoder.diffusion_transformer.layers = nn.ModuleList(
            [R.DiffusionTransformerLayer(HEADS, DIM, DIM) for _ in range(DEPTH)])
        self.out = nn.Linear(DIM, 3, bias=False)

    def stacks(self):
        return (*self.atom_attention_encoder.atom_encoder.diffusion_transformer.layers,
                *self.atom_attention_decoder.atom_decoder.diffusion_transformer.layers)


class Sampler(nn.Module):
    """A structure-module stand-in with an EDM-like loop: Gaussian start at
    sigma 160, fresh noise every step, the score model's update added."""

    def __init__(self):
        super().__init__()
        self.score_model = ScoreModel()

    def sample(self, atom_mask, num_sampling_steps=6, multiplicity=1, diffusion_conditioning=None, **kwargs):
        c = diffusion_conditioning["c"].repeat_interleave(multiplicity, 0)
        bias = diffusion_conditioning["token_trans_bias"]
        mask = atom_mask.repeat_interleave(multiplicity, 0).float()
        coords = 160.0 * torch.randn(mask.shape[0], ATOMS, 3, device=mask.device)
        self.cache_active, self.bias_seen = [], bias
        for step in range(num_sampling_steps):
            sigma = 160.0 * 0.5 ** step
            noise = torch.randn_like(coords) * sigma * 0.1
            q = self.score_model.embed(coords / (sigma ** 2 + 256.0) ** 0.5)
            for i, layer in enumerate(self.score_model.stacks()):
                sl = bias[..., HEADS * i:HEADS * (i + 1)].repeat_interleave(multiplicity, 0)
                q = layer(q, c, sl, mask)
            self.cache_active.append("forward" in vars(self.score_model.stacks()[0].adaln.s_scale))
            coords = coords + noise + self.score_model.out(q)
        return {"sample_atom_coords": coords}


@pytest.fixture()
def sampler(gpu):
    torch.manual_seed(4021)
    return R.randomize(Sampler(), std=0.07).to(gpu).eval()


def conditioning(gpu, batch=1):
    g = torch.Generator().manual_seed(5)
    return {"c": torch.randn(batch, ATOMS, DIM, generator=g).to(gpu),
            "token_trans_bias": torch.randn(batch, ATOMS, ATOMS, 2 * DEPTH * HEADS, generator=g).to(gpu)}


def run(fn, sampler, gpu, multiplicity, grad=False):
    torch.manual_seed(99)
    torch.cuda.manual_seed(99)
    mask = torch.ones(1, ATOMS, device=gpu)
    mask[:, -3:] = 0
    cond = conditioning(gpu)
    with torch.set_grad_enabled(grad), torch.inference_mode(not grad):
        out = fn(sampler, atom_mask=mask, num_sampling_steps=6, multiplicity=multiplicity,
                 diffusion_conditioning=cond)
    return out["sample_atom_coords"], torch.get_rng_state(), torch.cuda.get_rng_state(), cond


@pytest.mark.parametrize("multiplicity", [1, 2])
def test_optimized_sample_is_the_class_sample(sampler, gpu, multiplicity):
    want, cpu_rng, gpu_rng, _ = run(type(sampler).sample, sampler, gpu, multiplicity)
    assert sampler.cache_active == [False] * 6
    s_norm = sampler.score_model.stacks()[0].adaln.s_norm
    calls = []
    original = s_norm.forward
    s_norm.forward = lambda x: (calls.append(1), original(x))[1]
    try:
        got, cpu_rng2, gpu_rng2, cond = run(optimized_sample, sampler, gpu, multiplicity)
    finally:
        del s_norm.forward
    assert torch.equal(got, want)
    assert torch.equal(cpu_rng2, cpu_rng) and torch.equal(gpu_rng2, gpu_rng)
    single = multiplicity == 1
    assert sampler.cache_active == [single] * 6  # the cache engages for one sample of one structure only
    assert len(calls) == (1 if single else 6)  # once per call with the cache, once per step without
    seen = sampler.bias_seen
    assert torch.equal(seen, cond["token_trans_bias"]) and seen is not cond["token_trans_bias"]
    assert seen.movedim(-1, 1)[0].is_contiguous()  # packed head-major
    assert all("forward" not in vars(m) for m in sampler.modules())  # the cache restored every forward


def test_optimized_sample_passes_through_with_grad(sampler, gpu):
    want, cpu_rng, gpu_rng, _ = run(type(sampler).sample, sampler, gpu, 1, grad=True)
    got, cpu_rng2, gpu_rng2, cond = run(optimized_sample, sampler, gpu, 1, grad=True)
    assert torch.equal(got, want) and got.requires_grad
    assert torch.equal(cpu_rng2, cpu_rng) and torch.equal(gpu_rng2, gpu_rng)
    assert sampler.bias_seen is cond["token_trans_bias"]  # not repacked
    assert sampler.cache_active == [False] * 6
