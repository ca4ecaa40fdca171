"""BASELINE configs[4] on the GPU: the diffusion score model's transformer
stacks (atom encoder 3 blocks and atom decoder 3 blocks at 5 x 8192 atoms x
128 in windows of 32 queries over 128 keys, token transformer 24 blocks at
5 x 1024 tokens x 768 with 16 heads and a prepacked bias shared by the 5
samples) through the installed adapters, against the fp32 CPU oracle at the
north star's fp32-mode bar of 1e-4.

Weights are N(0, 1 / fan_in) with LayerNorm weights N(1, 0.08): with the
reference tests' N(0, 0.08) every 768-wide block would amplify its residual
stream about a hundredfold."""

import copy
import math

import pytest
import torch
from torch import nn

from boltz_lumi_amd import adapters, ops
from boltz_lumi_amd.pair_bias import prepare_token_bias
from oracle import boltz_ref as R

pytestmark = pytest.mark.gpu

SAMPLES, TOKENS, ATOMS = 5, 1024, 8192
W, H = 32, 128


def fan_in_init(module, seed):
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in module.named_parameters():
            if "norm" in name and name.endswith("weight"):
                p.copy_(1 + 0.08 * torch.randn(p.shape, generator=g))
            elif p.dim() == 2:
                p.copy_(torch.randn(p.shape, generator=g) / math.sqrt(p.shape[1]))
            else:
                p.copy_(0.08 * torch.randn(p.shape, generator=g))
    return module


def max_rel(got, want):
    got, want = got.double().cpu(), want.double().cpu()
    return ((got - want).abs().max() / want.abs().max()).item()


def step_inputs(seed, device, token_pad=16, atom_pad=40):
    """One denoiser step's inputs at configs[4] shapes (CPU-generated, then moved)."""
    g = torch.Generator().manual_seed(seed)
    nw = ATOMS // W
    t = dict(
        r=torch.randn(SAMPLES, ATOMS, 3, generator=g) * 160.0,  # noisy coordinates at sigma 160
        q=torch.randn(SAMPLES, ATOMS, 128, generator=g),
        c=torch.randn(SAMPLES, ATOMS, 128, generator=g),
        atom_mask=torch.ones(SAMPLES, ATOMS),
        enc_bias=torch.randn(1, nw, W, H, 3 * 4, generator=g),
        dec_bias=torch.randn(1, nw, W, H, 3 * 4, generator=g),
        a=torch.randn(SAMPLES, TOKENS, 768, generator=g),
        s=torch.randn(SAMPLES, TOKENS, 768, generator=g),
        token_bias=torch.randn(1, TOKENS, TOKENS, 24 * 16, generator=g),
        token_mask=torch.ones(SAMPLES, TOKENS),
    )
    if atom_pad:
        t["atom_mask"][:, -atom_pad:] = 0
    if token_pad:
        t["token_mask"][:, -token_pad:] = 0
    return {k: v.to(device) for k, v in t.items()}


def run_stacks(stacks, t, token_bias, index):
    def to_keys(x):
        return R.single_to_keys(x, index, W, H)

    return stacks(t["r"], t["q"], t["c"], t["atom_mask"], t["enc_bias"], t["dec_bias"], to_keys, t["a"], t["s"], token_bias,
                  t["token_mask"], multiplicity=SAMPLES)


def test_configs4_stacks_match_fp32_oracle(gpu, monkeypatch):
    ref = fan_in_init(R.DiffusionStacks(), 0).eval()
    host = nn.Module()  # the stacks at their Boltz paths, so install() selects them
    host.structure_module = nn.Module()
    host.structure_module.score_model = copy.deepcopy(ref).to(gpu)
    patched = adapters.install(host, require_boltz2=False)
    layers = 24 + 3 + 3
    # per layer: the layer, AdaLN, the transition's AdaLN, the transition, the attention; the three stacks and
    # the two atom transformers
    assert patched == 5 * layers + 3 + 2
    launches, windowed = [], []
    original, original_w = ops.seq_attention_batched, ops.seq_attention_windowed
    monkeypatch.setattr(ops, "seq_attention_batched", lambda *a, **k: launches.append(1) or original(*a, **k))
    monkeypatch.setattr(ops, "seq_attention_windowed", lambda *a, **k: windowed.append(1) or original_w(*a, **k))

    t_cpu = step_inputs(7, "cpu")
    print("configs[4] stacks: CPU oracle, 5 samples", flush=True)
    with torch.inference_mode():
        index = R.get_indexing_matrix(ATOMS // W, W, H)
        r_ref, q_ref, a_ref = run_stacks(ref, t_cpu, t_cpu["token_bias"], index)
    print("configs[4] stacks: native", flush=True)
    t = {k: v.to(gpu) for k, v in t_cpu.items()}
    with torch.inference_mode():
        packed = prepare_token_bias(t["token_bias"])  # what optimized_sample hands the token transformer
        r_got, q_got, a_got = run_stacks(host.structure_module.score_model, t, packed, index.to(gpu))
    torch.cuda.synchronize()
    # every attention ran on a fused kernel; the atom transformers' read their key windows by address
    assert len(launches) == 24 and len(windowed) == 6
    err_r, err_q, err_a = max_rel(r_got, r_ref), max_rel(q_got, q_ref), max_rel(a_got, a_ref)
    print(f"configs[4] stacks max_rel: coordinate update {err_r:.2e}, atoms {err_q:.2e}, tokens {err_a:.2e}",
          flush=True)
    assert err_r < 1e-4 and err_q < 1e-4 and err_a < 1e-4
    adapters.uninstall(host)
