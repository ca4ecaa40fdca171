"""Writes tests/golden/pair_modules_n6.npz: frozen input / output vectors of
the Pairformer pair modules and one whole PairformerLayer at their production
widths (128 pair channels, 384 single channels) and N = 6 tokens, and
tests/golden/diffusion_blocks_n6.npz: the score model's token-transformer
blocks at their width (768) for 2 samples of 6 tokens (AdaLN,
ConditionedTransitionBlock, AttentionPairBias with a given bias, multiplicity
2, one key masked).  The outputs are evaluated by the fp64 explicit-loop
restatement (oracle/brute.py) on the stored fp32 inputs.

The reference ships no golden vectors (its tests run live upstream Boltz on a
GPU), so these are self-fixtures: they freeze the oracle and the product
against refactors; what pins the oracle to upstream is tests/test_oracle_pins.py.

Weights are not stored.  Each module is initialised by
``oracle.boltz_ref.randomize`` from the seed stored with it, and the sum and
sum of squares of its parameters are stored too, so a changed initialisation
fails loudly instead of comparing different modules.

Run from the repository root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import boltz_ref as R  # noqa: E402
from oracle import brute as B  # noqa: E402

OUT = Path(__file__).resolve().parent / "pair_modules_n6.npz"
N = 6
MASKED_TOKEN = 3  # a token in the middle, so the masked rows and columns are not a suffix

# case -> (constructor, seed)
MODULES = {
    "tri_mul_out": (lambda: R.TriangleMultiplicationOutgoing(128), 101),
    "tri_mul_in": (lambda: R.TriangleMultiplicationIncoming(128), 102),
    "tri_att_start": (lambda: R.TriangleAttention(128, 32, 4), 103),
    "tri_att_end": (lambda: R.TriangleAttentionEndingNode(128, 32, 4), 104),
    "transition_z": (lambda: R.Transition(128, 512), 105),
}
LAYER_SEED = 106


def build(ctor, seed):
    return R.randomize(ctor(), generator=torch.Generator().manual_seed(seed)).double().eval()


def weight_stats(module):
    ps = [p.detach().double().flatten() for p in module.parameters()]
    flat = torch.cat(ps)
    return np.array([flat.sum().item(), (flat * flat).sum().item()])


def brute_module(name, module, z, pm):
    if name.startswith("tri_mul"):
        return B.triangle_multiplication(module, z, pm, outgoing=name.endswith("out"))
    if name.startswith("tri_att"):
        return B.triangle_attention(module, z, pm, starting=name.endswith("start"))
    return B.transition(module, z)


def brute_layer(layer, s, z, mask, pm):
    """PairformerLayer in eval: the five pair branches chained on z, then the
    sequence stack on the updated z (s_post_norm is the identity)."""
    for name in MODULES:
        z = z + brute_module(name, getattr(layer, name), z, pm)
    w, b = B._p(layer, "pre_norm_s.weight"), B._p(layer, "pre_norm_s.bias")
    sn = np.array([B.layer_norm_vec(list(r), w, b, layer.pre_norm_s.eps) for r in s])[None]
    s1 = s[None] + B.attention_pair_bias(layer.attention, sn, z[None], mask[None], sn)
    s2 = s1 + B.transition(layer.transition_s, s1)
    return s2[0], z


def main():
    g = torch.Generator().manual_seed(100)
    z = torch.randn(N, N, 128, generator=g).numpy()
    s = torch.randn(N, 384, generator=g).numpy()
    tok = np.ones(N, dtype=np.float32)
    tok[MASKED_TOKEN] = 0
    pm = (tok[:, None] * tok[None, :]).astype(np.float32)
    data = {"z": z, "s": s, "token_mask": tok, "pair_mask": pm}
    z64, s64, pm64, tok64 = (a.astype(np.float64) for a in (z, s, pm, tok))
    for name, (ctor, seed) in MODULES.items():
        module = build(ctor, seed)
        print(f"{name}: fp64 loops", flush=True)
        data[f"{name}/seed"] = np.array(seed)
        data[f"{name}/weight_stats"] = weight_stats(module)
        data[f"{name}/out"] = np.asarray(brute_module(name, module, z64, pm64), dtype=np.float32)
    layer = build(R.PairformerLayer, LAYER_SEED)
    print("pairformer_layer: fp64 loops", flush=True)
    s_out, z_out = brute_layer(layer, s64, z64, tok64, pm64)
    data["pairformer_layer/seed"] = np.array(LAYER_SEED)
    data["pairformer_layer/weight_stats"] = weight_stats(layer)
    data["pairformer_layer/s_out"] = np.asarray(s_out, dtype=np.float32)
    data["pairformer_layer/z_out"] = np.asarray(z_out, dtype=np.float32)
    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")
    diffusion_blocks()


DIFFUSION_OUT = Path(__file__).resolve().parent / "diffusion_blocks_n6.npz"
# case -> (constructor, seed)
DIFFUSION_MODULES = {
    "adaln": (lambda: R.AdaLN(768, 768), 201),
    "conditioned_transition": (lambda: R.ConditionedTransitionBlock(768, 768), 202),
    "attention_pair_bias": (lambda: R.AttentionPairBias(768, num_heads=16, compute_pair_bias=False), 203),
}
MULTIPLICITY = 2


def diffusion_blocks():
    g = torch.Generator().manual_seed(200)
    a = torch.randn(MULTIPLICITY, N, 768, generator=g).numpy()
    s = torch.randn(MULTIPLICITY, N, 768, generator=g).numpy()
    bias = torch.randn(1, N, N, 16, generator=g).numpy()  # [B / multiplicity, Q, K, H], shared by the samples
    mask = np.ones((MULTIPLICITY, N), dtype=np.float32)
    mask[1, 2] = 0  # one key of the second sample
    data = {"a": a, "s": s, "bias": bias, "mask": mask, "multiplicity": np.array(MULTIPLICITY)}
    a64, s64, bias64, mask64 = (x.astype(np.float64) for x in (a, s, bias, mask))
    for name, (ctor, seed) in DIFFUSION_MODULES.items():
        module = build(ctor, seed)
        print(f"{name}: fp64 loops", flush=True)
        if name == "adaln":
            out = B.adaln(module, a64, s64)
        elif name == "conditioned_transition":
            out = B.conditioned_transition(module, a64, s64)
        else:
            out = B.attention_pair_bias_keys(module, s64, s64, bias64, mask64, MULTIPLICITY)
        data[f"{name}/seed"] = np.array(seed)
        data[f"{name}/weight_stats"] = weight_stats(module)
        data[f"{name}/out"] = np.asarray(out, dtype=np.float32)
    np.savez_compressed(DIFFUSION_OUT, **data)
    print(f"wrote {DIFFUSION_OUT} ({DIFFUSION_OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
