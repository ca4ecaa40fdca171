"""Writes tests/golden/pair_modules_n6.npz: frozen input / output vectors of
the Pairformer pair modules and one whole PairformerLayer at their production
widths (128 pair channels, 384 single channels) and N = 6 tokens, the outputs
evaluated by the fp64 explicit-loop restatement (oracle/brute.py) on the
stored fp32 inputs.

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


if __name__ == "__main__":
    main()
