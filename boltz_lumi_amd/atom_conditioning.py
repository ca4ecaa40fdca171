"""Memoise the fixed atom-transformer conditioning projections within one
sampling call.

Reference: src/boltz_lumi/atom_conditioning.py:12-45.  Across the ~200
denoiser steps of one ``AtomDiffusion.sample`` call the atom encoder/decoder
see the same single conditioning ``s``, so ``s_norm``, ``s_scale``, ``s_bias``
of every AdaLN and the output-gate linears return the same tensors.  Inside
the context each of those submodules returns its first result for a given
(shape, stride, dtype, device) key.  The cache only engages for eval, no-grad,
autocast-off fp32 CUDA inputs; token conditioning (which changes with the
timestep) is not touched.  The fused AdaLN forward calls these submodules, so
it benefits from the cache.
"""

from __future__ import annotations

from contextlib import contextmanager

import torch


class _Cached:
    """Callable replacing ``module.forward`` while the context is active."""

    def __init__(self, module, original):
        self.module = module
        self.original = original
        self.memo = {}

    def __call__(self, x):
        m = self.module
        if (m.training or torch.is_grad_enabled() or torch.is_autocast_enabled("cuda") or not x.is_cuda
                or x.dtype != torch.float32):
            return self.original(x)
        key = (tuple(x.shape), tuple(x.stride()), x.dtype, x.device)
        hit = self.memo.get(key)
        if hit is None:
            hit = self.memo[key] = self.original(x)
        return hit


def conditioning_targets(score_model):
    """The conditioning submodules of the atom encoder and decoder layers."""
    encoder = score_model.atom_attention_encoder.atom_encoder.diffusion_transformer
    decoder = score_model.atom_attention_decoder.atom_decoder.diffusion_transformer
    found = []
    for layer in (*encoder.layers, *decoder.layers):
        for adaln in (layer.adaln, layer.transition.adaln):
            found += [adaln.s_norm, adaln.s_scale, adaln.s_bias]
        found += [layer.output_projection_linear, layer.transition.output_projection[0]]
    unique = []
    for mod in found:
        if all(mod is not u for u in unique):
            unique.append(mod)
    return unique


@contextmanager
def atom_conditioning_cache(score_model):
    patched = []
    missing = object()
    try:
        for module in conditioning_targets(score_model):
            own = vars(module).get("forward", missing)  # an instance-level forward, if any
            module.forward = _Cached(module, module.forward)
            patched.append((module, own))
        yield
    finally:
        for module, own in reversed(patched):
            if own is missing:
                del module.forward  # back to the class forward
            else:
                module.forward = own
