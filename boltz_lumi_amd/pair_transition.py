"""Pair transition forward patched onto ``*.transition_z`` Boltz modules.

Reference: src/boltz_lumi/pair_transition.py (transition_forward :8-28).
LN, fc1 | fc2, SwiGLU and fc3 run as one fused gfx950 kernel with the 512-wide
hidden activation kept on chip.  Guard failures call the class forward.
"""

from __future__ import annotations

import torch

from . import ops
from ._guards import bf16_autocast, gfx950_tensor, inference


def transition_forward(module, x, chunk_size=None):
    """Drop-in for ``Transition.forward(x, chunk_size)`` of the 128 -> 512 -> 128 pair transition."""
    supported = (
        inference(module)
        and chunk_size is None
        and gfx950_tensor(x)
        and bf16_autocast()
        and x.dtype in (torch.float32, torch.bfloat16)
        and x.shape[-1] == 128
        and tuple(module.fc1.weight.shape) == (512, 128)
        and tuple(module.fc2.weight.shape) == (512, 128)
        and tuple(module.fc3.weight.shape) == (128, 512)
        and module.norm.weight is not None
        and module.norm.bias is not None
    )
    if not supported:
        return type(module).forward(module, x, chunk_size=chunk_size)
    return ops.pair_transition(module, x.contiguous(), ops.OUT_BF16)
