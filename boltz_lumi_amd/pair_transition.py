"""Pair transition forward patched onto ``*.transition_z`` Boltz modules.

Reference: src/boltz_lumi/pair_transition.py (transition_forward :8-28).
The 128 -> 512 -> 128 transition of the trunk, MSA and confidence pair stacks
runs as one fused gfx950 kernel (LN, fc1 | fc2, SwiGLU, fc3) with the 512-wide
hidden activation kept on chip.  Other widths (the template stack's
64 -> 256 -> 64) take the reference's composition: LN and the three
projections on hipBLASLt with the native bf16 SiLU-product kernel between
them.  Guard failures call the class forward.
"""

from __future__ import annotations

import torch

from . import ops
from ._guards import bf16_autocast, gfx950_tensor, inference


def _fused_shape(module, x) -> bool:
    return (
        x.dtype in (torch.float32, torch.bfloat16)
        and x.shape[-1] == 128
        and tuple(module.fc1.weight.shape) == (512, 128)
        and tuple(module.fc2.weight.shape) == (512, 128)
        and tuple(module.fc3.weight.shape) == (128, 512)
        and module.norm.weight is not None
        and module.norm.bias is not None
    )


def transition_forward(module, x, chunk_size=None):
    """Drop-in for ``Transition.forward(x, chunk_size)`` of a pair transition.

    Native in bf16-autocast inference without ``chunk_size`` (the reference's
    guard, pair_transition.py:9-19); returns bf16 like the upstream autocast
    path."""
    if not (inference(module) and chunk_size is None and gfx950_tensor(x) and bf16_autocast()):
        return type(module).forward(module, x, chunk_size=chunk_size)
    if _fused_shape(module, x):
        return ops.pair_transition(module, x.contiguous(), ops.OUT_BF16)
    normalized = module.norm(x)
    a = module.fc1(normalized)
    b = module.fc2(normalized)
    del normalized
    if a.dtype == b.dtype == torch.bfloat16 and a.is_contiguous() and b.is_contiguous():
        value = ops.silu_mul(a, b)
    else:
        value = module.silu(a) * b
    del a, b
    return module.fc3(value)
