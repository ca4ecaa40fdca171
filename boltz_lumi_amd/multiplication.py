"""Triangle multiplication forward patched onto Boltz modules.

Reference: src/boltz_lumi/multiplication.py (normalized_forward :48-137).
The LN_in / p_in, g_in / gate+mask / per-channel product / LN_out / p_out,
g_out / gate chain runs as the three fused gfx950 kernels of libbmx
(projection into the per-channel operand planes, the batched MFMA product,
LN_out + output projection + gate).  Guard failures call the module's own
class forward unchanged.
"""

from __future__ import annotations

import torch

from . import ops
from ._guards import bf16_autocast, fp32_contiguous_on, gfx950_tensor, inference


def normalized_forward(module, x, mask, use_kernels=False):
    """Drop-in for ``TriangleMultiplication{Outgoing,Incoming}.forward(x, mask, use_kernels)``."""
    supported = (
        not use_kernels
        and inference(module)
        and gfx950_tensor(x)
        and x.ndim == 4
        and x.shape[1] == x.shape[2]
        and x.shape[-1] == 128
        and x.shape[1] <= 16384
        and x.dtype == torch.float32
        and x.is_contiguous()
        and bf16_autocast()
        and mask.dtype == torch.float32
        and mask.is_contiguous()
        and mask.device == x.device
        and tuple(mask.shape) == tuple(x.shape[:-1])
        and fp32_contiguous_on(x.device, module.norm_in.weight, module.norm_in.bias, module.norm_out.weight,
                               module.norm_out.bias)
    )
    if not supported:
        return type(module).forward(module, x, mask, use_kernels=use_kernels)
    outgoing = type(module).__name__ == "TriangleMultiplicationOutgoing"
    out = torch.empty(x.shape, device=x.device, dtype=torch.bfloat16)
    ws = ops.new_workspace(x.shape[1], x.device)
    for b in range(x.shape[0]):
        ops.trimul(module, x[b], mask[b], outgoing, ops.OUT_BF16, out[b], ws)
    return out
