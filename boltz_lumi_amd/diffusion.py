"""Diffusion AdaLN / conditioned-transition forwards patched onto the score model.

Reference: src/boltz_lumi/diffusion.py (adaln_forward :52-57,
transition_forward :60-68, eligibility :37-49).  As in the reference these
run in fp32 with autocast off.  AdaLN's a_norm + sigmoid(s_scale) modulation
+ s_bias become one LN/modulate kernel; the SwiGLU gate and the output gate
are fused epilogues.  The conditioning projections are still called as
submodules, so ``atom_conditioning_cache`` keeps working (reference
atom_conditioning.py:12-45).  Guard failures call the class forward.
"""

from __future__ import annotations

import torch

from . import ops
from ._guards import autocast_off, gfx950_tensor, inference


def eligible(module, *tensors) -> bool:
    return inference(module) and autocast_off() and all(
        gfx950_tensor(t) and t.dtype == torch.float32 and t.is_contiguous() for t in tensors)


def adaln_forward(self, a, s):
    """Drop-in for ``AdaLN.forward(a, s)``."""
    if not eligible(self, a, s) or a.shape[-1] % 4 or a.shape[-1] > 1024:
        return type(self).forward(self, a, s)
    sn = self.s_norm(s)
    return ops.adaln_modulate(a, self.s_scale(sn).contiguous(), self.s_bias(sn).contiguous(), self.a_norm.eps)


def transition_forward(self, a, s):
    """Drop-in for ``ConditionedTransitionBlock.forward(a, s)``."""
    if not eligible(self, a, s):
        return type(self).forward(self, a, s)
    a = self.adaln(a, s)
    b = ops.epilogue(self.swish_gate[0](a).contiguous(), self.a_to_b(a).contiguous(), None, ops.GATED_SWIGLU)
    return ops.epilogue(self.output_projection[0](s).contiguous(), self.b_to_a(b).contiguous(), None, ops.GATE)
