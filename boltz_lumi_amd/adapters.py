"""Install the gfx950 hot-path forwards on a Boltz-2 model.

Reference: src/boltz_lumi/adapters.py:7-47.  Same mechanism: walk
``model.named_modules()`` and rebind *instance* forwards with
``types.MethodType``, selected by class name and module path; idempotent via a
flag on the model; a no-op unless the model is a Boltz2 and the current device
is a gfx950 GPU of a ROCm build (the reference checks gfx90a).

Patched (class name, path rule -> replacement):
  TriangleAttention, TriangleAttentionEndingNode   -> triangle.triangle_attention_forward
      .layer_norm                                  -> triangle.normalization_forward
      ._chunk (ending node)                        -> triangle.contiguous_mask_chunk
  TriangleMultiplication{Outgoing,Incoming}        -> multiplication.normalized_forward
  Transition named "*.transition_z"                -> pair_transition.transition_forward
  PairformerLayer (trunk, confidence)              -> pairformer.pairformer_layer_forward (the
      five pair kernels adding into the fp32 stream in place, the dropout masks
      as row scales, the sequence stack fused with its pair bias written by the
      pair transition; beyond the reference, which leaves the layer upstream)
  PairformerNoSeqLayer (MSA, template)             -> pairformer.pairformer_noseq_forward
      (the template stack's 64-channel layers fall back to the class forward)
  AdaLN / ConditionedTransitionBlock under
      "structure_module.score_model."              -> diffusion.adaln_forward / transition_forward
  AttentionPairBias under
      "structure_module.score_model."              -> pair_bias.prepared_forward
      (the reference patches the token transformer's only, adapters.py:39-42;
      the atom transformer's windowed ones run on the same fused kernel here)
  DiffusionTransformerLayer under
      "structure_module.score_model."              -> diffusion.layer_forward (conditioning
      projections as two GEMMs, output gates and residual adds fused; beyond the
      reference, which leaves the layer upstream)
  DiffusionTransformer under
      "structure_module.score_model."              -> diffusion.stack_forward (operands of s
      built once per stack call; beyond the reference)
  AtomTransformer under
      "structure_module.score_model."              -> diffusion.atom_transformer_forward (key
      windows read by address instead of gathered; beyond the reference)
  structure_module.sample                          -> diffusion.optimized_sample
"""

from __future__ import annotations

from types import MethodType

from ._guards import gfx950_available

TRIANGLE_ATTENTION = {"TriangleAttention", "TriangleAttentionEndingNode"}
TRIANGLE_MULTIPLICATION = {"TriangleMultiplicationIncoming", "TriangleMultiplicationOutgoing"}
SCORE_MODEL = "structure_module.score_model."

FLAG = "_bmx_optimized"


def _is_boltz2(model) -> bool:
    return any(cls.__name__ == "Boltz2" for cls in type(model).__mro__)


def install(model, *, require_boltz2: bool = True, require_device: bool = True):
    """Patch the hot-path modules of ``model`` in place; returns the number of
    patched modules (0 when nothing applies).

    ``require_boltz2`` / ``require_device`` relax the model-class and
    gfx950-device gates (used by tests that install on stand-in modules)."""
    if require_boltz2 and not _is_boltz2(model):
        return 0
    if getattr(model, FLAG, False):
        return 0
    if require_device and not gfx950_available():
        return 0
    from . import _native

    _native.lib()  # fail loudly here, not inside the first forward
    from .diffusion import (adaln_forward, atom_transformer_forward, layer_forward, optimized_sample, stack_forward,
                            transition_forward)
    from .multiplication import normalized_forward
    from .pair_bias import prepared_forward
    from .pair_transition import transition_forward as pair_transition_forward
    from .pairformer import pairformer_layer_forward, pairformer_noseq_forward
    from .triangle import contiguous_mask_chunk, normalization_forward, triangle_attention_forward

    patched = 0
    for name, module in model.named_modules():
        cls = type(module).__name__
        if cls in TRIANGLE_ATTENTION:
            module.forward = MethodType(triangle_attention_forward, module)
            module.layer_norm.forward = MethodType(normalization_forward, module.layer_norm)
            if cls == "TriangleAttentionEndingNode" and hasattr(type(module), "_chunk"):
                module._chunk = MethodType(contiguous_mask_chunk, module)
            patched += 1
        elif cls in TRIANGLE_MULTIPLICATION:
            module.forward = MethodType(normalized_forward, module)
            patched += 1
        elif cls == "Transition" and name.endswith(".transition_z"):
            module.forward = MethodType(pair_transition_forward, module)
            patched += 1
        elif cls == "PairformerLayer":
            module.forward = MethodType(pairformer_layer_forward, module)
            patched += 1
        elif cls == "PairformerNoSeqLayer":
            module.forward = MethodType(pairformer_noseq_forward, module)
            patched += 1
        elif name.startswith(SCORE_MODEL) and cls == "AdaLN":
            module.forward = MethodType(adaln_forward, module)
            patched += 1
        elif name.startswith(SCORE_MODEL) and cls == "ConditionedTransitionBlock":
            module.forward = MethodType(transition_forward, module)
            patched += 1
        elif name.startswith(SCORE_MODEL) and cls == "AttentionPairBias":
            module.forward = MethodType(prepared_forward, module)
            patched += 1
        elif name.startswith(SCORE_MODEL) and cls == "DiffusionTransformerLayer":
            module.forward = MethodType(layer_forward, module)
            patched += 1
        elif name.startswith(SCORE_MODEL) and cls == "DiffusionTransformer":
            module.forward = MethodType(stack_forward, module)
            patched += 1
        elif name.startswith(SCORE_MODEL) and cls == "AtomTransformer":
            module.forward = MethodType(atom_transformer_forward, module)
            patched += 1
    structure = getattr(model, "structure_module", None)
    if structure is not None and hasattr(type(structure), "sample"):
        structure.sample = MethodType(optimized_sample, structure)
        patched += 1
    setattr(model, FLAG, True)
    return patched


def uninstall(model) -> int:
    """Remove the instance-level patches installed by :func:`install`."""
    removed = 0
    for _, module in model.named_modules():
        for owner, attr in ((module, "forward"), (module, "_chunk"), (module, "sample"),
                            (getattr(module, "layer_norm", None), "forward")):
            if owner is not None and attr in vars(owner) and isinstance(vars(owner)[attr], MethodType):
                if vars(owner)[attr].__func__.__module__.startswith(__package__):
                    del owner.__dict__[attr]
                    removed += 1
    if getattr(model, FLAG, False):
        delattr(model, FLAG)
    return removed
