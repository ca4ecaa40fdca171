"""PairformerLayer / PairformerNoSeqLayer forwards patched onto Boltz modules.

Upstream Boltz 2.2.1 (``boltz.model.layers.pairformer``) composes a layer as
    z = z + d1 * tri_mul_out(z);  z = z + d2 * tri_mul_in(z)
    z = z + d3 * tri_att_start(z);  z = z + d4 * tri_att_end(z)
    z = z + transition_z(z)
then, with autocast off, the fp32 sequence stack
    s = s + attention(pre_norm_s(s), z);  s = s + transition_s(s);  s = s_post_norm(s)
where ``d1..d4`` are ``get_dropout_mask`` draws ([B, N, 1, 1], column-wise
[B, 1, N, 1] for ``d4``): ``torch.rand_like(...) > dropout * training``, so in
eval they are ones, except where a draw is exactly 0, and each draw advances
the generator.  The reference keeps that composition and patches only the
modules inside it (src/boltz_lumi/adapters.py:24-46): every branch then makes a
bf16 module output, an fp32 product with its mask and an fp32 sum in HBM, and
the sequence stack runs upstream's fp32 AttentionPairBias, whose pair bias is a
LayerNorm + Linear(128 -> 16) over all N^2 pairs.

Here the layer itself is replaced (beyond the reference, like the diffusion
layers of ``diffusion.py``):
  * the five fused pair kernels add their bf16-rounded outputs into the fp32
    stream in place; the first writes a new tensor (``z`` + branch), so the
    caller's z is never modified;
  * the dropout masks are drawn exactly as upstream draws them (same shapes,
    order and generator) and applied as row scales inside the output kernels
    (``row_scale``; the ending node's column-wise mask is its frame's row);
  * the pair transition's epilogue also writes the sequence stack's pair bias
    from the updated rows, so z is not read again for it;
  * the sequence attention runs fused (``pair_bias.fused_attention``), with
    the residual adds in the epilogues of the fp32 output GEMMs.
A guard that fails runs the class forward unchanged (whose submodules may
still be the patched module forwards); the sequence stack alone falls back to
upstream's composition when only its modules do not qualify.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import ops
from ._guards import bf16_autocast, fp32_contiguous_on, gfx950_tensor, inference

MAX_N = 8192  # the fused triangle attention's limit


def _plain(module) -> bool:
    return not (module._forward_hooks or module._forward_pre_hooks)


def _forward_is(module, *funcs) -> bool:
    """``module`` runs its class forward or one of ``funcs`` (this package's
    patch of it), and has no hooks: a fused path may then skip its call."""
    fwd = vars(module).get("forward")
    return _plain(module) and (fwd is None or getattr(fwd, "__func__", None) in funcs)


def _no_bias(*linears) -> bool:
    return all(getattr(lin, "bias", None) is None for lin in linears)


def _shape(t, *shape) -> bool:
    return t is not None and tuple(t.shape) == shape


def _trimul_ok(module, outgoing, device) -> bool:
    from .multiplication import normalized_forward

    name = "TriangleMultiplicationOutgoing" if outgoing else "TriangleMultiplicationIncoming"
    return (type(module).__name__ == name and _forward_is(module, normalized_forward)
            and _shape(module.p_in.weight, 256, 128) and _shape(module.g_in.weight, 256, 128)
            and _shape(module.p_out.weight, 128, 128) and _shape(module.g_out.weight, 128, 128)
            and _no_bias(module.p_in, module.g_in, module.p_out, module.g_out)
            and fp32_contiguous_on(device, module.norm_in.weight, module.norm_in.bias, module.norm_out.weight,
                                   module.norm_out.bias))


def _triattn_ok(module, starting, device) -> bool:
    from .triangle import normalization_forward, triangle_attention_forward

    name = "TriangleAttention" if starting else "TriangleAttentionEndingNode"
    mha = getattr(module, "mha", None)
    ln = getattr(module, "layer_norm", None)
    return (type(module).__name__ == name and bool(getattr(module, "starting", True)) == starting
            and _forward_is(module, triangle_attention_forward) and ln is not None and mha is not None
            and _forward_is(ln, normalization_forward) and _plain(mha)
            and (getattr(module, "c_in", None), getattr(module, "c_hidden", None),
                 getattr(module, "no_heads", None)) == (128, 32, 4)
            and ln.weight is not None and ln.bias is not None
            and fp32_contiguous_on(device, ln.weight, ln.bias)
            and _shape(module.linear.weight, 4, 128) and _no_bias(module.linear, mha.linear_q, mha.linear_k,
                                                                   mha.linear_v)
            and mha.linear_g.bias is not None and mha.linear_o.bias is not None)


def _transition_z_ok(module) -> bool:
    from .pair_transition import transition_forward

    return (type(module).__name__ == "Transition" and _forward_is(module, transition_forward)
            and _shape(module.fc1.weight, 512, 128) and _shape(module.fc2.weight, 512, 128)
            and _shape(module.fc3.weight, 128, 512) and _no_bias(module.fc1, module.fc2, module.fc3)
            and module.norm.weight is not None and module.norm.bias is not None)


def pair_stack_ok(layer, z, pair_mask) -> bool:
    """The fused pair stack applies to ``layer`` (an upstream-structured
    Pairformer layer) on ``z``: bf16-autocast inference on a gfx950 tensor,
    fp32 contiguous z [B, N, N, 128] with N <= 8192, a [B, N, N] pair mask,
    and five unhooked pair modules of the expected classes and shapes."""
    return (inference(layer) and bf16_autocast() and gfx950_tensor(z) and z.dtype == torch.float32
            and z.is_contiguous() and z.dim() == 4 and z.shape[1] == z.shape[2] and z.shape[-1] == 128
            and 0 < z.shape[1] <= MAX_N and z.shape[0] > 0
            and pair_mask is not None and tuple(pair_mask.shape) == tuple(z.shape[:3]) and pair_mask.is_floating_point()
            and pair_mask.device == z.device
            and _trimul_ok(layer.tri_mul_out, True, z.device) and _trimul_ok(layer.tri_mul_in, False, z.device)
            and _triattn_ok(layer.tri_att_start, True, z.device) and _triattn_ok(layer.tri_att_end, False, z.device)
            and _transition_z_ok(layer.transition_z))


def dropout_mask(layer, z, columnwise=False):
    """Upstream ``get_dropout_mask(layer.dropout, z, layer.training, columnwise)``
    (boltz.model.layers.dropout): a draw per row ([B, N, 1, 1]) or per column
    ([B, 1, N, 1]) of z, kept where it exceeds the dropout rate times
    ``training`` and scaled by 1 / (1 - rate).  In eval the rate is 0: the mask
    is 1 except where a draw is exactly 0, and the draw advances the
    generator as upstream's does."""
    p = float(getattr(layer, "dropout", 0.0)) * layer.training
    v = z[:, 0:1, :, 0:1] if columnwise else z[:, :, 0:1, 0:1]
    d = torch.rand_like(v)
    if p == 0.0:
        # (d > 0) * 1.0 / 1.0 as one in-place comparison: the same 0 / 1
        # values in one kernel instead of three (the fused path runs in eval,
        # where the rate is always 0)
        return d.gt_(0.0)
    return (d > p) * 1.0 / (1.0 - p)


def _row_scales(mask):
    """Per batch element, the [N] fp32 row scale of a dropout mask."""
    flat = mask.reshape(mask.shape[0], -1)
    return [flat[b].contiguous() for b in range(flat.shape[0])]


def pair_stack(layer, z, pair_mask, z_out=None, workspace=None, bias_out=None, bias_mods=None, keep=None):
    """z_out = z + d1 tri_mul_out + d2 tri_mul_in + d3 tri_att_start + d4 tri_att_end
    + transition_z, each branch added in order into the fp32 stream by its
    fused kernel.  z is read and never written; ``z_out`` may be preallocated.
    ``keep``: the four dropout masks (None: no masks).  With ``bias_out``
    [B, 16, N, N] and ``bias_mods`` (proj_z's LayerNorm and Linear) the
    transition's epilogue also writes the sequence stack's pair bias of
    z_out."""
    if not z.is_cuda:
        raise RuntimeError("the fused pair stack needs a GPU tensor (got %s)" % z.device)
    if z.dtype != torch.float32:
        raise RuntimeError("the pair stream is fp32")
    z = z.contiguous()
    z_out = torch.empty_like(z) if z_out is None else z_out
    n = z.shape[1]
    ws = ops.new_workspace(n, z.device) if workspace is None else workspace
    scales = [None] * 4 if keep is None else [_row_scales(k) for k in keep]
    for b in range(z.shape[0]):
        zi, zo = z[b], z_out[b]
        mb = pair_mask[b].to(torch.float32).contiguous()
        rs = [None if s is None else s[b] for s in scales]
        ops.trimul(layer.tri_mul_out, zi, mb, True, ops.OUT_RESIDUAL, zo, ws, row_scale=rs[0])
        ops.trimul(layer.tri_mul_in, zo, mb, False, ops.OUT_ACCUMULATE, zo, ws, row_scale=rs[1])
        ops.triattn(layer.tri_att_start, zo, mb, True, ops.OUT_ACCUMULATE, zo, ws, row_scale=rs[2])
        ops.triattn(layer.tri_att_end, zo, mb, False, ops.OUT_ACCUMULATE, zo, ws, row_scale=rs[3])
        pb = None if bias_out is None else (bias_mods[0], bias_mods[1], bias_out[b])
        ops.pair_transition(layer.transition_z, zo, ops.OUT_ACCUMULATE, zo, pair_bias=pb)
    return z_out


def transition_residual(module, x, inplace=False):
    """``x + module(x)`` for an upstream Transition in fp32 (the sequence
    stack's 384 -> 1536 -> 384): fc1 | fc2 as one GEMM and the residual add in
    the fc3 GEMM's epilogue, written into x when ``inplace`` and x is
    contiguous.  Other cases run ``x + module(x)``."""
    hidden = module.fc1.weight.shape[0]
    if (x.dtype != torch.float32 or module.fc3.weight.dtype != x.dtype or torch.is_grad_enabled()
            or not _plain(module) or "forward" in vars(module) or not _no_bias(module.fc1, module.fc2, module.fc3)
            or not all(_plain(m) for m in (module.norm, module.fc1, module.fc2, module.fc3))
            or tuple(module.fc2.weight.shape) != tuple(module.fc1.weight.shape)
            or module.fc3.weight.shape[1] != hidden or module.fc3.weight.shape[0] != x.shape[-1]
            or type(getattr(module, "silu", torch.nn.SiLU())) is not torch.nn.SiLU):
        return x + module(x)
    w12 = ops.cached_weight(module, "w12", (module.fc1.weight, module.fc2.weight), lambda a, b: torch.cat([a, b], 0))
    h = F.linear(module.norm(x), w12)
    h = F.silu(h[..., :hidden]).mul_(h[..., hidden:])
    x2 = x.reshape(-1, x.shape[-1])
    if inplace and x.is_contiguous():
        x2.addmm_(h.reshape(-1, hidden), module.fc3.weight.t())
        return x
    return torch.addmm(x2, h.reshape(-1, hidden), module.fc3.weight.t()).view(x.shape)


def pair_bias_mods(attention):
    """(LayerNorm, Linear) of an upstream v2 AttentionPairBias whose pair bias
    ``proj_z(z)`` the pair transition's epilogue can write (LayerNorm(128) with
    affine, Linear(128 -> 16) without bias, both unhooked), else None."""
    if not getattr(attention, "compute_pair_bias", False):
        return None
    proj = getattr(attention, "proj_z", None)
    if not isinstance(proj, torch.nn.Sequential) or len(proj) < 2 or not _plain(proj):
        return None
    norm, lin = proj[0], proj[1]
    if not (isinstance(norm, torch.nn.LayerNorm) and isinstance(lin, torch.nn.Linear) and _plain(norm) and _plain(lin)
            and "forward" not in vars(norm) and "forward" not in vars(lin)
            and tuple(norm.normalized_shape) == (128,) and norm.weight is not None and norm.bias is not None
            and _shape(lin.weight, 16, 128) and lin.bias is None):
        return None
    # the remaining stages must be the parameter-free heads-first rearrangement
    rest = list(proj)[2:]
    if len(rest) != 1 or any(True for _ in rest[0].parameters()) or not _plain(rest[0]):
        return None
    return norm, lin


def sequence_ok(layer, s, z, mask) -> bool:
    """The fused sequence stack applies: an unhooked upstream v2
    AttentionPairBias of 16 heads x 24 over a 384-channel s of N tokens with an
    [B, N] mask, its proj_o without bias, a plain pre_norm_s."""
    att = getattr(layer, "attention", None)
    return (att is not None and type(att).__name__ == "AttentionPairBias" and _plain(att) and "forward" not in vars(att)
            and getattr(att, "num_heads", None) == 16 and getattr(att, "c_s", None) == 384
            and all(_plain(m) and "forward" not in vars(m)
                    for m in (att.proj_q, att.proj_k, att.proj_v, att.proj_g, att.proj_o))
            and att.proj_o.bias is None and _plain(layer.pre_norm_s) and "forward" not in vars(layer.pre_norm_s)
            and s is not None and s.dim() == 3 and s.shape[0] == z.shape[0] and s.shape[1] == z.shape[1]
            and s.shape[2] == 384 and s.device == z.device
            and mask is not None and tuple(mask.shape) == tuple(s.shape[:2]) and mask.device == z.device)


def sequence_stack(layer, s, z, mask, pair_bias=None):
    """Upstream's sequence stack in fp32 with autocast off:
    ``s + attention(pre_norm_s(s), z)``, then ``+ transition_s``, then
    ``s_post_norm``; on the fused path (``sequence_ok``) the attention is one
    kernel over the pair bias ``pair_bias`` (``attention.proj_z(z)``, computed
    here when None) and each residual add rides in the epilogue of its output
    GEMM."""
    with torch.autocast("cuda", enabled=False):
        s = s.float()
        s_normed = layer.pre_norm_s(s)
        o = None
        if sequence_ok(layer, s, z, mask):
            if pair_bias is None and pair_bias_mods(layer.attention) is not None:
                norm, lin = pair_bias_mods(layer.attention)
                pair_bias = torch.empty((z.shape[0], 16, z.shape[1], z.shape[2]), device=z.device,
                                        dtype=torch.float32)
                for b in range(z.shape[0]):
                    ops.pair_bias(norm, lin, z[b].contiguous(), out=pair_bias[b])
            from .pair_bias import fused_attention

            o = fused_attention(layer.attention, s_normed, z.float(), mask.float(), s_normed, bias=pair_bias)
        if o is None:
            s = s + layer.attention(s=s_normed, z=z.float(), mask=mask.float(), k_in=s_normed)
            s = s + layer.transition_s(s)
        else:
            s = torch.addmm(s.reshape(-1, s.shape[-1]), o.reshape(-1, o.shape[-1]),
                            layer.attention.proj_o.weight.float().t()).view(s.shape)
            s = transition_residual(layer.transition_s, s, inplace=True)
        return layer.s_post_norm(s)


def _kernels_requested(use_kernels, extra) -> bool:
    return bool(use_kernels) or any(bool(v) for v in extra)


def pairformer_layer_forward(self, s, z, mask, pair_mask, chunk_size_tri_attn=None, use_kernels=False, *args,
                             **kwargs):
    """Drop-in for upstream ``PairformerLayer.forward(s, z, mask, pair_mask,
    chunk_size_tri_attn, use_kernels, use_cuequiv_mul, use_cuequiv_attn)``.
    ``chunk_size_tri_attn`` changes nothing on the fused path (the attention
    never materialises its scores)."""
    extra = tuple(args) + tuple(kwargs.values())
    if _kernels_requested(use_kernels, extra) or not pair_stack_ok(self, z, pair_mask):
        return type(self).forward(self, s, z, mask, pair_mask, chunk_size_tri_attn, use_kernels, *args, **kwargs)
    keep = [dropout_mask(self, z), dropout_mask(self, z), dropout_mask(self, z), dropout_mask(self, z, True)]
    mods = pair_bias_mods(self.attention) if sequence_ok(self, s, z, mask) else None
    bias = None
    if mods is not None:
        bias = torch.empty((z.shape[0], 16, z.shape[1], z.shape[2]), device=z.device, dtype=torch.float32)
    z = pair_stack(self, z, pair_mask, bias_out=bias, bias_mods=mods, keep=keep)
    return sequence_stack(self, s, z, mask, pair_bias=bias), z


def pairformer_noseq_forward(self, z, pair_mask, chunk_size_tri_attn=None, use_kernels=False, *args, **kwargs):
    """Drop-in for upstream ``PairformerNoSeqLayer.forward(z, pair_mask,
    chunk_size_tri_attn, use_kernels, use_cuequiv_mul, use_cuequiv_attn)``
    (the MSA module's pair stack; the template stack's 64-channel layers fail
    the guard and run the class forward)."""
    extra = tuple(args) + tuple(kwargs.values())
    if _kernels_requested(use_kernels, extra) or not pair_stack_ok(self, z, pair_mask):
        return type(self).forward(self, z, pair_mask, chunk_size_tri_attn, use_kernels, *args, **kwargs)
    keep = [dropout_mask(self, z), dropout_mask(self, z), dropout_mask(self, z), dropout_mask(self, z, True)]
    return pair_stack(self, z, pair_mask, keep=keep)
