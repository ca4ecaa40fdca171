"""Diffusion forwards patched onto the score model (AdaLN, conditioned
transition, transformer layer, transformer stack, atom transformer) and the
``structure_module.sample`` wrapper.

Reference: src/boltz_lumi/diffusion.py (optimized_sample :13-23, adaln_forward
:52-57, transition_forward :60-68, eligibility :37-49).  As in the reference the
forwards run in fp32 with autocast off.  AdaLN's a_norm + sigmoid(s_scale)
modulation + s_bias is one LN/modulate kernel; the SwiGLU gate and the output
gates are fused epilogues.  Beyond the reference, a DiffusionTransformer builds
the operands of its conditioning s once per call and each layer runs its six
conditioning projections as two GEMMs (LayerNorm(s) with the s_norm affines
folded into the weights, and s), and an AtomTransformer reads its key windows
by address instead of gathering them.  Memoised (``atom_conditioning_cache``,
reference atom_conditioning.py:12-45) or hooked projections are called as
submodules.  The linears, fp32 hipBLASLt GEMMs in the reference, run as
split-bf16 GEMMs with fp32 accumulation from 512 input channels up (about 2^-16
relative per product).  Guard failures call the class forward.
"""

from __future__ import annotations

import weakref
from contextlib import nullcontext

import torch

from . import ops
from ._guards import autocast_off, gfx950_tensor, inference
from .atom_conditioning import atom_conditioning_cache
from .pair_bias import (attention_from_operand, operand_ok, prepare_token_bias, prepare_window_bias,
                        window_bias_prepared, windowed_attention, windowed_ok)


def optimized_sample(self, *args, **kwargs):
    """Drop-in for ``AtomDiffusion.sample`` (reference diffusion.py:13-23): in
    inference the token transformer's fixed bias is packed head-major once
    (``prepare_token_bias``, so each layer's attention reads a dense slice),
    the atom encoder's and decoder's window biases channel-major
    (``prepare_window_bias``; beyond the reference), and with one sample of one
    structure the atom conditioning projections are memoised for the call
    (``atom_conditioning_cache``)."""
    sample = type(self).sample
    if torch.is_grad_enabled() or self.training or "diffusion_conditioning" not in kwargs:
        return sample(self, *args, **kwargs)
    conditioning = dict(kwargs["diffusion_conditioning"])
    conditioning["token_trans_bias"] = prepare_token_bias(conditioning["token_trans_bias"])
    for name in ("atom_enc_bias", "atom_dec_bias"):
        value = conditioning.get(name)
        if isinstance(value, torch.Tensor) and value.dim() == 5 and value.is_cuda:
            conditioning[name] = prepare_window_bias(value)
    kwargs["diffusion_conditioning"] = conditioning
    single = kwargs.get("multiplicity", 1) == 1 and conditioning["c"].shape[0] == 1
    with atom_conditioning_cache(self.score_model) if single else nullcontext():
        return sample(self, *args, **kwargs)


def eligible(module, *tensors) -> bool:
    return inference(module) and autocast_off() and all(
        gfx950_tensor(t) and t.dtype == torch.float32 and t.is_contiguous() for t in tensors)


def _linear(linear, x):
    """``linear(x)`` for fp32 x: ``ops.linear_fp32`` (the split-bf16 GEMM with
    fp32 accumulation from 512 input channels up), or the submodule call when
    it has an instance-level forward, such as the memo of
    ``atom_conditioning_cache``."""
    if "forward" in vars(linear):
        return linear(x).contiguous()
    return ops.linear_fp32(x, linear).contiguous()


def adaln_forward(self, a, s):
    """Drop-in for ``AdaLN.forward(a, s)``."""
    if not eligible(self, a, s) or a.shape[-1] % 4 or a.shape[-1] > 1024:
        return type(self).forward(self, a, s)
    sn = self.s_norm(s)
    return ops.adaln_modulate(a, _linear(self.s_scale, sn), _linear(self.s_bias, sn), self.a_norm.eps)


def _transition_ok(block, a, s) -> bool:
    return eligible(block, a, s) and a.shape[-1] % 4 == 0 and block.a_to_b.weight.shape[0] % 4 == 0


def _transition_inner(block, a, s):
    """b_to_a(b) and the output-gate logits of a ConditionedTransitionBlock."""
    x = block.adaln(a, s)
    b = ops.epilogue(_linear(block.swish_gate[0], x), _linear(block.a_to_b, x), None, ops.GATED_SWIGLU)
    return _linear(block.b_to_a, b), _linear(block.output_projection[0], s)


def transition_forward(self, a, s):
    """Drop-in for ``ConditionedTransitionBlock.forward(a, s)``.  The fused
    epilogues take widths that are multiples of 4 (every Boltz-2 width is);
    other widths run the class forward."""
    if not _transition_ok(self, a, s):
        return type(self).forward(self, a, s)
    y, gate = _transition_inner(self, a, s)
    return ops.epilogue(gate, y, None, ops.GATE)


def _plain(module) -> bool:
    """No forward hooks on ``module``, so a fused path may skip its call."""
    return not (module._forward_hooks or module._forward_pre_hooks)


def _untouched(module) -> bool:
    """No hooks and no instance-level forward (such as the memo of
    ``atom_conditioning_cache``), so its math may be folded elsewhere."""
    return _plain(module) and "forward" not in vars(module)


def _patched_with(module, func) -> bool:
    return getattr(vars(module).get("forward"), "__func__", None) is func


def _adaln_foldable(adaln, c) -> bool:
    """AdaLN whose s-side (s_norm, s_scale, s_bias) may run as one projection
    of LayerNorm-without-affine(s) with the s_norm affine folded into the
    weights: an a_norm without affine, an s_norm over the c channels, nothing
    hooked or memoised."""
    fwd = vars(adaln).get("forward")
    an, sn = adaln.a_norm, adaln.s_norm
    return (_plain(adaln) and (fwd is None or getattr(fwd, "__func__", None) is adaln_forward)
            and isinstance(an, torch.nn.LayerNorm) and an.weight is None and an.bias is None
            and isinstance(sn, torch.nn.LayerNorm) and tuple(sn.normalized_shape) == (c,)
            and all(_untouched(m) for m in (sn, adaln.s_scale, adaln.s_bias)))


def _side_ok(layer, a, s) -> bool:
    """The whole layer may run with its conditioning projections as two GEMMs
    on operands of s shared by the stack (``_Side``)."""
    c = s.shape[-1]
    tr = layer.transition
    return (a.shape[-1] <= 1024 and _adaln_foldable(layer.adaln, c) and _adaln_foldable(tr.adaln, c)
            and _untouched(layer.output_projection_linear) and _plain(layer.output_projection)
            and _patched_with(tr, transition_forward) and _plain(tr) and _plain(tr.output_projection)
            and _untouched(tr.output_projection[0]) and _transition_ok(tr, a, s))


class _Side:
    """Operands of the conditioning projections built from ``s`` once per
    stack call: LayerNorm-without-affine(s) (every AdaLN's s_norm, whose
    affine is folded into the projection weights; one per eps) and s itself.
    Split-bf16 operands where the linears run split (``ops.use_split``), else
    fp32 rows."""

    def __init__(self, s):
        self.s = s.reshape(-1, s.shape[-1])
        self.split = ops.use_split(s.shape[-1], s.numel() // max(s.shape[-1], 1))
        self._norm = {}
        self._raw = None

    def norm(self, eps):
        if eps not in self._norm:
            self._norm[eps] = (ops.layernorm_split3(self.s, eps) if self.split
                               else ops.layer_norm(self.s, None, None, eps))
        return self._norm[eps]

    def raw(self):
        if self._raw is None:
            self._raw = ops.split3(self.s) if self.split else self.s
        return self._raw


def _folded(adaln):
    """[s_scale; s_bias] (weight [2 d, c], bias [2 d]) acting on
    LayerNorm-without-affine(s): s_scale(LN(s) w + b) = LN(s) (W diag(w)) + W b + bias."""
    lins = (adaln.s_scale, adaln.s_bias)
    w = torch.cat([lin.weight.detach().float() for lin in lins])
    b = torch.cat([lin.bias.detach().float() if lin.bias is not None
                   else w.new_zeros(lin.out_features) for lin in lins])
    sn = adaln.s_norm
    if sn.bias is not None:
        b = b + w @ sn.bias.detach().float()
    if sn.weight is not None:
        w = w * sn.weight.detach().float()
    return w, b


def _mods_sources(layer):
    out = []
    for adaln in (layer.adaln, layer.transition.adaln):
        for m in (adaln.s_norm, adaln.s_scale, adaln.s_bias):
            out += [p for p in (m.weight, m.bias) if p is not None]
    return tuple(out)


def _gate_linears(layer):
    return (layer.output_projection_linear, layer.transition.output_projection[0])


def _conditioning(layer, side, eps):
    """(mods [M, 4 d], gates [M, 2 d]) of one layer: the attention AdaLN's
    scale | shift and the transition AdaLN's scale | shift from LN(s), and the
    two output-gate logits from s, as two GEMMs (split-bf16 or fp32, the
    biases and s_norm affines folded in)."""
    gl = _gate_linears(layer)
    gw = tuple(lin.weight for lin in gl)
    gb = tuple(lin.bias for lin in gl)
    if side.split:
        wm = ops.cached_weight(layer, "cond_mods_x3", _mods_sources(layer), lambda *_: ops._x3_weight(
            *(torch.cat(t) for t in zip(_folded(layer.adaln), _folded(layer.transition.adaln)))))
        mods = ops.mm_split(side.norm(eps), wm)
        gates = ops.mm_split(side.raw(), ops.x3_weight(layer, "cond_gates_x3", gw, gb))
        return mods, gates
    wm = ops.cached_weight(layer, "cond_mods_w", _mods_sources(layer), lambda *_: torch.cat(
        [_folded(layer.adaln)[0], _folded(layer.transition.adaln)[0]]))
    bm = ops.cached_weight(layer, "cond_mods_b", _mods_sources(layer), lambda *_: torch.cat(
        [_folded(layer.adaln)[1], _folded(layer.transition.adaln)[1]]))
    wg = ops.cached_weight(layer, "cond_gates_w", gw, lambda *ws: torch.cat(ws).float())
    bg = ops.cached_weight(layer, "cond_gates_b", tuple(b for b in gb if b is not None), lambda *_: torch.cat(
        [lin.bias.detach().float() if lin.bias is not None else lin.weight.new_zeros(lin.out_features,
                                                                                        dtype=torch.float32)
         for lin in gl]))
    return (torch.nn.functional.linear(side.norm(eps), wm, bm),
            torch.nn.functional.linear(side.raw(), wg, bg))


def _operand_path(layer, side, to_keys, keys=None) -> bool:
    """Whether ``_layer_with_side`` feeds the attention from the AdaLN output's
    split operand (``adaln_split3``), the token transformer's path."""
    return keys is None and to_keys is None and side.split and operand_ok(layer.pair_bias_attn)


def _layer_with_side(self, a, s, side, bias, mask, to_keys, multiplicity, keys=None, carry=None, nxt=None):
    """The layer with its conditioning projections on the shared operands of s
    (``side``); with ``keys`` (a ``_WindowKeys``) the attention reads its key
    windows by address (``windowed_attention``) instead of ``to_keys``.

    ``carry`` = (attention operand, mods, gates) of this layer, computed by the
    previous layer's last pass; with ``nxt`` (the next layer, whose attention
    also starts from the AdaLN's split operand: the token path, or windows
    with split linears) this layer's last residual update also writes the next
    layer's attention operand (``gated_residual_adaln_split3``), and the
    result is (a, carry for ``nxt``) instead of a."""
    d = a.shape[-1]
    tr = self.transition
    eps = self.adaln.s_norm.eps
    mods, gates = _conditioning(self, side, eps) if carry is None else carry[1:]
    scale_a, shift_a, scale_t, shift_t = mods.split(d, dim=-1)
    gate_a, gate_t = gates.split(d, dim=-1)
    rows = a.reshape(-1, d)
    att = self.pair_bias_attn
    o = None
    if keys is None and to_keys is None and side.split and operand_ok(att):
        # the AdaLN output only as the q | k | v | g GEMM's split operand, and the
        # attention's output only as proj_o's, where proj_o is the plain linear
        plain_o = _untouched(att.proj_o)
        op = ops.adaln_split3(rows, scale_a, shift_a, self.adaln.a_norm.eps) if carry is None else carry[0]
        o = attention_from_operand(att, op, a.shape, bias, mask, multiplicity, split_out=plain_o)
    if o is not None and o.dtype == torch.bfloat16:
        pl = att.proj_o
        b = ops.mm_split(o, ops.x3_weight(pl, "x3", (pl.weight,), (pl.bias,))).view(a.shape)
    elif o is not None:
        b = att.proj_o(o) if "forward" in vars(att.proj_o) else ops.linear_fp32(o, att.proj_o)
    elif keys is not None and side.split:  # the AdaLN output only as the projection's split operand
        op = ops.adaln_split3(rows, scale_a, shift_a, self.adaln.a_norm.eps) if carry is None else carry[0]
        o = windowed_attention(att, None, bias, keys, op=op, shape=a.shape)
        b = att.proj_o(o) if "forward" in vars(att.proj_o) else ops.linear_fp32(o, att.proj_o)
    elif keys is not None:
        b = ops.adaln_modulate(rows, scale_a, shift_a, self.adaln.a_norm.eps).view(a.shape)
        o = windowed_attention(att, b, bias, keys)
        b = att.proj_o(o) if "forward" in vars(att.proj_o) else ops.linear_fp32(o, att.proj_o)
    else:
        b = ops.adaln_modulate(rows, scale_a, shift_a, self.adaln.a_norm.eps).view(a.shape)
        k_in = b
        if to_keys is not None:
            k_in = to_keys(b)
            mask = to_keys(mask.unsqueeze(-1)).squeeze(-1)
        b = self.pair_bias_attn(s=b, z=bias, mask=mask, multiplicity=multiplicity, k_in=k_in)
    t_eps = tr.adaln.a_norm.eps
    x_op = None
    if b.shape == a.shape and b.dtype == torch.float32:
        if side.split:  # the residual update and the transition's AdaLN operand in one pass
            rows, x_op = ops.gated_residual_adaln_split3(b.reshape(-1, d).contiguous(), gate_a, rows, scale_t, shift_t,
                                                         t_eps)
        else:
            rows = ops.gated_residual(b.reshape(-1, d).contiguous(), gate_a, rows)
    else:
        rows = (a + torch.sigmoid(gate_a).reshape(a.shape) * b).reshape(-1, d)
    if side.split:
        if x_op is None:
            x_op = ops.adaln_split3(rows, scale_t, shift_t, t_eps)
        u = ops.mm_split(x_op, ops.x3_weight(
            tr, "swish_a2b_x3", (tr.swish_gate[0].weight, tr.a_to_b.weight), (tr.swish_gate[0].bias, tr.a_to_b.bias)))
        b2a = tr.b_to_a
        y = ops.mm_split(ops.swiglu_split3(u, tr.a_to_b.out_features),
                         ops.x3_weight(b2a, "x3", (b2a.weight,), (b2a.bias,)))
    else:
        x = ops.adaln_modulate(rows, scale_t, shift_t, t_eps)
        y = _linear(tr.b_to_a, ops.epilogue(_linear(tr.swish_gate[0], x), _linear(tr.a_to_b, x), None,
                                            ops.GATED_SWIGLU))
    if nxt is not None:  # the residual update and the next layer's attention operand in one pass
        mods_n, gates_n = _conditioning(nxt, side, nxt.adaln.s_norm.eps)
        rows, op_n = ops.gated_residual_adaln_split3(y.reshape(rows.shape), gate_t, rows, mods_n[:, :d],
                                                     mods_n[:, d:2 * d], nxt.adaln.a_norm.eps, out=rows)
        return rows.view(a.shape), (op_n, mods_n, gates_n)
    rows = ops.gated_residual(y.reshape(rows.shape), gate_t, rows, out=rows)
    return self.post_lnorm(rows.view(a.shape))


def _layer_per_linear(self, a, s, bias, mask, to_keys, multiplicity):
    """The layer with each conditioning projection called on its own (memoised
    or hooked projections keep their behaviour); output gates fused."""
    b = self.adaln(a, s)
    k_in = b
    if to_keys is not None:
        k_in = to_keys(b)
        mask = to_keys(mask.unsqueeze(-1)).squeeze(-1)
    b = self.pair_bias_attn(s=b, z=bias, mask=mask, multiplicity=multiplicity, k_in=k_in)
    if b.shape == a.shape and b.dtype == torch.float32:
        a = ops.epilogue(b.contiguous(), _linear(self.output_projection_linear, s), a, ops.MODULATION)
    else:
        a = a + self.output_projection(s) * b
    block = self.transition
    if _patched_with(block, transition_forward) and _plain(block) and _transition_ok(block, a, s):
        y, gate = _transition_inner(block, a, s)
        a = ops.epilogue(y, gate, a, ops.MODULATION)
    else:
        a = a + block(a, s)
    return self.post_lnorm(a)


def _with_side_ok(layer, a, s) -> bool:
    """Whether ``_layer`` runs the layer as ``_layer_with_side``."""
    return (eligible(layer, a, s) and a.shape == s.shape and a.shape[-1] % 4 == 0 and _plain(layer.output_projection)
            and _side_ok(layer, a, s) and layer.transition.adaln.s_norm.eps == layer.adaln.s_norm.eps)


def _layer(self, a, s, bias, mask, to_keys, multiplicity, side):
    if not (eligible(self, a, s) and a.shape == s.shape and a.shape[-1] % 4 == 0 and _plain(self.output_projection)):
        return type(self).forward(self, a, s, bias, mask, to_keys, multiplicity)
    if _side_ok(self, a, s) and self.transition.adaln.s_norm.eps == self.adaln.s_norm.eps:
        return _layer_with_side(self, a, s, side if side is not None else _Side(s), bias, mask, to_keys,
                                multiplicity)
    return _layer_per_linear(self, a, s, bias, mask, to_keys, multiplicity)


def layer_forward(self, a, s, bias=None, mask=None, to_keys=None, multiplicity=1):
    """Drop-in for ``DiffusionTransformerLayer.forward``.

    With nothing hooked or memoised on the conditioning path, the layer's six
    conditioning projections (both AdaLNs' s_scale / s_bias after s_norm, both
    output gates) run as two GEMMs, one on LayerNorm-without-affine(s) with the
    s_norm affines folded into the weights and one on s; the AdaLN
    modulations, the transition's swish_gate | a_to_b projection and SwiGLU,
    and both output gates with their residual adds
    (``a + sigmoid(gate) * b``) read column slices of those projections.  In
    split-bf16 mode the AdaLN and SwiGLU passes write the split operands of
    the next GEMM directly.  Otherwise (memoised or hooked projections, a
    transition forward other than ``transition_forward``) each projection is
    called on its own and only the gates are fused; off the kernels' domain the
    class forward runs."""
    return _layer(self, a, s, bias, mask, to_keys, multiplicity, None)


def stack_forward(self, a, s, bias=None, mask=None, to_keys=None, multiplicity=1):
    """Drop-in for ``DiffusionTransformer.forward`` (upstream transformersv2):
    the same per-layer loop, with the layers' operands of s built once per
    call and shared (``_Side``).  Upstream runs when a layer is not patched
    with ``layer_forward`` or is hooked, in training and under grad."""
    layers = list(self.layers)
    if not (inference(self) and layers and all(_patched_with(l, layer_forward) and _plain(l) for l in layers)
            and eligible(self, a, s)):
        return type(self).forward(self, a, s, bias, mask, to_keys, multiplicity)
    if getattr(self, "pair_bias_attn", True):
        n_b, n, m, d = bias.shape
        bias = bias.view(n_b, n, m, len(layers), d // len(layers))
    side = _Side(s)
    # consecutive layers on the operand path chain their boundary passes: layer
    # i's last residual update also writes layer i + 1's attention operand
    chain = [_with_side_ok(l, a, s) and _operand_path(l, side, to_keys) for l in layers]
    carry = None
    for i, layer in enumerate(layers):
        bias_l = bias[:, :, :, i] if getattr(self, "pair_bias_attn", True) else None
        if chain[i]:
            nxt = layers[i + 1] if (i + 1 < len(layers) and chain[i + 1]
                                    and isinstance(layer.post_lnorm, torch.nn.Identity)) else None
            out = _layer_with_side(layer, a, s, side, bias_l, mask, to_keys, multiplicity, carry=carry, nxt=nxt)
            a, carry = out if nxt is not None else (out, None)
        else:
            a, carry = _layer(layer, a, s, bias_l, mask, to_keys, multiplicity, side), None
    return a


# ---------------------------------------------------------------- atom windows

_WINDOW_PROBES = weakref.WeakKeyDictionary()  # to_keys -> {(n, w, h, device): key offset or None}


def window_key_offset(to_keys, n, w, h, device):
    """The key offset koff if ``to_keys`` maps [1, n, 1] atom rows to [1, n / w,
    h, 1] key windows as the window gather (key j of window k is atom
    k w + koff + j, zero outside 0 .. n - 1; koff = (w - h) / 2, the map of
    upstream single_to_keys through get_indexing_matrix), else None.  Checked
    once per to_keys object and shape on a probe of atom numbers (upstream's
    to_keys is one 0/1 matrix product per channel, so the probe's image fixes
    it); the check synchronises with the device once."""
    key = (n, w, h, str(device))
    try:
        seen = _WINDOW_PROBES.setdefault(to_keys, {})
    except TypeError:  # not weak-referenceable: probe every time
        seen = {}
    if key not in seen:
        koff = (w - h) // 2
        ok = n % w == 0 and (w - h) % 2 == 0
        if ok:
            probe = torch.arange(1, n + 1, device=device, dtype=torch.float32).view(1, n, 1)
            t = torch.arange(n // w, device=device)[:, None] * w + koff + torch.arange(h, device=device)[None, :]
            want = torch.where((t >= 0) & (t < n), t + 1, torch.zeros_like(t)).float()
            got = to_keys(probe)
            ok = isinstance(got, torch.Tensor) and got.numel() == want.numel() and torch.equal(
                got.reshape(want.shape).float(), want)
        seen[key] = koff if ok else None
    return seen[key]


class _WindowKeys:
    """The atom transformer's to_keys as addressing for ``windowed_attention``:
    ``windows`` per sample, keys from atom ``offset`` relative to each window,
    ``bias_group`` windows (the samples of one structure) sharing bias
    elements, and the flat atom ``mask``."""

    def __init__(self, windows, offset, bias_group, mask):
        self.windows, self.offset, self.bias_group, self.mask = windows, offset, bias_group, mask


def _windowed_layer_ok(layer, a, s) -> bool:
    return (_patched_with(layer, layer_forward) and _plain(layer) and eligible(layer, a, s) and a.shape == s.shape
            and a.shape[-1] % 4 == 0 and _plain(layer.output_projection) and _side_ok(layer, a, s)
            and layer.transition.adaln.s_norm.eps == layer.adaln.s_norm.eps and windowed_ok(layer.pair_bias_attn))


def atom_transformer_forward(self, q, c, bias, to_keys, mask, multiplicity=1, *args, **kwargs):
    """Drop-in for ``AtomTransformer.forward`` (upstream transformersv2).

    Upstream windows q and c into [B * N / W, W, D], repeats the per-structure
    bias [B, N / W, W, H, layers * heads] over the samples and runs its
    DiffusionTransformer with ``to_keys`` gathering each window's H key atoms
    (single_to_keys: a 0/1 matrix product, zero rows past the ends).  Here,
    when the stack's layers run the fused path and ``to_keys`` is verified to
    be that gather (``window_key_offset``), nothing is gathered or repeated:
    each layer projects q | k | v | g on the atom rows and the attention kernel
    reads each window's keys, key mask and the shared bias by address.
    Otherwise upstream."""
    stack = getattr(self, "diffusion_transformer", None)
    w, h = self.attn_window_queries, self.attn_window_keys
    if args or kwargs or stack is None or not _patched_with(stack, stack_forward) or not _plain(stack):
        return type(self).forward(self, q, c, bias, to_keys, mask, multiplicity, *args, **kwargs)
    layers = list(stack.layers)
    b, n, d = q.shape
    nw = n // w if w else 0
    ok = (inference(self) and layers and getattr(stack, "pair_bias_attn", True) and nw > 0 and n % w == 0
          and isinstance(bias, torch.Tensor) and bias.dim() == 5 and bias.shape[0] * multiplicity == b
          and tuple(bias.shape[1:4]) == (nw, w, h) and bias.shape[4] % len(layers) == 0
          and bias.dtype == torch.float32 and c.shape[:2] == (b, n) and mask.shape == (b, n))
    if ok:
        qw, cw = q.reshape(b * nw, w, d), c.reshape(b * nw, w, -1)
        ok = all(_windowed_layer_ok(layer, qw, cw) for layer in layers)
    koff = window_key_offset(to_keys, n, w, h, q.device) if ok else None
    if koff is None:
        return type(self).forward(self, q, c, bias, to_keys, mask, multiplicity, *args, **kwargs)
    keys = _WindowKeys(nw, koff, multiplicity * nw, mask.float().reshape(-1).contiguous())
    if not window_bias_prepared(bias):
        bias = prepare_window_bias(bias)
    heads = bias.shape[4] // len(layers)
    side = _Side(cw)
    a = qw
    carry = None
    for i, layer in enumerate(layers):
        # with split linears, consecutive layers chain their boundary pass as the token transformer's do
        nxt = (layers[i + 1] if side.split and i + 1 < len(layers) and isinstance(layer.post_lnorm, torch.nn.Identity)
               else None)
        out = _layer_with_side(layer, a, cw, side, bias[..., i * heads:(i + 1) * heads], None, None, 1, keys,
                               carry=carry, nxt=nxt)
        a, carry = out if nxt is not None else (out, None)
    return a.view(b, n, d)
