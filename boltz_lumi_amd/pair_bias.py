"""AttentionPairBias on gfx950: the fused pair-biased attention and the
dense token-transformer bias storage.

Reference: src/boltz_lumi/pair_bias.py.
  prepare_token_bias (:6-13)  packs the diffusion token transformer's fixed
                              [B, Q, K, layers * heads] bias so that every
                              layer's [B, heads, Q, K] slice is dense.
  prepared_forward (:15-36)   the token transformer's AttentionPairBias
                              forward (installed at adapters.py:39-42).
Here the logits / softmax / PV / gate part of the token transformer's, the
atom transformer's (windows of 32 queries over 128 ``to_keys`` rows) and the
Pairformer trunk's AttentionPairBias runs as one kernel
(``bmx_seq_attention_batched_fwd``, 24, 32 or 48 dims per head, every batch
element in one launch): the [B, H, NQ, NK] logits never exist in HBM.
Projections stay on hipBLASLt; with ``k_in is s`` the four input projections
are one GEMM whose column slices the kernel reads in place.  In fp32 at 512 channels and up (the token
transformer's 768) the projections are split-bf16 GEMMs with fp32
accumulation (``ops.mm_x3``, about 2^-16 relative per product).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import ops


def prepare_token_bias(value: torch.Tensor) -> torch.Tensor:
    """The same logical [B, Q, K, L*H] tensor (values unchanged, fp32) stored
    head-major, so ``value[..., l*H:(l+1)*H].movedim(-1, 1)`` is dense per batch
    element (reference pair_bias.py:6-13)."""
    dense = torch.empty((value.shape[0], value.shape[3], value.shape[1], value.shape[2]), device=value.device,
                        dtype=torch.float32)
    dense.copy_(value.movedim(-1, 1))
    return dense.movedim(1, -1)


def prepare_window_bias(value: torch.Tensor) -> torch.Tensor:
    """The atom transformer's window bias, logically [B, K, W, H, layers * heads]
    (values unchanged, fp32), stored channel-major: every head's [K, W, H] block
    is dense, so a layer's heads (``value[..., l*heads:(l+1)*heads]``) give the
    windowed attention 16-byte bias rows.  Like ``prepare_token_bias`` for the
    token transformer; done once per sampling call, or per stack call where the
    bias arrives in upstream's layout."""
    dense = torch.empty((value.shape[0], value.shape[4]) + tuple(value.shape[1:4]), device=value.device,
                        dtype=torch.float32)
    dense.copy_(value.movedim(-1, 1))
    return dense.movedim(1, -1)


def window_bias_prepared(value: torch.Tensor) -> bool:
    """``value`` has the layout ``prepare_window_bias`` writes."""
    if value.dim() != 5 or value.dtype != torch.float32:
        return False
    _, k, w, h, _ = value.shape
    return value.stride()[1:] == (w * h, h, 1, k * w * h)


def _joint_projection(module, name, x, linears):
    """``cat([lin(x) for lin in linears], -1)`` as one GEMM (fp32 result) with the
    concatenated weights cached on ``module``: in the autocast dtype under
    autocast, else fp32 (split-bf16 where ``ops.use_split`` says so)."""
    weights = tuple(lin.weight for lin in linears)
    biases = [lin.bias for lin in linears]
    if not torch.is_autocast_enabled() and ops.use_split(x.shape[-1], x.numel() // max(x.shape[-1], 1),
                                                         sum(lin.weight.shape[0] for lin in linears)):
        y = ops.mm_x3(x.reshape(-1, x.shape[-1]), ops.x3_weight(module, name + "_x3", weights, biases))
        return y.view(x.shape[:-1] + (y.shape[-1],))
    bias = None
    if any(b is not None for b in biases):
        srcs = tuple(b for b in biases if b is not None)
        bias = ops.cached_weight(module, name + "_bias", srcs, lambda *bs: torch.cat(
            [b.float() if b is not None else lin.weight.new_zeros(lin.out_features, dtype=torch.float32)
             for b, lin in zip(biases, linears)]))
    w = ops.cached_weight(module, name, weights, lambda *ws: torch.cat(ws, 0).float())
    return F.linear(x if torch.is_autocast_enabled() else x.float(), w, bias).float()


def fused_attention(module, s, z, mask, k_in, multiplicity=1, bias=None):
    """``sigmoid(proj_g(s)) * attention`` of an upstream-style AttentionPairBias
    ``module`` before ``proj_o`` ([B, NQ, c_s], fp32), or None where the kernel
    does not apply (CPU, grad, training, a head width other than 24, 32 or 48,
    shapes upstream would not broadcast the same way).

    ``bias`` is ``module.proj_z(z)`` ([B / multiplicity, H, NQ, NK]) when not
    given; batch element i uses bias ``i // multiplicity`` (upstream
    ``repeat_interleave``, pair_bias.py:26-27).  ``k_in`` may differ from ``s``
    in length (the atom transformer's windows attend ``to_keys`` rows).  Under
    autocast the projections run in its dtype and are widened to fp32 for the
    attention, as upstream does (:29-33).  All batch elements run in one
    launch."""
    heads, width = module.num_heads, module.c_s
    if not (s.is_cuda and k_in.is_cuda and s.dim() == 3 and k_in.dim() == 3 and k_in.shape[0] == s.shape[0]
            and width % heads == 0 and width // heads in (24, 32, 48) and heads <= 64
            and not module.training and not torch.is_grad_enabled()):
        return None
    batch, nq, nk = s.shape[0], s.shape[1], k_in.shape[1]
    if k_in is s:
        weights = (module.proj_q.weight, module.proj_k.weight, module.proj_v.weight, module.proj_g.weight)
        if not torch.is_autocast_enabled() and ops.use_split(width, s.numel() // width, 4 * width):
            # fp32 at the token transformer's width or rows: one split-bf16 GEMM with fp32 accumulation
            biases = (module.proj_q.bias, module.proj_k.bias, module.proj_v.bias, module.proj_g.bias)
            proj = ops.mm_x3(s.reshape(-1, width), ops.x3_weight(module, "qkvg_x3", weights, biases))
            proj = proj.view(s.shape[:-1] + (4 * width,))
        else:
            bq = ops.cached_weight(module, "qkvg_bias", (module.proj_q.bias,),
                                   lambda b: torch.cat([b.float(), b.new_zeros(3 * width)]))
            w = ops.cached_weight(module, "qkvg", weights, lambda *ws: torch.cat(ws, 0).float())
            proj = F.linear(s if torch.is_autocast_enabled() else s.float(), w, bq).float()
        q, k, v, g = proj.split(width, dim=-1)
    else:  # q | g on the queries and k | v on the key rows, two GEMMs whose column slices the kernel reads
        q, g = _joint_projection(module, "qg", s, (module.proj_q, module.proj_g)).split(width, dim=-1)
        k, v = _joint_projection(module, "kv", k_in, (module.proj_k, module.proj_v)).split(width, dim=-1)
    return _attend(module, q, k, v, g, z, mask, multiplicity, bias)


def _attend(module, q, k, v, g, z, mask, multiplicity, bias=None, split_out=False):
    """The attention of ``fused_attention`` from its projections ([B, NQ / NK,
    H * D] column slices), or None where shapes do not match; ``split_out``:
    as the split-bf16 operand of ``proj_o`` (``ops.seq_attention_batched``)."""
    heads = module.num_heads
    batch, nq, nk = q.shape[0], q.shape[1], k.shape[1]
    if bias is None:
        bias = module.proj_z(z)
    bias = bias.float()
    if bias.dim() != 4 or bias.shape[0] * multiplicity != batch or tuple(bias.shape[1:]) != (heads, nq, nk):
        return None
    if not bias[0].is_contiguous():
        bias = bias.contiguous()
    m = mask.float()
    if m.dim() != 2 or m.shape[1] != nk or m.shape[0] not in (1, batch):
        return None
    if m.stride(1) != 1:
        m = m.contiguous()
    if split_out:
        return ops.seq_attention_batched(q, k, v, bias, m, g, module.inf, bias_div=multiplicity, split=True,
                                         split_out=True)
    return ops.seq_attention_batched(q, k, v, bias, m, g, module.inf, bias_div=multiplicity)


def operand_ok(module) -> bool:
    """``attention_from_operand`` applies: a patched, unhooked AttentionPairBias
    with a given bias, 24 / 32 / 48 dims per head, whose linears run split
    (``ops.use_split``)."""
    fwd = vars(module).get("forward")
    heads, width = module.num_heads, module.c_s
    return (getattr(fwd, "__func__", None) is prepared_forward and not module._forward_hooks
            and not module._forward_pre_hooks and not module.compute_pair_bias and not module.training
            and width % heads == 0 and width // heads in (24, 32, 48) and heads <= 64 and ops.use_split(width))


def attention_from_operand(module, op, shape, z, mask, multiplicity=1, split_out=False):
    """``fused_attention(module, s, z, mask, s, multiplicity)`` when the caller
    holds s only as its split-bf16 operand ``op`` ([B * N, 3 c_s + 64], e.g.
    the AdaLN output written by ``ops.adaln_split3``): the q | k | v | g
    projection is one GEMM of ``op``.  ``shape`` is s's [B, N, c_s].  With
    ``split_out`` the result comes as the split-bf16 operand of ``proj_o``
    when the split-bf16 attention kernel applies (else fp32 [B, N, c_s])."""
    width = module.c_s
    lin = (module.proj_q, module.proj_k, module.proj_v, module.proj_g)
    w3 = ops.x3_weight(module, "qkvg_x3", tuple(m.weight for m in lin), tuple(m.bias for m in lin))
    proj = ops.mm_split(op, w3).view(tuple(shape[:-1]) + (4 * width,))
    q, k, v, g = proj.split(width, dim=-1)
    split_out = split_out and ops.seq_attention_split_ok(q, g, k.shape[1])
    return _attend(module, q, k, v, g, z, mask, multiplicity, split_out=split_out)


def windowed_ok(module) -> bool:
    """``windowed_attention`` applies: a patched, unhooked AttentionPairBias with
    a given bias, 24 / 32 / 48 dims per head and no bias on proj_k / proj_v (a
    zero key row then projects to zero, as the gather's zero rows do)."""
    fwd = vars(module).get("forward")
    heads, width = module.num_heads, module.c_s
    return (getattr(fwd, "__func__", None) is prepared_forward and not module._forward_hooks
            and not module._forward_pre_hooks and not module.compute_pair_bias and not module.training
            and width % heads == 0 and width // heads in (24, 32, 48) and heads <= 64
            and module.proj_k.bias is None and module.proj_v.bias is None)


def windowed_attention(module, s, bias, keys, op=None, shape=None):
    """``sigmoid(proj_g(s)) * attention`` of AttentionPairBias ``module`` (before
    ``proj_o``) for query windows s [E, W, c_s] whose keys are the window gather
    of the same rows (upstream ``to_keys``): q | k | v | g are one projection of
    the atom rows and the kernel reads each window's keys by address
    (``ops.seq_attention_windowed``), so neither the gathered rows nor their
    projection is materialised.  ``keys`` carries the gather (``windows``,
    ``offset``, ``bias_group``, the atom ``mask``); ``bias`` is this layer's
    [Eb, ..., W, NK, heads] view of the atom bias.  With ``op`` the rows come
    as their split-bf16 operand ([E W, 3 c_s + 64], e.g. written by
    ``ops.adaln_split3``; s is then None and ``shape`` its [E, W, c_s])."""
    e, w, width = s.shape if op is None else shape
    lin = (module.proj_q, module.proj_k, module.proj_v, module.proj_g)
    if op is None:
        proj = _joint_projection(module, "qkvg", s.reshape(e * w, width), lin)
    else:  # the weights _joint_projection caches for its split form
        proj = ops.mm_split(op, ops.x3_weight(module, "qkvg_x3", tuple(m.weight for m in lin),
                                              tuple(m.bias for m in lin)))
    q, k, v, g = proj.split(width, dim=-1)
    return ops.seq_attention_windowed(q.view(e, w, width), k, v, bias.float(), keys.mask, g.view(e, w, width),
                                      module.inf, windows=keys.windows, key_offset=keys.offset,
                                      bias_group=keys.bias_group)


def prepared_forward(module, s, z, mask, k_in, multiplicity=1):
    """Drop-in for the score model's ``AttentionPairBias.forward`` (reference
    pair_bias.py:15-36, installed there on the token transformer's; here also
    on the atom transformer's windowed ones); upstream forward under grad, in
    training, for ``compute_pair_bias`` modules and where the kernel does not
    apply."""
    o = None
    if not (torch.is_grad_enabled() or module.training or module.compute_pair_bias):
        o = fused_attention(module, s, z, mask, k_in, multiplicity)
    if o is None:
        return type(module).forward(module, s, z, mask, k_in, multiplicity)
    if torch.is_autocast_enabled() or "forward" in vars(module.proj_o):
        return module.proj_o(o)
    return ops.linear_fp32(o, module.proj_o)
