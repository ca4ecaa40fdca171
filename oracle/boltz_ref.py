"""fp32 CPU restatement of the upstream Boltz 2.2.1 hot-path modules.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Upstream Boltz (``boltz==2.2.1``, commit cb04aec, pinned by the reference at
``requirements.txt:1`` and ``third_party/README.md:8-9``) is not vendored in
``/root/reference`` and is not installed here.  Each class below restates the
upstream module's published algorithm with the same class name, parameter
names and shapes, and cites the reference lines that call or corroborate it.
Forward passes run in fp32 (Boltz with autocast disabled).  Under
``torch.autocast(bf16)`` the same modules follow upstream's bf16-mixed
inference (linears and matmuls autocast, LayerNorm and softmax in fp32, the
Pairformer sequence stack with autocast disabled), which the GPU tests use as
upstream's own bf16 path.
"""

from __future__ import annotations

import math

import torch
from torch import nn
import torch.nn.functional as F


# --------------------------------------------------------------------------
# Primitives
# --------------------------------------------------------------------------


class LayerNorm(nn.Module):
    """OpenFold-style LayerNorm used by Boltz's triangle attention.

    Upstream ``boltz.model.layers.triangular_attention.primitives.LayerNorm``:
    ``c_in`` is stored as a tuple and the forward is ``F.layer_norm`` (the
    reference checks ``c_in == (128,)`` and reads ``eps`` at
    ``triangle.py:119,139``).
    """

    def __init__(self, c_in: int, eps: float = 1e-5):
        super().__init__()
        self.c_in = (c_in,)
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(c_in))
        self.bias = nn.Parameter(torch.zeros(c_in))

    def forward(self, x):
        return F.layer_norm(x, self.c_in, self.weight, self.bias, self.eps)


def _at_least_f32(t: torch.Tensor) -> torch.Tensor:
    """Upstream's ``.float()`` casts; kept a no-op for fp64 pinning runs."""
    return t if t.dtype == torch.float64 else t.float()


def permute_final_dims(t: torch.Tensor, inds):
    zero_index = -1 * len(inds)
    first_inds = list(range(len(t.shape[:zero_index])))
    return t.permute(first_inds + [zero_index + i for i in inds])


def flatten_final_dims(t: torch.Tensor, no_dims: int):
    return t.reshape(t.shape[:-no_dims] + (-1,))


class Attention(nn.Module):
    """Gated multi-head attention with a list of additive biases.

    Upstream ``primitives.Attention``.  The reference's replacement
    (``triangle.py:32-104``) follows it step by step: ``_prep_qkv`` with
    ``q /= sqrt(c_hidden)`` (``:80``), ``S = q k^T`` (``:87``), mask bias then
    triangle bias added (``kernels/triangle_softmax.py:90-92``), softmax over
    keys, ``P v`` and the transpose (``:101``), then ``_wrap_up``: sigmoid gate
    from ``linear_g(q_x)`` and ``linear_o`` (``:104``).
    """

    def __init__(self, c_q, c_k, c_v, c_hidden, no_heads, gating=True):
        super().__init__()
        self.c_q, self.c_k, self.c_v = c_q, c_k, c_v
        self.c_hidden = c_hidden
        self.no_heads = no_heads
        self.gating = gating
        self.linear_q = nn.Linear(c_q, c_hidden * no_heads, bias=False)
        self.linear_k = nn.Linear(c_k, c_hidden * no_heads, bias=False)
        self.linear_v = nn.Linear(c_v, c_hidden * no_heads, bias=False)
        self.linear_o = nn.Linear(c_hidden * no_heads, c_q)
        self.linear_g = nn.Linear(c_q, c_hidden * no_heads) if gating else None
        self.sigmoid = nn.Sigmoid()

    def _prep_qkv(self, q_x, kv_x, apply_scale=True):
        q = self.linear_q(q_x)
        k = self.linear_k(kv_x)
        v = self.linear_v(kv_x)
        q = q.view(q.shape[:-1] + (self.no_heads, -1)).transpose(-2, -3)
        k = k.view(k.shape[:-1] + (self.no_heads, -1)).transpose(-2, -3)
        v = v.view(v.shape[:-1] + (self.no_heads, -1)).transpose(-2, -3)
        if apply_scale:
            q = q / math.sqrt(self.c_hidden)
        return q, k, v

    def _wrap_up(self, o, q_x):
        if self.linear_g is not None:
            g = self.sigmoid(self.linear_g(q_x))
            g = g.view(g.shape[:-1] + (self.no_heads, -1))
            o = o * g
        o = flatten_final_dims(o, 2)
        return self.linear_o(o)

    def forward(self, q_x, kv_x, tri_bias, mask_bias, mask=None, use_kernels=False):
        q, k, v = self._prep_qkv(q_x, kv_x)
        a = torch.matmul(q, k.transpose(-1, -2))
        a = a + mask_bias
        a = a + tri_bias
        a = torch.softmax(a, dim=-1)
        o = torch.matmul(a, v).transpose(-2, -3)
        return self._wrap_up(o, q_x)


# --------------------------------------------------------------------------
# Triangle attention  (reference: triangle.py)
# --------------------------------------------------------------------------


class TriangleAttention(nn.Module):
    """Upstream ``triangular_attention.attention.TriangleAttention``.

    Ending node: transpose x and mask, run the starting-node math, transpose
    back (reference comment ``triangle.py:131``).  ``mask_bias =
    inf * (mask - 1)`` shaped ``[*, I, 1, 1, J]`` and the triangle bias
    ``linear(x)`` permuted to ``[*, 1, H, I, J]`` (shapes asserted by the
    reference at ``kernels/triangle_block_softmax_hip.cu:132-133``).
    ``chunk_size`` only bounds memory (upstream ``chunk_layer`` over the row
    axis); the math per row is unchanged.
    """

    def __init__(self, c_in, c_hidden, no_heads, starting=True, inf=1e9):
        super().__init__()
        self.c_in = c_in
        self.c_hidden = c_hidden
        self.no_heads = no_heads
        self.starting = starting
        self.inf = inf
        self.layer_norm = LayerNorm(c_in)
        self.linear = nn.Linear(c_in, no_heads, bias=False)
        self.mha = Attention(c_in, c_in, c_in, c_hidden, no_heads)

    def forward(self, x, mask=None, chunk_size=None, use_kernels=False):
        if mask is None:
            mask = x.new_ones(x.shape[:-1])
        if not self.starting:
            x = x.transpose(-2, -3)
            mask = mask.transpose(-1, -2)
        x = self.layer_norm(x)
        mask_bias = (self.inf * (mask - 1))[..., :, None, None, :]
        tri_bias = permute_final_dims(self.linear(x), (2, 0, 1)).unsqueeze(-4)
        if chunk_size is None:
            out = self.mha(x, x, tri_bias, mask_bias, mask)
        else:
            rows = x.shape[-3]
            parts = []
            for start in range(0, rows, chunk_size):
                sl = slice(start, start + chunk_size)
                parts.append(
                    self.mha(x[..., sl, :, :], x[..., sl, :, :], tri_bias, mask_bias[..., sl, :, :, :], None)
                )
            out = torch.cat(parts, dim=-3)
        if not self.starting:
            out = out.transpose(-2, -3)
        return out

    def forward_rows(self, x, mask, rows, chunk: int = 64):
        """``forward(x, mask)`` restricted to the output pairs of the given
        rows: ``[*, R, N, C]`` for the starting node (pairs ``(i, :)``) and
        ``[*, N, R, C]`` for the ending node (pairs ``(:, i)``).  It is the
        chunk path of :meth:`forward`, one selected row per chunk, with the
        triangle bias (which needs all of ``x``) built from ``chunk`` rows of
        ``x`` at a time, so no intermediate exceeds ``max(chunk, H) * N^2 * C``
        elements."""
        if mask is None:
            mask = x.new_ones(x.shape[:-1])
        if not self.starting:
            x = x.transpose(-2, -3)
            mask = mask.transpose(-1, -2)
        n = x.shape[-3]
        tri_bias = torch.cat(
            [permute_final_dims(self.linear(self.layer_norm(x[..., s:s + chunk, :, :])), (2, 0, 1))
             for s in range(0, n, chunk)], dim=-2).unsqueeze(-4)
        mask_bias = (self.inf * (mask - 1))[..., :, None, None, :]
        parts = []
        for i in rows:
            xi = self.layer_norm(x[..., i:i + 1, :, :])
            parts.append(self.mha(xi, xi, tri_bias, mask_bias[..., i:i + 1, :, :, :], None))
        out = torch.cat(parts, dim=-3)
        if not self.starting:
            out = out.transpose(-2, -3)
        return out


class TriangleAttentionEndingNode(TriangleAttention):
    def __init__(self, c_in, c_hidden, no_heads, inf=1e9):
        super().__init__(c_in, c_hidden, no_heads, starting=False, inf=inf)


TriangleAttentionStartingNode = TriangleAttention


# --------------------------------------------------------------------------
# Triangle multiplication  (reference: multiplication.py, rows A4-A6)
# --------------------------------------------------------------------------


class _TriangleMultiplication(nn.Module):
    """Upstream ``triangular_mult.TriangleMultiplication{Outgoing,Incoming}``.

    ``x = norm_in(x)``; ``x = p_in(x) * sigmoid(g_in(x)) * mask``; ``a, b``
    are channels 0..C-1 and C..2C-1 (``multiplication_gate_hip.cu:38-40``);
    outgoing ``o_ijc = sum_k a_ikc b_jkc``, incoming ``o_ijc = sum_k a_kic
    b_kjc`` (operand layouts ``multiplication.py:105-116``); then
    ``p_out(norm_out(o)) * sigmoid(g_out(x_in))`` (``multiplication.py:124-137``).
    """

    outgoing = True

    def __init__(self, dim: int = 128):
        super().__init__()
        self.norm_in = nn.LayerNorm(dim, eps=1e-5)
        self.p_in = nn.Linear(dim, 2 * dim, bias=False)
        self.g_in = nn.Linear(dim, 2 * dim, bias=False)
        self.norm_out = nn.LayerNorm(dim)
        self.p_out = nn.Linear(dim, dim, bias=False)
        self.g_out = nn.Linear(dim, dim, bias=False)

    def forward(self, x, mask, use_kernels=False):
        x = self.norm_in(x)
        x_in = x
        x = self.p_in(x) * self.g_in(x).sigmoid()
        x = x * mask.unsqueeze(-1)
        a, b = torch.chunk(_at_least_f32(x), 2, dim=-1)
        if self.outgoing:
            x = torch.einsum("bikd,bjkd->bijd", a, b)
        else:
            x = torch.einsum("bkid,bkjd->bijd", a, b)
        return self.p_out(self.norm_out(x)) * self.g_out(x_in).sigmoid()

    def _operands(self, x, mask):
        x = self.norm_in(x)
        x = self.p_in(x) * self.g_in(x).sigmoid()
        return torch.chunk(_at_least_f32(x * mask.unsqueeze(-1)), 2, dim=-1)

    def forward_rows(self, x, mask, rows, chunk: int = 256):
        """``forward(x, mask)[..., rows, :, :]`` (output pairs ``(i, :)``,
        ``i`` in ``rows``) without the ``N x N x 2C`` operands: the sum over
        ``k`` runs over chunks of ``chunk`` tokens, each chunk's ``a`` / ``b``
        computed from its slice of ``x`` by the same layers as
        :meth:`forward` (outgoing: ``o_ijc = sum_k a_ikc b_jkc``, chunks of
        ``j`` with every ``k``; incoming: ``o_ijc = sum_k a_kic b_kjc``, chunks
        of ``k``).  Rows are gathered by slicing, and each intermediate holds
        at most ``chunk * N * 2C`` elements."""
        n = x.shape[-2]
        x_rows = torch.cat([x[..., i:i + 1, :, :] for i in rows], dim=-3)
        if self.outgoing:
            a, _ = self._operands(x_rows, torch.cat([mask[..., i:i + 1, :] for i in rows], dim=-2))
            parts = []
            for start in range(0, n, chunk):
                _, b = self._operands(x[..., start:start + chunk, :, :], mask[..., start:start + chunk, :])
                parts.append(torch.einsum("bikd,bjkd->bijd", a, b))
            o = torch.cat(parts, dim=-2)
        else:
            o = None
            for start in range(0, n, chunk):
                xs, ms = x[..., start:start + chunk, :, :], mask[..., start:start + chunk, :]
                a, _ = self._operands(torch.cat([xs[..., i:i + 1, :] for i in rows], dim=-2),
                                      torch.cat([ms[..., i:i + 1] for i in rows], dim=-1))
                _, b = self._operands(xs, ms)
                part = torch.einsum("bkid,bkjd->bijd", a, b)
                o = part if o is None else o + part
        x_in = self.norm_in(x_rows)
        return self.p_out(self.norm_out(o)) * self.g_out(x_in).sigmoid()


class TriangleMultiplicationOutgoing(_TriangleMultiplication):
    outgoing = True


class TriangleMultiplicationIncoming(_TriangleMultiplication):
    outgoing = False


# --------------------------------------------------------------------------
# Transition  (reference: pair_transition.py, row A7)
# --------------------------------------------------------------------------


class Transition(nn.Module):
    """Upstream ``layers.transition.Transition``: LN, ``fc3(silu(fc1 x) * fc2 x)``.

    The reference's replacement keeps this order (``pair_transition.py:20-28``)
    and the SiLU-then-multiply rounding (``kernels/pair_hip.cu:12-17``).  The
    chunked branch (taken when ``chunk_size`` is given in eval) splits the
    hidden dimension and sums the partial ``fc3`` products.
    """

    def __init__(self, dim: int = 128, hidden: int = 512, out_dim=None):
        super().__init__()
        out_dim = dim if out_dim is None else out_dim
        self.norm = nn.LayerNorm(dim, eps=1e-5)
        self.fc1 = nn.Linear(dim, hidden, bias=False)
        self.fc2 = nn.Linear(dim, hidden, bias=False)
        self.fc3 = nn.Linear(hidden, out_dim, bias=False)
        self.silu = nn.SiLU()
        self.hidden = hidden

    def forward(self, x, chunk_size=None):
        x = self.norm(x)
        if chunk_size is None or self.training:
            return self.fc3(self.silu(self.fc1(x)) * self.fc2(x))
        w1 = self.fc1.weight.chunk(self.hidden // chunk_size, dim=0)
        w2 = self.fc2.weight.chunk(self.hidden // chunk_size, dim=0)
        w3 = self.fc3.weight.chunk(self.hidden // chunk_size, dim=1)
        out = torch.zeros(x.shape[:-1] + (self.fc3.out_features,), dtype=x.dtype)
        for a, b, c in zip(w1, w2, w3):
            out = out + F.linear(F.silu(F.linear(x, a)) * F.linear(x, b), c)
        return out


# --------------------------------------------------------------------------
# Attention with pair bias (v2)  (reference: pair_bias.py:15-36)
# --------------------------------------------------------------------------


class Rearrange(nn.Module):
    """``einops`` ``"b ... h -> b h ..."`` (moves the last axis to position 1)."""

    def forward(self, x):
        return x.movedim(-1, 1)


class AttentionPairBias(nn.Module):
    """Upstream ``layers.attentionv2.AttentionPairBias``.

    The math is the reference's own restatement (``pair_bias.py:21-36``) with
    ``bias = proj_z(z).repeat_interleave(multiplicity, 0)``.  ``inf`` defaults
    to 1e6 (read as ``module.inf`` at ``pair_bias.py:32``).
    """

    def __init__(self, c_s, c_z=None, num_heads=None, inf=1e6, compute_pair_bias=True):
        super().__init__()
        assert c_s % num_heads == 0
        self.c_s = c_s
        self.num_heads = num_heads
        self.head_dim = c_s // num_heads
        self.inf = inf
        self.proj_q = nn.Linear(c_s, c_s)
        self.proj_k = nn.Linear(c_s, c_s, bias=False)
        self.proj_v = nn.Linear(c_s, c_s, bias=False)
        self.proj_g = nn.Linear(c_s, c_s, bias=False)
        self.compute_pair_bias = compute_pair_bias
        if compute_pair_bias:
            self.proj_z = nn.Sequential(nn.LayerNorm(c_z), nn.Linear(c_z, num_heads, bias=False), Rearrange())
        else:
            self.proj_z = Rearrange()
        self.proj_o = nn.Linear(c_s, c_s, bias=False)

    def forward(self, s, z, mask, k_in, multiplicity=1):
        b = s.shape[0]
        q = self.proj_q(s).view(b, -1, self.num_heads, self.head_dim)
        k = self.proj_k(k_in).view(b, -1, self.num_heads, self.head_dim)
        v = self.proj_v(k_in).view(b, -1, self.num_heads, self.head_dim)
        bias = self.proj_z(z).repeat_interleave(multiplicity, 0)
        g = self.proj_g(s).sigmoid()
        f = _at_least_f32
        attn = torch.einsum("bihd,bjhd->bhij", f(q), f(k))
        attn = attn / (self.head_dim**0.5) + f(bias)
        attn = attn + (1 - f(mask[:, None, None])) * -self.inf
        attn = attn.softmax(dim=-1)
        o = torch.einsum("bhij,bjhd->bihd", attn, f(v)).to(v.dtype)
        o = o.reshape(b, -1, self.c_s)
        return self.proj_o(g * o)


# --------------------------------------------------------------------------
# Pairformer layer
# --------------------------------------------------------------------------


def get_dropout_mask(dropout: float, z: torch.Tensor, training: bool, columnwise: bool = False) -> torch.Tensor:
    """Upstream ``layers.dropout.get_dropout_mask``: one uniform draw per row
    ([B, N, 1, 1]) or per column ([B, 1, N, 1]) of z, kept where it exceeds
    ``dropout * training`` and scaled by ``1 / (1 - dropout * training)``.  The
    draw happens in eval too (rate 0): the mask is then 1 except where a draw
    is exactly 0, and the generator advances."""
    dropout = dropout * training
    v = z[:, 0:1, :, 0:1] if columnwise else z[:, :, 0:1, 0:1]
    d = torch.rand_like(v) > dropout
    return d * 1.0 / (1.0 - dropout)


def _pair_stack(layer, z, pair_mask, chunk_size_tri_attn=None):
    """The pair stack of upstream ``PairformerLayer`` / ``PairformerNoSeqLayer``:
    each of the four triangle updates added through its dropout mask (the
    ending node's column-wise), then the transition."""
    d = get_dropout_mask(layer.dropout, z, layer.training)
    z = z + d * layer.tri_mul_out(z, mask=pair_mask)
    d = get_dropout_mask(layer.dropout, z, layer.training)
    z = z + d * layer.tri_mul_in(z, mask=pair_mask)
    d = get_dropout_mask(layer.dropout, z, layer.training)
    z = z + d * layer.tri_att_start(z, mask=pair_mask, chunk_size=chunk_size_tri_attn)
    d = get_dropout_mask(layer.dropout, z, layer.training, columnwise=True)
    z = z + d * layer.tri_att_end(z, mask=pair_mask, chunk_size=chunk_size_tri_attn)
    return z + layer.transition_z(z)


class PairformerLayer(nn.Module):
    """Upstream ``layers.pairformer.PairformerLayer`` (v2, eval mode).

    Pair stack: ``z += d * tri_mul_out``, ``tri_mul_in``, ``tri_att_start``,
    ``tri_att_end`` (``d`` the ``get_dropout_mask`` draw of each: ones in eval
    except where a draw is exactly 0), then ``z += transition_z``.  Then
    the fp32 sequence stack with autocast disabled: ``s += attention(
    pre_norm_s(s), z)``, ``s += transition_s(s)``, ``s_post_norm`` (Identity in
    the trunk).  Pinned by branch isolation (every branch but one zeroed gives
    ``z + branch(z)`` of the fp64 loop modules), chained branches, and the
    sequence stack on the updated z in fp32 (``tests/test_oracle_pins.py``).
    The op order itself is a restatement of upstream: the reference
    corroborates fp32 ``z`` inputs (``multiplication.py:59``,
    ``triangle.py:113``) and an unpatched s-stack (``adapters.py:39-45``).
    """

    def __init__(self, token_s=384, token_z=128, num_heads=16, dropout=0.25, pairwise_head_width=32,
                 pairwise_num_heads=4, post_layer_norm=False):
        super().__init__()
        self.token_z = token_z
        self.num_heads = num_heads
        self.dropout = dropout
        self.pre_norm_s = nn.LayerNorm(token_s)
        self.attention = AttentionPairBias(token_s, token_z, num_heads)
        self.tri_mul_out = TriangleMultiplicationOutgoing(token_z)
        self.tri_mul_in = TriangleMultiplicationIncoming(token_z)
        self.tri_att_start = TriangleAttention(token_z, pairwise_head_width, pairwise_num_heads, inf=1e9)
        self.tri_att_end = TriangleAttentionEndingNode(token_z, pairwise_head_width, pairwise_num_heads, inf=1e9)
        self.transition_s = Transition(token_s, token_s * 4)
        self.transition_z = Transition(token_z, token_z * 4)
        self.s_post_norm = nn.LayerNorm(token_s) if post_layer_norm else nn.Identity()

    def forward(self, s, z, mask, pair_mask, chunk_size_tri_attn=None, use_kernels=False, use_cuequiv_mul=False,
                use_cuequiv_attn=False):
        z = _pair_stack(self, z, pair_mask, chunk_size_tri_attn)
        # Upstream runs the sequence stack in fp32 with autocast disabled, on
        # the updated z (the reference leaves it unpatched, adapters.py:39-45).
        f = _at_least_f32
        with torch.autocast(device_type=s.device.type, enabled=False):
            s_normed = self.pre_norm_s(f(s))
            s = f(s) + self.attention(s=s_normed, z=f(z), mask=f(mask), k_in=s_normed)
            s = s + self.transition_s(s)
            s = self.s_post_norm(s)
        return s, z


class PairformerNoSeqLayer(nn.Module):
    """Upstream ``layers.pairformer.PairformerNoSeqLayer`` (eval mode): the
    pair stack of ``PairformerLayer`` without the sequence stack.  Upstream
    builds one per ``MSALayer`` (``token_z`` 128) and one per template
    pairformer block (``template_dim`` 64).  The reference patches its modules
    by class name and by the ``.transition_z`` suffix (``adapters.py:24-45``),
    as in the trunk.  ``tests/test_oracle_pins.py`` checks it bit for bit
    against the pair stack of ``PairformerLayer`` (pinned there).
    """

    def __init__(self, token_z=128, dropout=0.25, pairwise_head_width=32, pairwise_num_heads=4):
        super().__init__()
        self.token_z = token_z
        self.dropout = dropout
        self.tri_mul_out = TriangleMultiplicationOutgoing(token_z)
        self.tri_mul_in = TriangleMultiplicationIncoming(token_z)
        self.tri_att_start = TriangleAttention(token_z, pairwise_head_width, pairwise_num_heads, inf=1e9)
        self.tri_att_end = TriangleAttentionEndingNode(token_z, pairwise_head_width, pairwise_num_heads, inf=1e9)
        self.transition_z = Transition(token_z, token_z * 4)

    def forward(self, z, pair_mask, chunk_size_tri_attn=None, use_kernels=False, use_cuequiv_mul=False,
                use_cuequiv_attn=False):
        return _pair_stack(self, z, pair_mask, chunk_size_tri_attn)


# --------------------------------------------------------------------------
# Diffusion conditioning blocks  (reference: diffusion.py, rows A8-A10)
# --------------------------------------------------------------------------


class AdaLN(nn.Module):
    """Upstream ``modules.transformersv2.AdaLN``.

    ``sigmoid(s_scale(s_norm(s))) * a_norm(a) + s_bias(s_norm(s))``; the
    multiply and add round separately (``diffusion.py:55-57``,
    ``kernels/diffusion_hip.cu:15-18``).
    """

    def __init__(self, dim, dim_single_cond):
        super().__init__()
        self.a_norm = nn.LayerNorm(dim, elementwise_affine=False, bias=False)
        self.s_norm = nn.LayerNorm(dim_single_cond, bias=False)
        self.s_scale = nn.Linear(dim_single_cond, dim)
        self.s_bias = nn.Linear(dim_single_cond, dim, bias=False)

    def forward(self, a, s):
        a = self.a_norm(a)
        s = self.s_norm(s)
        return torch.sigmoid(self.s_scale(s)) * a + self.s_bias(s)


class SwiGLU(nn.Module):
    """``silu(u[..., D:]) * u[..., :D]`` (half order: ``diffusion_hip.cu:39-42``)."""

    def forward(self, x):
        x, gates = x.chunk(2, dim=-1)
        return F.silu(gates) * x


class ConditionedTransitionBlock(nn.Module):
    """Upstream ``transformersv2.ConditionedTransitionBlock`` (expansion 2).

    ``b = swish_gate(adaln(a, s)) * a_to_b(adaln(a, s))``;
    ``out = sigmoid(output_projection[0](s)) * b_to_a(b)``
    (``diffusion.py:63-67``).
    """

    def __init__(self, dim_single, dim_single_cond, expansion_factor=2):
        super().__init__()
        self.adaln = AdaLN(dim_single, dim_single_cond)
        dim_inner = int(dim_single * expansion_factor)
        self.swish_gate = nn.Sequential(nn.Linear(dim_single, dim_inner * 2, bias=False), SwiGLU())
        self.a_to_b = nn.Linear(dim_single, dim_inner, bias=False)
        self.b_to_a = nn.Linear(dim_inner, dim_single, bias=False)
        output_projection_linear = nn.Linear(dim_single_cond, dim_single)
        nn.init.zeros_(output_projection_linear.weight)
        nn.init.constant_(output_projection_linear.bias, -2.0)
        self.output_projection = nn.Sequential(output_projection_linear, nn.Sigmoid())

    def forward(self, a, s):
        a = self.adaln(a, s)
        b = self.swish_gate(a) * self.a_to_b(a)
        return self.output_projection(s) * self.b_to_a(b)


class DiffusionTransformerLayer(nn.Module):
    """Upstream ``transformersv2.DiffusionTransformerLayer`` (module names as
    walked by the reference at ``atom_conditioning.py:29-35``)."""

    def __init__(self, heads, dim=384, dim_single_cond=None):
        super().__init__()
        dim_single_cond = dim if dim_single_cond is None else dim_single_cond
        self.adaln = AdaLN(dim, dim_single_cond)
        self.pair_bias_attn = AttentionPairBias(c_s=dim, num_heads=heads, compute_pair_bias=False)
        self.output_projection_linear = nn.Linear(dim_single_cond, dim)
        nn.init.zeros_(self.output_projection_linear.weight)
        nn.init.constant_(self.output_projection_linear.bias, -2.0)
        self.output_projection = nn.Sequential(self.output_projection_linear, nn.Sigmoid())
        self.transition = ConditionedTransitionBlock(dim, dim_single_cond)
        self.post_lnorm = nn.Identity()

    def forward(self, a, s, bias=None, mask=None, to_keys=None, multiplicity=1):
        b = self.adaln(a, s)
        k_in = b
        if to_keys is not None:
            k_in = to_keys(b)
            mask = to_keys(mask.unsqueeze(-1)).squeeze(-1)
        b = self.pair_bias_attn(s=b, z=bias, mask=mask, multiplicity=multiplicity, k_in=k_in)
        b = self.output_projection(s) * b
        a = a + b
        a = a + self.transition(a, s)
        return self.post_lnorm(a)


# --------------------------------------------------------------------------
# Helpers used by the tests and the CPU baseline
# --------------------------------------------------------------------------


def randomize(module: nn.Module, std: float = 0.08, generator=None):
    """Weight convention of the reference tests: every parameter N(0, std),
    norm weights N(1, std) (``tests/test_operator_additions.py:43-47``)."""
    with torch.no_grad():
        for name, p in module.named_parameters():
            mean = 1.0 if "norm" in name and name.endswith("weight") else 0.0
            p.copy_(torch.randn(p.shape, generator=generator) * std + mean)
    return module


# --------------------------------------------------------------------------
# Diffusion transformer stacks (the score model's stacks at configs[4])
# --------------------------------------------------------------------------


class DiffusionTransformer(nn.Module):
    """Upstream ``transformersv2.DiffusionTransformer``: ``depth``
    DiffusionTransformerLayers; the pair bias ``[B, N, M, depth * heads]`` is
    split into per-layer ``[B, N, M, heads]`` slices, layer ``i`` taking
    channels ``i * heads .. (i + 1) * heads - 1`` (the layout
    ``prepare_token_bias`` packs densely, reference ``pair_bias.py:6-13``)."""

    def __init__(self, depth, heads, dim=384, dim_single_cond=None):
        super().__init__()
        self.heads = heads
        self.layers = nn.ModuleList([DiffusionTransformerLayer(heads, dim, dim_single_cond) for _ in range(depth)])

    def forward(self, a, s, bias=None, mask=None, to_keys=None, multiplicity=1):
        b, n, m, d = bias.shape
        bias = bias.view(b, n, m, len(self.layers), d // len(self.layers))
        for i, layer in enumerate(self.layers):
            a = layer(a, s, bias[:, :, :, i], mask, to_keys, multiplicity)
        return a


def get_indexing_matrix(k_windows, w, h, device=None):
    """Upstream ``encodersv2.get_indexing_matrix``: the one-hot [2K, (H / (W/2)) K]
    map from half-windows of W/2 atoms to the key windows of H atoms, key
    window k covering half-windows 2k - h/2 + 1 .. 2k + h/2 (h = H / (W/2)),
    with half-windows outside the sequence left out (zero keys)."""
    assert w % 2 == 0 and h % (w // 2) == 0
    hh = h // (w // 2)
    assert hh % 2 == 0
    ar = torch.arange(2 * k_windows, device=device)
    index = ((ar.unsqueeze(0) - ar.unsqueeze(1)) + hh // 2).clamp(min=0, max=hh + 1)
    index = index.view(k_windows, 2, 2 * k_windows)[:, 0, :]
    onehot = F.one_hot(index, num_classes=hh + 2)[..., 1:-1].transpose(1, 0)
    return onehot.reshape(2 * k_windows, hh * k_windows).float()


def single_to_keys(single, indexing_matrix, w, h):
    """Upstream ``encodersv2.single_to_keys``: [B, N, D] atom rows to
    [B, N / W, H, D] key windows through the indexing matrix."""
    b, n, d = single.shape
    k_windows = n // w
    single = single.view(b, 2 * k_windows, w // 2, d)
    return torch.einsum("bjid,jk->bkid", single, indexing_matrix.to(single.dtype)).reshape(b, k_windows, h, d)


class AtomTransformer(nn.Module):
    """Upstream ``transformersv2.AtomTransformer`` (windowed, eval): atoms in
    windows of ``attn_window_queries`` (32) attend to the ``attn_window_keys``
    (128) atoms ``to_keys`` gathers around them.  The per-window pair bias
    ``[B, N / W, W, H, depth * heads]`` is repeated per sample
    (``multiplicity``) and the stack runs with multiplicity 1 on
    ``[B * mult * N / W, W, D]``.  The reference walks these layers at
    ``atom_conditioning.py:27-35``."""

    def __init__(self, attn_window_queries=32, attn_window_keys=128, depth=3, heads=4, dim=128,
                 dim_single_cond=None):
        super().__init__()
        self.attn_window_queries = attn_window_queries
        self.attn_window_keys = attn_window_keys
        self.diffusion_transformer = DiffusionTransformer(depth, heads, dim, dim_single_cond)

    def forward(self, q, c, bias, to_keys, mask, multiplicity=1):
        w, h = self.attn_window_queries, self.attn_window_keys
        b, n, d = q.shape
        nw = n // w
        q = q.view(b * nw, w, -1)
        c = c.view(b * nw, w, -1)
        mask = mask.view(b * nw, w)
        bias = bias.repeat_interleave(multiplicity, 0)
        bias = bias.view(bias.shape[0] * nw, w, h, -1)

        def window_keys(x):
            return to_keys(x.view(b, nw * w, -1)).view(b * nw, h, -1)

        q = self.diffusion_transformer(a=q, s=c, bias=bias, mask=mask.float(), multiplicity=1, to_keys=window_keys)
        return q.view(b, nw * w, d)


class DiffusionStacks(nn.Module):
    """The three transformer stacks of Boltz-2's score model at their module
    paths (``atom_attention_encoder.atom_encoder``, ``token_transformer``,
    ``atom_attention_decoder.atom_decoder``: atom
    encoder / decoder 3 blocks x 4 heads at 128 channels with 32 / 128
    windows, token transformer 24 blocks x 16 heads at 768).  One denoiser
    step here embeds the noisy coordinates r (EDM input scaling
    1 / sqrt(sigma^2 + sigma_data^2), sigma_data 16, then a 3 -> 128 linear
    added to the atom queries), runs the atom encoder on the atom queries,
    the token transformer on the token activations and the atom decoder on
    the encoder's output, and maps the decoder's atoms to a coordinate
    update (LayerNorm + 128 -> 3 linear).  Those two small linears stand in
    for upstream's coordinate embedding and update head; the atom <-> token
    aggregation linears between the stacks are outside the hot path and
    left out."""

    def __init__(self, token_depth=24, token_heads=16, token_dim=768, atom_depth=3, atom_heads=4, atom_dim=128,
                 window_queries=32, window_keys=128):
        super().__init__()
        self.atom_attention_encoder = nn.Module()
        self.atom_attention_encoder.atom_encoder = AtomTransformer(window_queries, window_keys, atom_depth,
                                                                   atom_heads, atom_dim, atom_dim)
        self.token_transformer = DiffusionTransformer(token_depth, token_heads, token_dim, token_dim)
        self.atom_attention_decoder = nn.Module()
        self.atom_attention_decoder.atom_decoder = AtomTransformer(window_queries, window_keys, atom_depth,
                                                                   atom_heads, atom_dim, atom_dim)
        self.r_to_q = nn.Linear(3, atom_dim, bias=False)
        self.pos_update = nn.Sequential(nn.LayerNorm(atom_dim), nn.Linear(atom_dim, 3, bias=False))

    def forward(self, r, q, c, atom_mask, enc_bias, dec_bias, to_keys, a, s, token_bias, token_mask,
                multiplicity=1, sigma=160.0, sigma_data=16.0):
        q = q + self.r_to_q(r / math.sqrt(sigma ** 2 + sigma_data ** 2))
        q = self.atom_attention_encoder.atom_encoder(q, c, enc_bias, to_keys, atom_mask, multiplicity)
        a = self.token_transformer(a, s, token_bias, token_mask, multiplicity=multiplicity)
        q = self.atom_attention_decoder.atom_decoder(q, c, dec_bias, to_keys, atom_mask, multiplicity)
        return self.pos_update(q), q, a
