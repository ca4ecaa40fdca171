"""Boltz-compatible modules whose forward runs the gfx950 kernels.

Class names, parameter names and shapes follow upstream Boltz 2.2.1 (the
modules lauritsf/boltz-lumi patches, adapters.py:24-46), so a Boltz
``state_dict`` loads into them unchanged and vice versa.  The pair-path
forwards call libbmx directly and raise when it is missing or the tensors are
not on a GPU; there is no CPU path.

``PairformerLayer`` composes the pair stack with the fused kernels writing the
fp32 residual stream in place (no separate ``z + out`` pass), then runs the
sequence stack (AttentionPairBias + Transition(384)), which upstream keeps in
fp32 outside the pair hot path, with PyTorch on the GPU.
"""

from __future__ import annotations

import math

import torch
from torch import nn
import torch.nn.functional as F

from . import ops, pairformer
from .pair_bias import fused_attention


def _require_cuda(x: torch.Tensor, what: str) -> None:
    if not x.is_cuda:
        raise RuntimeError(f"{what}: the gfx950 path needs a GPU tensor (got {x.device})")


def _batch_out(x, out, out_mode):
    """The module output for a batch: ``out`` when given (accumulate mode
    needs it), else one tensor of x's shape that each batch element's kernel
    writes its slice of (no stacking copy)."""
    if out is not None or out_mode == ops.OUT_ACCUMULATE:
        return out
    dtype = torch.bfloat16 if out_mode == ops.OUT_BF16 else torch.float32
    return torch.empty(x.shape, device=x.device, dtype=dtype)


class LayerNorm(nn.Module):
    """Triangle-attention LayerNorm (upstream ``primitives.LayerNorm``; ``c_in`` is a tuple)."""

    def __init__(self, c_in: int, eps: float = 1e-5):
        super().__init__()
        self.c_in = (c_in,)
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(c_in))
        self.bias = nn.Parameter(torch.zeros(c_in))

    def forward(self, x):
        return F.layer_norm(x, self.c_in, self.weight.to(x.dtype), self.bias.to(x.dtype), self.eps)


class Attention(nn.Module):
    """Parameter container of upstream ``primitives.Attention`` (gated)."""

    def __init__(self, c_q, c_k, c_v, c_hidden, no_heads):
        super().__init__()
        self.c_q, self.c_k, self.c_v = c_q, c_k, c_v
        self.c_hidden, self.no_heads = c_hidden, no_heads
        self.linear_q = nn.Linear(c_q, c_hidden * no_heads, bias=False)
        self.linear_k = nn.Linear(c_k, c_hidden * no_heads, bias=False)
        self.linear_v = nn.Linear(c_v, c_hidden * no_heads, bias=False)
        self.linear_o = nn.Linear(c_hidden * no_heads, c_q)
        self.linear_g = nn.Linear(c_q, c_hidden * no_heads)


class TriangleAttention(nn.Module):
    """Triangle attention around the starting (or ending) node, fused on gfx950."""

    def __init__(self, c_in=128, c_hidden=32, no_heads=4, starting=True, inf=1e9):
        super().__init__()
        if (c_in, c_hidden, no_heads) != (128, 32, 4):
            raise ValueError("the fused kernel is built for c_in=128, 4 heads x 32")
        self.c_in, self.c_hidden, self.no_heads = c_in, c_hidden, no_heads
        self.starting, self.inf = starting, inf
        self.layer_norm = LayerNorm(c_in)
        self.linear = nn.Linear(c_in, no_heads, bias=False)
        self.mha = Attention(c_in, c_in, c_in, c_hidden, no_heads)

    def forward(self, x, mask=None, chunk_size=None, use_kernels=False, out_mode=ops.OUT_BF16, out=None,
                workspace=None):
        _require_cuda(x, type(self).__name__)
        out = _batch_out(x, out, out_mode)
        for b in range(x.shape[0]):
            mb = None if mask is None else mask[b].float().contiguous()
            ops.triattn(self, x[b].contiguous(), mb, self.starting, out_mode, None if out is None else out[b],
                        workspace)
        return out


class TriangleAttentionEndingNode(TriangleAttention):
    def __init__(self, c_in=128, c_hidden=32, no_heads=4, inf=1e9):
        super().__init__(c_in, c_hidden, no_heads, starting=False, inf=inf)


TriangleAttentionStartingNode = TriangleAttention


class _TriangleMultiplication(nn.Module):
    outgoing = True

    def __init__(self, dim: int = 128):
        super().__init__()
        if dim != 128:
            raise ValueError("the fused kernel is built for 128 pair channels")
        self.norm_in = nn.LayerNorm(dim, eps=1e-5)
        self.p_in = nn.Linear(dim, 2 * dim, bias=False)
        self.g_in = nn.Linear(dim, 2 * dim, bias=False)
        self.norm_out = nn.LayerNorm(dim)
        self.p_out = nn.Linear(dim, dim, bias=False)
        self.g_out = nn.Linear(dim, dim, bias=False)

    def forward(self, x, mask, use_kernels=False, out_mode=ops.OUT_BF16, out=None, workspace=None):
        _require_cuda(x, type(self).__name__)
        out = _batch_out(x, out, out_mode)
        for b in range(x.shape[0]):
            ops.trimul(self, x[b].float().contiguous(), mask[b].float().contiguous(), self.outgoing, out_mode,
                       None if out is None else out[b], workspace)
        return out


class TriangleMultiplicationOutgoing(_TriangleMultiplication):
    outgoing = True


class TriangleMultiplicationIncoming(_TriangleMultiplication):
    outgoing = False


class Transition(nn.Module):
    """Upstream ``Transition``; the 128 -> 512 -> 128 pair instance is fused,
    other sizes (the sequence stack's 384 -> 1536) run the upstream math."""

    def __init__(self, dim: int = 128, hidden: int = 512, out_dim=None):
        super().__init__()
        out_dim = dim if out_dim is None else out_dim
        self.norm = nn.LayerNorm(dim, eps=1e-5)
        self.fc1 = nn.Linear(dim, hidden, bias=False)
        self.fc2 = nn.Linear(dim, hidden, bias=False)
        self.fc3 = nn.Linear(hidden, out_dim, bias=False)
        self.silu = nn.SiLU()
        self.hidden = hidden
        self.fused = (dim, hidden, out_dim) == (128, 512, 128)

    def forward(self, x, chunk_size=None, out_mode=ops.OUT_BF16, out=None):
        if self.fused:
            _require_cuda(x, "Transition")
            return ops.pair_transition(self, x.contiguous(), out_mode, out)
        x = self.norm(x)
        return self.fc3(self.silu(self.fc1(x)) * self.fc2(x))

    def residual(self, x, inplace=False):
        """``x + self(x)`` for the unfused sizes: fc1 | fc2 as one GEMM and the
        residual add in the fc3 GEMM's epilogue (fp32 x; written into x when
        ``inplace`` and x is contiguous)."""
        if self.fused:
            return x + self(x)
        return pairformer.transition_residual(self, x, inplace)


class _HeadsFirst(nn.Module):
    """``Rearrange("b ... h -> b h ...")`` of upstream proj_z (parameter-free)."""

    def forward(self, x):
        return x.movedim(-1, 1)


class AttentionPairBias(nn.Module):
    """Upstream ``attentionv2.AttentionPairBias`` (sequence stack, fp32)."""

    def __init__(self, c_s, c_z=None, num_heads=None, inf=1e6, compute_pair_bias=True):
        super().__init__()
        self.c_s, self.num_heads = c_s, num_heads
        self.head_dim = c_s // num_heads
        self.inf = inf
        self.proj_q = nn.Linear(c_s, c_s)
        self.proj_k = nn.Linear(c_s, c_s, bias=False)
        self.proj_v = nn.Linear(c_s, c_s, bias=False)
        self.proj_g = nn.Linear(c_s, c_s, bias=False)
        self.compute_pair_bias = compute_pair_bias
        if compute_pair_bias:
            self.proj_z = nn.Sequential(nn.LayerNorm(c_z), nn.Linear(c_z, num_heads, bias=False), _HeadsFirst())
        else:
            self.proj_z = _HeadsFirst()
        self.proj_o = nn.Linear(c_s, c_s, bias=False)

    def pair_bias(self, z):
        """[B, N, N, c_z] -> [B, H, N, N]; the 128 -> 16 projection of the trunk
        runs as one fused gfx950 kernel (LN + fp32 MFMA, head-major output)."""
        if not self.compute_pair_bias:
            return z.movedim(-1, 1)
        norm, lin = self.proj_z[0], self.proj_z[1]
        if z.is_cuda and z.shape[-1] == 128 and lin.weight.shape[0] == 16 and z.shape[1] == z.shape[2]:
            out = torch.empty((z.shape[0], 16, z.shape[1], z.shape[2]), device=z.device, dtype=torch.float32)
            for b in range(z.shape[0]):
                ops.pair_bias(norm, lin, z[b].contiguous(), out=out[b])
            return out
        return self.proj_z(z)

    def fused_bias_ok(self, z):
        """Whether ``pair_bias(z)`` is the fused 128 -> 16 kernel's (so a
        producer of z may compute it in its own epilogue instead)."""
        return (self.compute_pair_bias and z.is_cuda and z.shape[-1] == 128 and z.shape[1] == z.shape[2]
                and self.proj_z[1].weight.shape == (16, 128))

    def attend(self, s, z, mask, k_in, multiplicity=1, bias=None):
        """``g * attention`` before ``proj_o`` from the fused kernel
        (``pair_bias.fused_attention``), or None where it does not apply.
        ``bias``, when given, is ``pair_bias(z)`` computed already."""
        if (bias is None and s.is_cuda and self.head_dim in (24, 48) and not torch.is_grad_enabled()
                and not self.training):
            bias = self.pair_bias(z)
        return fused_attention(self, s, z, mask, k_in, multiplicity, bias)

    def forward(self, s, z, mask, k_in, multiplicity=1):
        o = self.attend(s, z, mask, k_in, multiplicity)
        if o is not None:
            return self.proj_o(o) if torch.is_autocast_enabled() else ops.linear_fp32(o, self.proj_o)
        b = s.shape[0]
        q = self.proj_q(s).view(b, -1, self.num_heads, self.head_dim).transpose(1, 2)
        k = self.proj_k(k_in).view(b, -1, self.num_heads, self.head_dim).transpose(1, 2)
        v = self.proj_v(k_in).view(b, -1, self.num_heads, self.head_dim).transpose(1, 2)
        bias = self.pair_bias(z).float()
        if multiplicity != 1:
            bias = bias.repeat_interleave(multiplicity, 0)
        g = torch.sigmoid(self.proj_g(s))
        logits = (q.float() @ k.float().transpose(-1, -2)) / math.sqrt(self.head_dim) + bias
        logits = logits + (1 - mask[:, None, None].float()) * -self.inf
        o = (torch.softmax(logits, -1) @ v.float()).to(v.dtype)
        o = o.transpose(1, 2).reshape(b, -1, self.c_s)
        return self.proj_o(g * o)


class PairformerLayer(nn.Module):
    """Boltz-2 ``PairformerLayer`` (v2, eval) with the fused pair stack."""

    def __init__(self, token_s=384, token_z=128, num_heads=16, dropout=0.25, pairwise_head_width=32,
                 pairwise_num_heads=4, post_layer_norm=False):
        super().__init__()
        self.token_z = token_z
        self.num_heads = num_heads
        self.dropout = dropout  # upstream's rate; this module's own forward runs eval only (no masks)
        self.pre_norm_s = nn.LayerNorm(token_s)
        self.attention = AttentionPairBias(token_s, token_z, num_heads)
        self.tri_mul_out = TriangleMultiplicationOutgoing(token_z)
        self.tri_mul_in = TriangleMultiplicationIncoming(token_z)
        self.tri_att_start = TriangleAttention(token_z, pairwise_head_width, pairwise_num_heads, inf=1e9)
        self.tri_att_end = TriangleAttentionEndingNode(token_z, pairwise_head_width, pairwise_num_heads, inf=1e9)
        self.transition_s = Transition(token_s, token_s * 4)
        self.transition_z = Transition(token_z, token_z * 4)
        self.s_post_norm = nn.LayerNorm(token_s) if post_layer_norm else nn.Identity()

    def pair_stack(self, z, pair_mask, z_out=None, workspace=None, bias_out=None):
        """z_out = z + tri_mul_out + tri_mul_in + tri_att_start + tri_att_end + transition_z,
        each added in order into the fp32 stream (``pairformer.pair_stack``; no
        dropout masks).  z is read once and never written; z_out may be
        preallocated.  With ``bias_out`` [B, 16, N, N] the transition's
        epilogue also writes the sequence stack's pair bias of z_out
        (``attention.pair_bias(z_out)``)."""
        _require_cuda(z, "PairformerLayer")
        mods = None if bias_out is None else (self.attention.proj_z[0], self.attention.proj_z[1])
        return pairformer.pair_stack(self, z, pair_mask, z_out, workspace, bias_out, mods)

    def sequence_stack(self, s, z, mask, pair_bias=None):
        """s + attention, then + transition_s (upstream order, fp32); on the
        fused path each residual add rides in the epilogue of its output GEMM
        (``pairformer.sequence_stack``).  ``pair_bias``:
        ``attention.pair_bias(z)`` if already computed."""
        return pairformer.sequence_stack(self, s, z, mask, pair_bias)

    def forward(self, s, z, mask, pair_mask, chunk_size_tri_attn=None, use_kernels=False, z_out=None,
                workspace=None):
        bias = None
        if self.attention.fused_bias_ok(z) and not torch.is_grad_enabled():
            bias = torch.empty((z.shape[0], 16, z.shape[1], z.shape[2]), device=z.device, dtype=torch.float32)
        z = self.pair_stack(z, pair_mask, z_out, workspace, bias_out=bias)
        return self.sequence_stack(s, z, mask, pair_bias=bias), z


class PairformerModule(nn.Module):
    """A trunk of ``num_blocks`` Pairformer layers sharing one workspace and
    ping-ponging two pair buffers."""

    def __init__(self, token_s=384, token_z=128, num_blocks=64, num_heads=16, pairwise_head_width=32,
                 pairwise_num_heads=4, post_layer_norm=False):
        super().__init__()
        self.token_z = token_z
        self.layers = nn.ModuleList([
            PairformerLayer(token_s, token_z, num_heads, 0.25, pairwise_head_width, pairwise_num_heads,
                            post_layer_norm)
            for _ in range(num_blocks)])

    def forward(self, s, z, mask, pair_mask, use_kernels=False):
        ws = ops.new_workspace(z.shape[1], z.device)
        bufs = [torch.empty_like(z, dtype=torch.float32), torch.empty_like(z, dtype=torch.float32)]
        for idx, layer in enumerate(self.layers):
            s, z = layer(s, z, mask, pair_mask, z_out=bufs[idx % 2], workspace=ws)
        return s, z


# ------------------------------------------------------ diffusion blocks


class AdaLN(nn.Module):
    """Upstream ``transformersv2.AdaLN`` with the LN + modulation fused."""

    def __init__(self, dim, dim_single_cond):
        super().__init__()
        self.a_norm = nn.LayerNorm(dim, elementwise_affine=False, bias=False)
        self.s_norm = nn.LayerNorm(dim_single_cond, bias=False)
        self.s_scale = nn.Linear(dim_single_cond, dim)
        self.s_bias = nn.Linear(dim_single_cond, dim, bias=False)

    def forward(self, a, s):
        _require_cuda(a, "AdaLN")
        sn = ops.layer_norm(s.contiguous(), self.s_norm.weight, None, self.s_norm.eps)
        scale, shift = ops.linear_fp32(sn, self.s_scale), ops.linear_fp32(sn, self.s_bias)
        return ops.adaln_modulate(a.contiguous(), scale.contiguous(), shift.contiguous(), self.a_norm.eps)


class SwiGLU(nn.Module):
    def forward(self, x):
        x, gates = x.chunk(2, dim=-1)
        return F.silu(gates) * x


class ConditionedTransitionBlock(nn.Module):
    """Upstream ``transformersv2.ConditionedTransitionBlock`` with fused epilogues."""

    def __init__(self, dim_single, dim_single_cond, expansion_factor=2):
        super().__init__()
        self.adaln = AdaLN(dim_single, dim_single_cond)
        dim_inner = int(dim_single * expansion_factor)
        self.swish_gate = nn.Sequential(nn.Linear(dim_single, dim_inner * 2, bias=False), SwiGLU())
        self.a_to_b = nn.Linear(dim_single, dim_inner, bias=False)
        self.b_to_a = nn.Linear(dim_inner, dim_single, bias=False)
        self.output_projection = nn.Sequential(nn.Linear(dim_single_cond, dim_single), nn.Sigmoid())

    def forward(self, a, s):
        a = self.adaln(a, s)
        u, v = ops.linear_fp32(a, self.swish_gate[0]), ops.linear_fp32(a, self.a_to_b)
        b = ops.epilogue(u.contiguous(), v.contiguous(), None, ops.GATED_SWIGLU)
        g, y = ops.linear_fp32(s, self.output_projection[0]), ops.linear_fp32(b, self.b_to_a)
        return ops.epilogue(g.contiguous(), y.contiguous(), None, ops.GATE)
