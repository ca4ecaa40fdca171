"""Pin the CPU oracle (oracle/boltz_ref.py) before trusting it.

The reference ships no golden vectors (its tests run live upstream Boltz on a
gfx90a GPU), so every oracle function is pinned here by something other than
a retyped formula:

* fp64 explicit-loop evaluation (oracle/brute.py) at tiny sizes;
* the reference's own operand layouts / recipes restated independently
  (permute + bmm of ``multiplication.py:105-122``; the softmax test recipe of
  ``tests/test_triangle_softmax.py:38-47``; the epilogue formulas of
  ``kernels/diffusion_hip.cu:14-27``);
* closed forms and invariants that a dropped term, a wrong sign/index or a
  transposed operand would break.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import boltz_ref as R
from oracle import brute as B


def _gen(seed):
    g = torch.Generator().manual_seed(seed)
    return g


def _rel(a, b):
    a, b = torch.as_tensor(a).double(), torch.as_tensor(b).double()
    return ((a - b).abs().max() / b.abs().max().clamp_min(1e-30)).item()


# ---------------------------------------------------------------- LayerNorm


def test_layernorm_matches_textbook_and_loops():
    g = _gen(1)
    ln = R.randomize(R.LayerNorm(16), generator=g)
    x = torch.randn(5, 16, generator=g) * 3 + 1
    y = ln(x)
    assert torch.allclose(y, F.layer_norm(x, (16,), ln.weight, ln.bias, 1e-5), atol=1e-6)
    loops = np.array([B.layer_norm_vec(list(r), ln.weight.detach().double().numpy(),
                                       ln.bias.detach().double().numpy()) for r in x.double().numpy()])
    assert _rel(y.detach(), loops) < 1e-5
    # invariants: output has (weighted) zero mean / unit variance before the affine
    plain = F.layer_norm(x, (16,))
    assert plain.mean(-1).abs().max() < 1e-5
    assert (plain.var(-1, unbiased=False) - 1).abs().max() < 1e-3


# ---------------------------------------------------- triangle multiplication


@pytest.mark.parametrize("outgoing", [True, False])
@pytest.mark.parametrize("mask_kind", ["ones", "partial", "fractional", "zero"])
def test_trimul_matches_fp64_loops(outgoing, mask_kind):
    g = _gen(2)
    cls = R.TriangleMultiplicationOutgoing if outgoing else R.TriangleMultiplicationIncoming
    m = R.randomize(cls(8), generator=g).double()
    n = 5
    x = torch.randn(1, n, n, 8, generator=g, dtype=torch.float64)
    mask = torch.ones(1, n, n, dtype=torch.float64)
    if mask_kind == "partial":
        mask[:, -2:, :] = 0
    elif mask_kind == "fractional":
        mask = torch.rand(1, n, n, generator=g, dtype=torch.float64)
    elif mask_kind == "zero":
        mask.zero_()
    with torch.no_grad():
        y = m(x, mask)[0]
    ref = B.triangle_multiplication(m, x[0].numpy(), mask[0].numpy(), outgoing)
    assert _rel(y, ref) < 1e-10


@pytest.mark.parametrize("outgoing", [True, False])
def test_trimul_matches_reference_bmm_layout(outgoing):
    """Restate the reference's channel-major bmm (multiplication.py:105-122):
    outgoing: left=a.permute(0,3,1,2), right=b.permute(0,3,2,1);
    incoming: left=a.permute(0,3,2,1), right=b.permute(0,3,1,2)."""
    g = _gen(3)
    cls = R.TriangleMultiplicationOutgoing if outgoing else R.TriangleMultiplicationIncoming
    m = R.randomize(cls(16), generator=g)
    n = 9
    x = torch.randn(1, n, n, 16, generator=g)
    mask = (torch.rand(1, n, n, generator=g) > 0.2).float()
    with torch.no_grad():
        xn = m.norm_in(x)
        h = m.p_in(xn) * torch.sigmoid(m.g_in(xn)) * mask[..., None]
        a, b = h[..., :16], h[..., 16:]
        if outgoing:
            left, right = a.permute(0, 3, 1, 2), b.permute(0, 3, 2, 1)
        else:
            left, right = a.permute(0, 3, 2, 1), b.permute(0, 3, 1, 2)
        prod = torch.bmm(left.reshape(16, n, n), right.reshape(16, n, n))
        o = prod.reshape(1, 16, n, n).permute(0, 2, 3, 1)
        want = m.p_out(m.norm_out(o)) * torch.sigmoid(m.g_out(xn))
        got = m(x, mask)
    assert _rel(got, want) < 1e-5


def test_trimul_incoming_is_transposed_outgoing_with_swapped_halves():
    g = _gen(4)
    inc = R.randomize(R.TriangleMultiplicationIncoming(16), generator=g)
    out = R.TriangleMultiplicationOutgoing(16)
    sd = {k: v.clone() for k, v in inc.state_dict().items()}
    for name in ("p_in.weight", "g_in.weight"):
        w = sd[name]
        sd[name] = torch.cat([w[16:], w[:16]], 0)
    out.load_state_dict(sd)
    n = 7
    x = torch.randn(1, n, n, 16, generator=g)
    mask = (torch.rand(1, n, n, generator=g) > 0.3).float()
    with torch.no_grad():
        a = inc(x, mask)
        b = out(x.transpose(1, 2), mask.transpose(1, 2)).transpose(1, 2)
    assert _rel(a, b) < 1e-5
    # and the two directions really differ (catches a swapped einsum)
    with torch.no_grad():
        out.load_state_dict(inc.state_dict())
        assert _rel(out(x, mask), inc(x, mask)) > 1e-2


def test_trimul_zero_mask_closed_form():
    g = _gen(5)
    m = R.randomize(R.TriangleMultiplicationOutgoing(16), generator=g)
    x = torch.randn(1, 6, 6, 16, generator=g)
    with torch.no_grad():
        y = m(x, torch.zeros(1, 6, 6))
        # o == 0 -> norm_out(0) == norm_out.bias
        want = m.p_out(m.norm_out.bias.expand(1, 6, 6, 16)) * torch.sigmoid(m.g_out(m.norm_in(x)))
    assert _rel(y, want) < 1e-5


@pytest.mark.parametrize("cls", [R.TriangleMultiplicationOutgoing, R.TriangleMultiplicationIncoming,
                                 R.TriangleAttention, R.TriangleAttentionEndingNode])
def test_pair_ops_permutation_equivariant(cls):
    g = _gen(6)
    m = cls(16) if "Multiplication" in cls.__name__ else cls(16, 4, 2)
    R.randomize(m, generator=g)
    n = 8
    x = torch.randn(1, n, n, 16, generator=g)
    mask = (torch.rand(1, n, n, generator=g) > 0.25).float()
    perm = torch.randperm(n, generator=g)
    with torch.no_grad():
        y = m(x, mask)
        yp = m(x[:, perm][:, :, perm], mask[:, perm][:, :, perm])
    assert _rel(yp, y[:, perm][:, :, perm]) < 1e-5


# ------------------------------------------------------- triangle attention


@pytest.mark.parametrize("starting", [True, False])
def test_triattn_matches_fp64_loops(starting):
    g = _gen(7)
    cls = R.TriangleAttention if starting else R.TriangleAttentionEndingNode
    m = R.randomize(cls(8, 4, 2), generator=g).double()
    n = 5
    x = torch.randn(1, n, n, 8, generator=g, dtype=torch.float64)
    mask = torch.ones(1, n, n, dtype=torch.float64)
    mask[:, -1, :] = 0
    mask[:, :, -2] = 0
    with torch.no_grad():
        y = m(x, mask)[0]
    ref = B.triangle_attention(m, x[0].numpy(), mask[0].numpy(), starting)
    assert _rel(y, ref) < 1e-10


def test_triattn_softmax_recipe_of_reference_test():
    """tests/test_triangle_softmax.py:38-47: ``s += mask; s += bias; softmax``
    with mask [B,I,1,1,K], bias [B,1,H,Q,K]; Attention must apply exactly that."""
    g = _gen(8)
    att = R.randomize(R.Attention(8, 8, 8, 4, 2), generator=g)
    x = torch.randn(1, 3, 6, 8, generator=g)
    mask_bias = torch.zeros(1, 3, 1, 1, 6)
    mask_bias[..., -2:] = -1e9
    tri_bias = torch.randn(1, 1, 2, 6, 6, generator=g) * 2
    with torch.no_grad():
        q, k, v = att._prep_qkv(x, x)
        s = q @ k.transpose(-1, -2)
        s += mask_bias
        s += tri_bias
        p = torch.softmax(s, -1)
        want = att._wrap_up((p @ v).transpose(-2, -3), x)
        got = att(x, x, tri_bias, mask_bias)
    assert _rel(got, want) < 1e-6
    assert torch.allclose(p[..., -2:], torch.zeros(())), "masked keys get zero weight"


def test_triattn_fully_masked_row_is_uniform():
    """A row whose mask is all zero gets -1e9 on every key: the softmax is
    uniform, so each query sees the mean of V (not zero, not NaN)."""
    g = _gen(9)
    m = R.randomize(R.TriangleAttention(16, 8, 2), generator=g)
    n = 6
    x = torch.randn(1, n, n, 16, generator=g) * 0.3
    mask = torch.ones(1, n, n)
    mask[:, 2, :] = 0
    with torch.no_grad():
        y = m(x, mask)
        xn = m.layer_norm(x)
        q, k, v = m.mha._prep_qkv(xn, xn)  # [1, I, H, J, d]
        mean_v = v[0, 2].mean(dim=-2, keepdim=True).expand(2, n, 8)  # [H, J, d]
        want = m.mha._wrap_up(mean_v.transpose(0, 1)[None], xn[:, 2])
    assert torch.isfinite(y).all()
    assert _rel(y[:, 2], want) < 1e-5


def test_triattn_single_token_closed_form():
    """N=1: softmax over one key is 1, so o = v (no scale, no bias effect)."""
    g = _gen(10)
    m = R.randomize(R.TriangleAttention(16, 8, 2), generator=g)
    x = torch.randn(1, 1, 1, 16, generator=g)
    with torch.no_grad():
        xn = m.layer_norm(x)
        v = m.mha.linear_v(xn).view(1, 1, 1, 2, 8)
        want = m.mha._wrap_up(v, xn)
        assert _rel(m(x), want) < 1e-6


def test_triattn_ending_is_transposed_starting():
    g = _gen(11)
    st = R.randomize(R.TriangleAttention(16, 8, 2), generator=g)
    en = R.TriangleAttentionEndingNode(16, 8, 2)
    en.load_state_dict(st.state_dict())
    x = torch.randn(1, 7, 7, 16, generator=g)
    mask = (torch.rand(1, 7, 7, generator=g) > 0.2).float()
    with torch.no_grad():
        a = en(x, mask)
        b = st(x.transpose(1, 2), mask.transpose(1, 2)).transpose(1, 2)
        assert _rel(a, b) < 1e-6
        assert _rel(a, st(x, mask)) > 1e-2


def test_triattn_chunking_does_not_change_math():
    g = _gen(12)
    m = R.randomize(R.TriangleAttentionEndingNode(16, 8, 2), generator=g)
    x = torch.randn(1, 9, 9, 16, generator=g)
    mask = (torch.rand(1, 9, 9, generator=g) > 0.2).float()
    with torch.no_grad():
        assert _rel(m(x, mask, chunk_size=4), m(x, mask)) < 1e-6


@pytest.mark.parametrize("starting", [True, False])
def test_triattn_rows_are_rows_of_the_full_forward(starting):
    """``forward_rows`` (the large-size checker) against the full forward,
    in fp64, with masked rows among the selected ones."""
    g = _gen(14)
    m = R.randomize(R.TriangleAttention(16, 8, 2, starting=starting), generator=g).double()
    n = 13
    x = torch.randn(1, n, n, 16, generator=g, dtype=torch.float64)
    tok = torch.ones(n, dtype=torch.float64)
    tok[[2, 11]] = 0
    mask = (tok[:, None] * tok[None, :])[None]
    mask[0, 4, 6] = 0  # asymmetric
    rows = [0, 2, 7, 12]
    with torch.no_grad():
        full = m(x, mask)
        part = m.forward_rows(x, mask, rows, chunk=5)  # ragged last chunk
    want = full[:, rows] if starting else full[:, :, rows]
    assert part.shape == want.shape
    assert _rel(part, want) < 1e-13


@pytest.mark.parametrize("outgoing", [True, False])
def test_trimul_rows_are_rows_of_the_full_forward(outgoing):
    """``forward_rows`` sums over k in chunks (here 4 tokens, the last one
    ragged) with each chunk's operands computed separately; fp64 against
    the full forward."""
    g = _gen(15)
    cls = R.TriangleMultiplicationOutgoing if outgoing else R.TriangleMultiplicationIncoming
    m = R.randomize(cls(16), generator=g).double()
    n = 11
    x = torch.randn(1, n, n, 16, generator=g, dtype=torch.float64)
    mask = (torch.rand(1, n, n, generator=g) > 0.25).double()
    rows = [1, 5, 10]
    with torch.no_grad():
        want = m(x, mask)[:, rows]
        part = m.forward_rows(x, mask, rows, chunk=4)
    assert part.shape == want.shape
    assert _rel(part, want) < 1e-13


# ---------------------------------------------------------------- transition


def test_transition_matches_loops_and_closed_forms():
    g = _gen(13)
    t = R.randomize(R.Transition(8, 32), generator=g).double()
    x = torch.randn(2, 3, 8, generator=g, dtype=torch.float64)
    with torch.no_grad():
        y = t(x)
    assert _rel(y, B.transition(t, x.numpy())) < 1e-10
    with torch.no_grad():
        assert _rel(t(x, chunk_size=8), y) < 1e-10  # upstream chunked branch
        t.fc3.weight.zero_()
        assert t(x).abs().max() == 0


def test_transition_silu_then_multiply():
    """pair_hip.cu:12-17: silu(a) * b, not a * silu(b)."""
    g = _gen(14)
    t = R.randomize(R.Transition(8, 16), generator=g)
    x = torch.randn(4, 8, generator=g)
    with torch.no_grad():
        xn = t.norm(x)
        want = t.fc3(F.silu(t.fc1(xn)) * t.fc2(xn))
        wrong = t.fc3(t.fc1(xn) * F.silu(t.fc2(xn)))
        assert _rel(t(x), want) < 1e-6 and _rel(t(x), wrong) > 1e-3


# ---------------------------------------------------------- diffusion blocks


def test_adaln_matches_loops_and_epilogue_formula():
    g = _gen(15)
    m = R.randomize(R.AdaLN(8, 6), generator=g).double()
    a = torch.randn(2, 5, 8, generator=g, dtype=torch.float64)
    s = torch.randn(2, 5, 6, generator=g, dtype=torch.float64)
    with torch.no_grad():
        y = m(a, s)
        assert _rel(y, B.adaln(m, a.numpy(), s.numpy())) < 1e-10
        # diffusion_hip.cu:15-18: MODULATION(a=a_norm(a), b=s_scale, c=s_bias)
        sn = m.s_norm(s)
        mod = torch.sigmoid(m.s_scale(sn)) * m.a_norm(a) + m.s_bias(sn)
        assert _rel(y, mod) < 1e-12
        # zero scale weight: sigmoid(bias) * a_hat + s_bias(s_hat)
        m.s_scale.weight.zero_()
        want = torch.sigmoid(m.s_scale.bias) * F.layer_norm(a, (8,)) + m.s_bias(sn)
        assert _rel(m(a, s), want) < 1e-12


def test_conditioned_transition_matches_loops_and_swiglu_order():
    g = _gen(16)
    m = R.randomize(R.ConditionedTransitionBlock(8, 6), generator=g).double()
    a = torch.randn(3, 8, generator=g, dtype=torch.float64)
    s = torch.randn(3, 6, generator=g, dtype=torch.float64)
    with torch.no_grad():
        y = m(a, s)
        assert _rel(y, B.conditioned_transition(m, a.numpy(), s.numpy())) < 1e-10
        u = m.swish_gate[0](m.adaln(a, s))
        # diffusion_hip.cu:39-42: silu of the SECOND half times the first half
        assert _rel(m.swish_gate[1](u), F.silu(u[:, 16:]) * u[:, :16]) < 1e-12
        # zero output-projection weight (upstream init): gate = sigmoid(-2)
        m.output_projection[0].weight.zero_()
        m.output_projection[0].bias.fill_(-2.0)
        base = m.b_to_a(m.swish_gate(m.adaln(a, s)) * m.a_to_b(m.adaln(a, s)))
        assert _rel(m(a, s), base * (1 / (1 + math.exp(2.0)))) < 1e-12


# ------------------------------------------------------ attention pair bias


def test_attention_pair_bias_matches_loops():
    g = _gen(17)
    m = R.randomize(R.AttentionPairBias(8, 6, 2), generator=g).double()
    n = 4
    s = torch.randn(1, n, 8, generator=g, dtype=torch.float64)
    z = torch.randn(1, n, n, 6, generator=g, dtype=torch.float64)
    mask = torch.ones(1, n, dtype=torch.float64)
    mask[:, -1] = 0
    with torch.no_grad():
        y = m(s, z, mask, s)
    assert _rel(y, B.attention_pair_bias(m, s.numpy(), z.numpy(), mask.numpy(), s.numpy())) < 1e-10


def test_pairformer_layer_runs_and_is_residual():
    """Composition is parity unpinned; this checks only structure: zero
    final projections leave z and s unchanged (the layer is residual)."""
    g = _gen(18)
    layer = R.randomize(R.PairformerLayer(token_s=32, token_z=16, num_heads=4, pairwise_head_width=8,
                                          pairwise_num_heads=2), generator=g)
    with torch.no_grad():
        for mod in (layer.tri_mul_out.p_out, layer.tri_mul_in.p_out, layer.tri_att_start.mha.linear_o,
                    layer.tri_att_end.mha.linear_o, layer.transition_z.fc3, layer.attention.proj_o,
                    layer.transition_s.fc3):
            mod.weight.zero_()
            if getattr(mod, "bias", None) is not None:
                mod.bias.zero_()
        s = torch.randn(1, 6, 32, generator=g)
        z = torch.randn(1, 6, 6, 16, generator=g)
        mask = torch.ones(1, 6)
        s2, z2 = layer(s, z, mask, mask[:, :, None] * mask[:, None, :])
    assert torch.equal(z2, z) and torch.equal(s2, s)


@pytest.mark.parametrize("token_z", [16, 8])
def test_pairformer_no_seq_layer_is_the_trunk_pair_stack(token_z):
    """The MSA / template stack layer with the trunk layer's pair weights
    gives the trunk layer's z bit for bit (same modules, same order), at the
    trunk's width and at a template-like narrower one."""
    g = _gen(19)
    layer = R.randomize(R.PairformerLayer(token_s=32, token_z=token_z, num_heads=4, pairwise_head_width=8,
                                          pairwise_num_heads=2), generator=g)
    noseq = R.PairformerNoSeqLayer(token_z, pairwise_head_width=8, pairwise_num_heads=2)
    own = noseq.state_dict()
    noseq.load_state_dict({k: v for k, v in layer.state_dict().items() if k in own})
    with torch.no_grad():
        s = torch.randn(1, 6, 32, generator=g)
        z = torch.randn(1, 6, 6, token_z, generator=g)
        mask = torch.ones(1, 6)
        mask[:, -1] = 0
        pair_mask = mask[:, :, None] * mask[:, None, :]
        _, want = layer(s, z, mask, pair_mask)
        got = noseq(z, pair_mask)
    assert set(own) <= set(layer.state_dict())
    assert torch.equal(got, want)
