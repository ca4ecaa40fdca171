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
                                          pairwise_num_heads=2), generator=g).eval()
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
                                          pairwise_num_heads=2), generator=g).eval()
    noseq = R.PairformerNoSeqLayer(token_z, pairwise_head_width=8, pairwise_num_heads=2).eval()
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


# -------------------------------------------- PairformerLayer composition
#
# The op order of upstream PairformerLayer is a restatement (only an import
# of upstream Boltz could show it); what these pins fix is that each branch
# is the pinned module applied to the current z and added to it, that the
# branches chain (each reads the z its predecessor updated), and that the
# sequence stack runs in fp32 on the updated z.

_SMALL = dict(token_s=16, token_z=8, num_heads=2, pairwise_head_width=4, pairwise_num_heads=2)
_BRANCHES = ("tri_mul_out", "tri_mul_in", "tri_att_start", "tri_att_end", "transition_z")


def _small_layer(seed):
    return R.randomize(R.PairformerLayer(**_SMALL), generator=_gen(seed)).double().eval()


def _silence(layer, names):
    """Zero the final projection of each named branch (its output is then 0)."""
    final = {"tri_mul_out": "p_out", "tri_mul_in": "p_out", "tri_att_start": "mha.linear_o",
             "tri_att_end": "mha.linear_o", "transition_z": "fc3", "attention": "proj_o", "transition_s": "fc3"}
    with torch.no_grad():
        for name in names:
            mod = getattr(layer, name)
            for part in final[name].split("."):
                mod = getattr(mod, part)
            mod.weight.zero_()
            if getattr(mod, "bias", None) is not None:
                mod.bias.zero_()


def _brute_branch(layer, name, z, pair_mask):
    mod = getattr(layer, name)
    if name.startswith("tri_mul"):
        return B.triangle_multiplication(mod, z, pair_mask, outgoing=name.endswith("out"))
    if name.startswith("tri_att"):
        return B.triangle_attention(mod, z, pair_mask, starting=name.endswith("start"))
    return B.transition(mod, z)


def _small_inputs(seed, n=4):
    g = _gen(seed)
    s = torch.randn(1, n, _SMALL["token_s"], generator=g, dtype=torch.float64)
    z = torch.randn(1, n, n, _SMALL["token_z"], generator=g, dtype=torch.float64)
    mask = torch.ones(1, n, dtype=torch.float64)
    mask[:, -1] = 0
    return s, z, mask, mask[:, :, None] * mask[:, None, :]


@pytest.mark.parametrize("branch", _BRANCHES)
def test_pairformer_single_branch_is_residual_of_the_pinned_module(branch):
    """Every pair branch but one silenced (and the sequence stack too): z_out
    = z + branch(z) with the branch evaluated by the fp64 loops, s_out = s."""
    layer = _small_layer(20)
    _silence(layer, [b for b in _BRANCHES if b != branch] + ["attention", "transition_s"])
    s, z, mask, pm = _small_inputs(21)
    with torch.no_grad():
        s2, z2 = layer(s, z, mask, pm)
    want = z[0].numpy() + _brute_branch(layer, branch, z[0].numpy(), pm[0].numpy())
    assert _rel(z2[0], want) < 1e-10
    assert torch.equal(s2, s)


@pytest.mark.parametrize("first,second", [("tri_mul_out", "tri_att_end"), ("tri_mul_in", "transition_z"),
                                          ("tri_att_start", "tri_att_end")])
def test_pairformer_branches_chain_on_the_updated_z(first, second):
    """Two active branches: the second reads the z the first updated
    (z1 = z + f(z), z2 = z1 + g(z1)), not the layer input."""
    layer = _small_layer(22)
    _silence(layer, [b for b in _BRANCHES if b not in (first, second)] + ["attention", "transition_s"])
    s, z, mask, pm = _small_inputs(23)
    with torch.no_grad():
        _, z2 = layer(s, z, mask, pm)
    z0, m = z[0].numpy(), pm[0].numpy()
    z1 = z0 + _brute_branch(layer, first, z0, m)
    want = z1 + _brute_branch(layer, second, z1, m)
    parallel = z0 + _brute_branch(layer, first, z0, m) + _brute_branch(layer, second, z0, m)
    assert _rel(z2[0], want) < 1e-10
    assert _rel(want, parallel) > 1e-6  # far above the 1e-10 bar: the check tells chained from parallel


def test_pairformer_sequence_stack_runs_on_the_updated_z():
    """With the pair stack reduced to its transition, s_out = s1 + transition_s(s1),
    s1 = s + attention(pre_norm_s(s), z_out, mask, k_in=pre_norm_s(s)), every
    module by the fp64 loops: the sequence stack follows the pair stack and
    reads its result."""
    layer = _small_layer(24)
    _silence(layer, [b for b in _BRANCHES if b != "transition_z"])
    s, z, mask, pm = _small_inputs(25)
    with torch.no_grad():
        s2, z2 = layer(s, z, mask, pm)
    z_out = z[0].numpy() + B.transition(layer.transition_z, z[0].numpy())
    assert _rel(z2[0], z_out) < 1e-10
    sn = np.array([B.layer_norm_vec(list(r), B._p(layer, "pre_norm_s.weight"), B._p(layer, "pre_norm_s.bias"),
                                    layer.pre_norm_s.eps) for r in s[0].numpy()])[None]
    s1 = s.numpy() + B.attention_pair_bias(layer.attention, sn, z_out[None], mask.numpy(), sn)
    want = s1 + B.transition(layer.transition_s, s1)
    assert _rel(s2, want) < 1e-10
    stale = s.numpy() + B.attention_pair_bias(layer.attention, sn, z.numpy(), mask.numpy(), sn)
    assert _rel(stale + B.transition(layer.transition_s, stale), want) > 1e-7  # reading the old z would show


def test_pairformer_sequence_stack_is_fp32_under_autocast():
    """Under bf16 autocast the pair stack autocasts, but the sequence stack
    runs with autocast disabled: s_out equals the fp32 sequence stack applied
    to the (bf16-path) z_out, far inside the bf16 rounding it would show
    otherwise."""
    layer = R.randomize(R.PairformerLayer(**_SMALL), generator=_gen(26)).eval()
    g = _gen(27)
    n = 6
    s = torch.randn(1, n, 16, generator=g)
    z = torch.randn(1, n, n, 8, generator=g)
    mask = torch.ones(1, n)
    pm = mask[:, :, None] * mask[:, None, :]
    with torch.no_grad(), torch.autocast("cpu", dtype=torch.bfloat16):
        s_mix, z_mix = layer(s, z, mask, pm)
    with torch.no_grad():
        sn = layer.pre_norm_s(s)
        s1 = s + layer.attention(s=sn, z=z_mix.float(), mask=mask, k_in=sn)
        want = s1 + layer.transition_s(s1)
        # what the same stack gives when it autocasts
        with torch.autocast("cpu", dtype=torch.bfloat16):
            sn_b = layer.pre_norm_s(s)
            s1_b = s + layer.attention(s=sn_b, z=z_mix.float(), mask=mask, k_in=sn_b)
            bf16_stack = s1_b + layer.transition_s(s1_b)
    assert z_mix.dtype == torch.float32 and s_mix.dtype == torch.float32
    assert _rel(s_mix, want) < 1e-6
    assert _rel(bf16_stack, want) > 2e-5  # 20x the bar: a bf16 stack would fail it


# ------------------------------------ DiffusionTransformerLayer composition


def _dtl(seed, dim=8, heads=2, cond=6):
    layer = R.randomize(R.DiffusionTransformerLayer(heads, dim, cond), generator=_gen(seed)).double()
    return layer


def _dtl_inputs(seed, batch=2, n=5, dim=8, cond=6, heads=2, nk=None, bias_batch=None):
    g = _gen(seed)
    nk = n if nk is None else nk
    a = torch.randn(batch, n, dim, generator=g, dtype=torch.float64)
    s = torch.randn(batch, n, cond, generator=g, dtype=torch.float64)
    bias = torch.randn(bias_batch or batch, n, nk, heads, generator=g, dtype=torch.float64)
    mask = torch.ones(batch, n, dtype=torch.float64)
    mask[0, -2:] = 0
    return a, s, bias, mask


def test_diffusion_layer_without_attention_is_residual_transition():
    """pair_bias_attn.proj_o zeroed: out = a + transition(a, s), the
    conditioned transition by the fp64 loops (it acts on the updated a)."""
    layer = _dtl(30)
    with torch.no_grad():
        layer.pair_bias_attn.proj_o.weight.zero_()
    a, s, bias, mask = _dtl_inputs(31)
    with torch.no_grad():
        got = layer(a, s, bias=bias, mask=mask)
    want = a.numpy() + B.conditioned_transition(layer.transition, a.numpy(), s.numpy())
    assert _rel(got, want) < 1e-10


@pytest.mark.parametrize("multiplicity", [1, 2])
def test_diffusion_layer_without_transition_is_gated_attention(multiplicity):
    """transition.b_to_a zeroed: out = a + sigmoid(output_projection_linear(s))
    * attention(adaln(a, s), k_in=adaln(a, s)), AdaLN and the attention by the
    fp64 loops; with multiplicity m, sample b uses bias b // m."""
    layer = _dtl(32)
    with torch.no_grad():
        layer.transition.b_to_a.weight.zero_()
    a, s, bias, mask = _dtl_inputs(33, batch=2, bias_batch=2 // multiplicity)
    with torch.no_grad():
        got = layer(a, s, bias=bias, mask=mask, multiplicity=multiplicity)
    ad = B.adaln(layer.adaln, a.numpy(), s.numpy())
    att = B.attention_pair_bias_keys(layer.pair_bias_attn, ad, ad, bias.numpy(), mask.numpy(), multiplicity)
    w, b = B._p(layer, "output_projection_linear.weight"), B._p(layer, "output_projection_linear.bias")
    gate = np.array([[[B.sigmoid(t) for t in B.linear_vec(list(r), w, b)] for r in sb] for sb in s.numpy()])
    assert _rel(got, a.numpy() + gate * att) < 1e-10


def test_diffusion_layer_gathers_keys_and_their_mask():
    """With ``to_keys`` (the atom transformer's windows) the keys are the
    gathered AdaLN rows and the mask is gathered the same way: here windows
    of 2 queries over 4 keys of one 8-atom sample, the key indices written out
    by hand and clamped at the ends, with the transition silenced."""
    layer = _dtl(34)
    with torch.no_grad():
        layer.transition.b_to_a.weight.zero_()
    g = _gen(35)
    atoms, w, h = 8, 2, 4
    nw = atoms // w
    a = torch.randn(nw, w, 8, generator=g, dtype=torch.float64)
    s = torch.randn(nw, w, 6, generator=g, dtype=torch.float64)
    bias = torch.randn(nw, w, h, 2, generator=g, dtype=torch.float64)
    atom_mask = torch.tensor([1, 1, 1, 0, 1, 1, 0, 1], dtype=torch.float64)
    keys = [[max(0, min(atoms - 1, w * i + t - 1)) for t in range(h)] for i in range(nw)]  # centred, clamped
    index = torch.tensor(keys)

    def to_keys(x):
        return x.reshape(1, atoms, -1)[:, index].reshape(nw, h, -1)

    with torch.no_grad():
        got = layer(a, s, bias=bias, mask=atom_mask.view(nw, w), to_keys=to_keys)
    ad = B.adaln(layer.adaln, a.numpy(), s.numpy())  # [nw, w, 8]
    flat = ad.reshape(atoms, 8)
    k_in = np.array([[flat[keys[i][t]] for t in range(h)] for i in range(nw)])
    kmask = np.array([[atom_mask[keys[i][t]].item() for t in range(h)] for i in range(nw)])
    att = B.attention_pair_bias_keys(layer.pair_bias_attn, ad, k_in, bias.numpy(), kmask)
    wl, bl = B._p(layer, "output_projection_linear.weight"), B._p(layer, "output_projection_linear.bias")
    gate = np.array([[[B.sigmoid(t) for t in B.linear_vec(list(r), wl, bl)] for r in sb] for sb in s.numpy()])
    assert _rel(got, a.numpy() + gate * att) < 1e-10
    # the masked atoms 3 and 6 are masked as keys wherever a window gathers them
    assert kmask.tolist() == [[1, 1, 1, 1], [1, 1, 0, 1], [0, 1, 1, 0], [1, 0, 1, 1]]


def test_diffusion_layer_default_gate_init():
    """Upstream initialises both output gates to weight 0, bias -2
    (sigmoid(-2) ~ 0.119 on every channel before training)."""
    layer = R.DiffusionTransformerLayer(2, 8, 6)
    for lin in (layer.output_projection_linear, layer.transition.output_projection[0]):
        assert not lin.weight.any() and torch.all(lin.bias == -2.0)


# ------------------------------------------------ diffusion transformer stacks


def _window_keys_by_formula(x, w, h):
    """Key t of window k is atom W k - (H - W) / 2 + t, zero outside the
    sequence (upstream's centred windows written out directly)."""
    b, n, d = x.shape
    out = torch.zeros(b, n // w, h, d, dtype=x.dtype)
    for k in range(n // w):
        for t in range(h):
            atom = w * k - (h - w) // 2 + t
            if 0 <= atom < n:
                out[:, k, t] = x[:, atom]
    return out


@pytest.mark.parametrize("n,w,h", [(128, 32, 128), (96, 8, 32), (64, 16, 64)])
def test_single_to_keys_is_the_centred_window(n, w, h):
    x = torch.randn(2, n, 3, generator=_gen(40), dtype=torch.float64)
    got = R.single_to_keys(x, R.get_indexing_matrix(n // w, w, h), w, h)
    assert torch.equal(got, _window_keys_by_formula(x, w, h))


def test_diffusion_transformer_slices_the_bias_per_layer():
    """Layer i of the stack sees bias channels i*H .. i*H+H-1, in dense and in
    head-major (prepacked) storage alike."""
    torch.manual_seed(41)
    stack = R.randomize(R.DiffusionTransformer(3, 2, 8, 6), generator=_gen(42)).double()
    a, s, _, mask = _dtl_inputs(43)
    bias = torch.randn(2, 5, 5, 6, generator=_gen(44), dtype=torch.float64)
    packed = bias.permute(0, 3, 1, 2).contiguous().permute(0, 2, 3, 1)  # upstream-layout, head-major storage
    with torch.no_grad():
        got = stack(a, s, bias, mask)
        got_packed = stack(a, s, packed, mask)
        want = a
        for i, layer in enumerate(stack.layers):
            want = layer(want, s, bias[..., 2 * i:2 * i + 2].contiguous(), mask)
    assert torch.equal(got, want) and torch.equal(got_packed, want)


@pytest.mark.parametrize("multiplicity", [1, 2])
def test_atom_transformer_windows_and_multiplicity(multiplicity):
    """The windowed stack equals its layers applied window by window, with
    keys and key mask gathered by the centred-window formula, zero keys
    masked, and sample j of a structure using that structure's window bias."""
    w, h, n, heads, depth = 8, 16, 32, 2, 2
    nw = n // w
    tr = R.randomize(R.AtomTransformer(w, h, depth, heads, 8, 6), generator=_gen(45)).double()
    g = _gen(46)
    batch = 2 * multiplicity  # 2 structures x multiplicity samples
    q = torch.randn(batch, n, 8, generator=g, dtype=torch.float64)
    c = torch.randn(batch, n, 6, generator=g, dtype=torch.float64)
    mask = (torch.rand(batch, n, generator=g) > 0.2).double()
    bias = torch.randn(2, nw, w, h, depth * heads, generator=g, dtype=torch.float64)
    index = R.get_indexing_matrix(nw, w, h)

    def to_keys(x):
        return R.single_to_keys(x, index, w, h)

    with torch.no_grad():
        got = tr(q, c, bias, to_keys, mask, multiplicity)
        want = torch.empty_like(q)
        for bi in range(batch):
            x, cond = q[bi], c[bi]  # this sample's atoms, all windows
            kmask = _window_keys_by_formula(mask[bi].view(1, n, 1), w, h)[0, :, :, 0]  # [nw, h]
            for i, layer in enumerate(tr.diffusion_transformer.layers):
                ad = layer.adaln(x[None], cond[None])[0]
                keys = _window_keys_by_formula(ad[None], w, h)[0]  # [nw, h, D]
                nxt = torch.empty_like(x)
                for k in range(nw):
                    rows = slice(w * k, w * (k + 1))
                    sl = bias[bi // multiplicity, k, :, :, heads * i:heads * (i + 1)][None]
                    att = layer.pair_bias_attn(s=ad[None, rows], z=sl, mask=kmask[k][None], k_in=keys[k][None])
                    y = x[None, rows] + layer.output_projection(cond[None, rows]) * att
                    nxt[rows] = (y + layer.transition(y, cond[None, rows]))[0]
                x = nxt
            want[bi] = x
    assert _rel(got, want) < 1e-12


@pytest.mark.parametrize("branch,columnwise", [("tri_mul_out", False), ("tri_att_start", False),
                                               ("tri_att_end", True)])
def test_pairformer_dropout_masks_rows_or_columns(branch, columnwise):
    """The dropout masks (upstream ``get_dropout_mask``): in training with rate
    1/2 and only ``branch`` left on, z_out - z is, per row (per column for the
    ending node), either zero or twice the branch output on the same z, and
    both kinds occur; in eval the layer equals the unmasked sum, and it draws
    from the generator exactly what the four masks' shapes draw (3 x [B, N]
    and 1 x [B, N]), so a caller's later draws are those of the upstream layer."""
    layer = _small_layer(30)
    layer.dropout = 0.5
    _silence(layer, [b for b in _BRANCHES if b != branch])
    g = _gen(31)
    n = 12
    s = torch.randn(1, n, 16, generator=g, dtype=torch.float64)
    z = torch.randn(1, n, n, 8, generator=g, dtype=torch.float64)
    mask = torch.ones(1, n, dtype=torch.float64)
    pm = mask[:, :, None] * mask[:, None, :]
    mod = getattr(layer, branch)
    with torch.no_grad():
        y = mod(z, mask=pm)
        layer.train()
        torch.manual_seed(5)
        _, z2 = layer(s, z, mask, pm)
        layer.eval()
        torch.manual_seed(6)
        _, z_eval = layer(s, z, mask, pm)
        after = torch.rand(3)
        torch.manual_seed(6)
        for _ in range(4):
            torch.rand(1, n, dtype=torch.float64)
        expected_after = torch.rand(3)
    d = (z2 - z)[0]
    y = y[0]
    if columnwise:
        d, y = d.transpose(0, 1), y.transpose(0, 1)
    kinds = set()
    for r in range(n):
        if torch.equal(d[r], torch.zeros_like(d[r])):
            kinds.add(0)
        else:
            assert torch.allclose(d[r], 2 * y[r], rtol=1e-12, atol=1e-12)
            kinds.add(1)
    assert kinds == {0, 1}
    assert torch.allclose(z_eval, z + y[None] if not columnwise else z + y.transpose(0, 1)[None], rtol=1e-12,
                          atol=1e-12)
    assert torch.equal(after, expected_after)
