"""bmx_seq_attention_x3_batched_fwd (the split-bf16 pair-biased attention the
token transformer runs by default) against the float64 CPU restatement of
upstream AttentionPairBias (math as reference pair_bias.py:21-36) at the fp32
bar, 1e-4, and against the fp32-MFMA kernel on the same inputs: head widths 24,
32 and 48; key counts that are and are not multiples of the 32-key step
(1, 17, 300, 1000, 1024); query rows past a 16-row tile; bias shared by
groups of batch elements (upstream repeat_interleave); masked keys, one
broadcast mask or one per element; q / k / v / g as column slices of one fused
projection (row stride 4 H D)."""

import pytest
import torch

from boltz_lumi_amd import ops

pytestmark = pytest.mark.gpu


def max_rel(got, want):
    got, want = got.double().cpu(), want.double().cpu()
    return ((got - want).abs().max() / want.abs().max()).item()


def reference(q, k, v, bias, mask, gate, inf, bias_div):
    b, nq, width = q.shape
    heads = bias.shape[1]
    d = width // heads
    qh, kh, vh = (t.double().view(b, -1, heads, d).transpose(1, 2) for t in (q, k, v))
    logits = qh @ kh.transpose(-1, -2) / d ** 0.5 + bias.double().repeat_interleave(bias_div, 0)
    logits = logits + (1 - mask.double()[:, None, None]) * -inf
    o = (torch.softmax(logits, -1) @ vh).transpose(1, 2).reshape(b, nq, width)
    return torch.sigmoid(gate.double()) * o


def inputs(seed, b, nq, nk, heads, d, bias_div, mask_kind, fused):
    g = torch.Generator().manual_seed(seed)
    width = heads * d
    if fused:  # one [B, N, 4 H D] projection, as the token transformer's q | k | v | g GEMM
        proj = torch.randn(b, nq, 4 * width, generator=g)
        q, k, v, gate = proj.split(width, dim=-1)
    else:
        q, gate = torch.randn(b, nq, width, generator=g), torch.randn(b, nq, width, generator=g)
        k, v = torch.randn(b, nk, width, generator=g), torch.randn(b, nk, width, generator=g)
    bias = torch.randn(b // bias_div, heads, nq, nk, generator=g) * 2
    if mask_kind == "none":
        mask = torch.ones(b, nk)
    elif mask_kind == "shared":
        mask = (torch.rand(1, nk, generator=g) > 0.25).float()
        mask[:, 0] = 1
    else:
        mask = (torch.rand(b, nk, generator=g) > 0.25).float()
        mask[:, 0] = 1
    return q, k, v, bias, mask, gate


CASES = [  # b, nq, nk, heads, d, bias_div, mask, fused
    (5, 300, 300, 16, 48, 5, "none", True),     # token transformer shape, 5 samples sharing the bias
    (2, 1024, 1024, 4, 48, 1, "each", False),   # full key row, per-element masks
    (1, 200, 1000, 4, 48, 1, "shared", False),  # keys not a multiple of 32
    (3, 33, 17, 4, 32, 3, "each", False),       # short rows, queries past a 16-row tile
    (2, 77, 300, 16, 24, 1, "shared", False),   # head width 24 (Pairformer sequence stack width)
    (1, 1, 1, 16, 24, 1, "none", False),        # one query, one key
]


@pytest.mark.parametrize("b,nq,nk,heads,d,bias_div,mask_kind,fused", CASES)
def test_split_attention_matches_fp64_and_fp32_kernel(gpu, b, nq, nk, heads, d, bias_div, mask_kind, fused):
    q, k, v, bias, mask, gate = inputs(7 + nq + nk + d, b, nq, nk, heads, d, bias_div, mask_kind, fused)
    want = reference(q, k, v, bias, mask, gate, 1e6, bias_div)
    dev = [t.to(gpu) for t in (q, k, v, bias, mask, gate)]
    if fused:  # keep the column slices of one device tensor
        proj = torch.cat([q, k, v, gate], dim=-1).to(gpu)
        w = q.shape[-1]
        dev[0], dev[1], dev[2], dev[5] = proj[..., :w], proj[..., w:2 * w], proj[..., 2 * w:3 * w], proj[..., 3 * w:]
    with torch.inference_mode():
        got = ops.seq_attention_batched(*dev, 1e6, bias_div=bias_div, split=True)
        exact = ops.seq_attention_batched(*dev, 1e6, bias_div=bias_div, split=False)
    torch.cuda.synchronize()
    assert torch.isfinite(got).all()
    assert max_rel(got, want) < 1e-4
    assert max_rel(got, exact) < 1e-4


@pytest.mark.parametrize("b,nq,nk,heads,d,bias_div,mask_kind,fused", [CASES[0], CASES[2], CASES[3]])
def test_split_attention_split_output_is_the_split_of_its_output(gpu, b, nq, nk, heads, d, bias_div, mask_kind, fused):
    """split_out writes each output row as the split-bf16 operand of proj_o:
    [hi | hi | lo | 1 1 0 ...] of the fp32 output of the same kernel, bit for bit."""
    q, k, v, bias, mask, gate = inputs(11 + nq + nk + d, b, nq, nk, heads, d, bias_div, mask_kind, fused)
    dev = [t.to(gpu) for t in (q, k, v, bias, mask, gate)]
    with torch.inference_mode():
        out = ops.seq_attention_batched(*dev, 1e6, bias_div=bias_div, split=True)
        op = ops.seq_attention_batched(*dev, 1e6, bias_div=bias_div, split=True, split_out=True)
    w = heads * d
    rows = out.reshape(-1, w).cpu()
    op = op.cpu()
    hi = rows.bfloat16()
    assert op.shape == (b * nq, 3 * w + 64)
    assert torch.equal(op[:, :w], hi) and torch.equal(op[:, w:2 * w], hi)
    assert torch.equal(op[:, 2 * w:3 * w], (rows - hi.float()).bfloat16())
    assert (op[:, 3 * w:3 * w + 2] == 1).all() and (op[:, 3 * w + 2:] == 0).all()


def test_split_attention_is_the_default_for_the_token_transformer(gpu, monkeypatch):
    """Width 768 with 1024 keys takes the split kernel, 384 (the sequence
    stack) and short key rows the fp32 kernel, and exact fp32 mode turns the
    split off."""
    calls = []
    real = ops.N.call
    monkeypatch.setattr(ops.N, "call", lambda name, *a: (calls.append(name), real(name, *a))[1])

    def run(width, heads, nk):
        q, k, v, bias, mask, gate = inputs(3, 1, 16, nk, heads, width // heads, 1, "none", False)
        calls.clear()
        with torch.inference_mode():
            ops.seq_attention_batched(*(t.to(gpu) for t in (q, k, v, bias, mask, gate)), 1e6)
        return calls[-1]

    assert run(768, 16, 1024) == "bmx_seq_attention_x3_batched_fwd"
    assert run(384, 16, 1024) == "bmx_seq_attention_batched_fwd"
    assert run(768, 16, 128) == "bmx_seq_attention_batched_fwd"
    before = ops.exact_fp32_linears(True)
    try:
        assert run(768, 16, 1024) == "bmx_seq_attention_batched_fwd"
    finally:
        ops.exact_fp32_linears(before)


def test_split_attention_is_deterministic_at_the_token_shape(gpu):
    """Every block writes whole query rows from LDS stages that its own barrier
    publishes, so repeated calls on the same inputs must be bit-identical (the
    configs[4] shape: 5 samples x 1024 tokens, 16 heads x 48, one shared bias)."""
    b, n, heads, d = 5, 1024, 16, 48
    q, k, v, bias, mask, gate = inputs(5, b, n, n, heads, d, b, "none", True)
    mask[:, -37:] = 0
    proj = torch.cat([q, k, v, gate], dim=-1).to(gpu)
    w = heads * d
    dev = (proj[..., :w], proj[..., w:2 * w], proj[..., 2 * w:3 * w], bias.to(gpu), mask.to(gpu), proj[..., 3 * w:])
    with torch.inference_mode():
        runs = [ops.seq_attention_batched(*dev, 1e6, bias_div=b, split=True) for _ in range(3)]
        ops_ = [ops.seq_attention_batched(*dev, 1e6, bias_div=b, split=True, split_out=True) for _ in range(2)]
    torch.cuda.synchronize()
    assert torch.isfinite(runs[0]).all()
    assert all(torch.equal(r, runs[0]) for r in runs[1:])
    assert torch.equal(ops_[0], ops_[1])
