"""The triangle-attention core (stage 2 of bmx_triattn_fwd) against an fp32
softmax of its own bf16 workspace inputs: q, k, v^T, the triangle bias and the
mask bias are read back from the workspace after the projection stage, so the
check isolates the core's online softmax.  Covers the speculative pass (the
running max frozen after the first 64 keys) and its fall-back, which must
redo a block whose later scores rise far above the first stage's."""

import pytest
import torch

from boltz_lumi_amd import layers, ops

pytestmark = pytest.mark.gpu

H, D = 4, 32


def _views(ws, n):
    npad = (n + 255) // 256 * 256
    e = npad * H * npad * D
    w = ws.view(torch.bfloat16)
    q = w[0:e].view(npad, H, npad, D)
    k = w[e:2 * e].view(npad, H, npad, D)
    vt = w[2 * e:3 * e].view(npad, H, D, npad)
    o_elems = (n * n * 128 * 2 + 255) // 256 * 256 // 2
    o = w[3 * e:3 * e + n * n * 128].view(n, n, 128)
    tb = w[3 * e + o_elems:3 * e + o_elems + H * npad * npad]
    mb = ws[(3 * e + o_elems + H * npad * npad) * 2:].view(torch.float32)[:npad * npad].view(npad, npad)
    return npad, q, k, vt, o, tb, mb


def _reference(n, npad, q, k, vt, tb, mb):
    """softmax_j(q.k + tb + mb) (log2 units) times v, fp32, [n, n, 128]."""
    dev = q.device
    nb = npad // 16
    hh = torch.arange(H, device=dev)[:, None, None]
    qq = torch.arange(n, device=dev)[None, :, None]
    kk = torch.arange(n, device=dev)[None, None, :]
    off = ((hh * nb + qq // 16) * nb + kk // 16) * 256 + (((kk % 16) // 8) * 16 + qq % 16) * 8 + kk % 8
    bias = tb[off].float()                                    # [H, q, k]
    j = torch.arange(n, device=dev)
    jb = j % 32
    slot = (j - jb) + ((jb >> 2) & 3) * 8 + ((jb >> 4) & 1) * 4 + (jb & 3)
    v = vt[:n, :, :, slot].float()                            # [i, H, D, k]
    s = torch.einsum("ihqd,ihkd->ihqk", q[:n, :, :n].float(), k[:n, :, :n].float())
    s = s + bias[None] + mb[:n, None, None, :n]
    p = torch.softmax(s * 0.6931471805599453, dim=-1)         # 2^s normalised
    o = torch.matmul(p, v.transpose(-1, -2).contiguous())    # [i, H, q, D]
    return o.permute(0, 2, 1, 3).reshape(n, n, H * D)


@pytest.mark.parametrize("boost", [1.0, 20.0, 3000.0])
def test_core_matches_fp32_softmax_of_its_inputs(gpu, boost):
    """boost scales k of the keys past the first 64 (the first stage).  The
    unboosted scores have std 0.5 and max 2.3 (log2 units); 20 lifts later
    scores up to ~45 above the first stage's max (the speculative pass keeps
    p far above 2^8 and must stay exact); 3000 lifts them past 2^100, so the
    speculative pass overflows and the block is redone with the tracked max."""
    torch.manual_seed(5)
    n = 200
    m = layers.TriangleAttention().to(gpu).eval()
    x = torch.randn(1, n, n, 128, device=gpu)
    ws = ops.new_workspace(n, gpu)
    with torch.inference_mode():
        ops.triattn(m, x[0], None, True, ops.OUT_BF16, None, ws, stages=1)
        npad, q, k, vt, o, tb, mb = _views(ws, n)
        if boost != 1.0:
            k[:, :, 64:n] = (k[:, :, 64:n].float() * boost).bfloat16()
        ops.triattn(m, x[0], None, True, ops.OUT_BF16, None, ws, stages=2)
        want = _reference(n, npad, q, k, vt, tb, mb)
        got = o.float()
    assert torch.isfinite(got).all()
    err = ((got - want).abs().max() / want.abs().max()).item()
    assert err < 2e-2, err


@pytest.mark.parametrize("gap", [50.0, 200.0])
def test_core_rows_far_below_their_block_partner(gpu, gap):
    """A block's rows share one softmax offset in the speculative pass.  Even
    rows get q = 1 and k = -gap/32, so their scores sit ``gap`` (log2 units)
    below the odd rows': at 50 the shared offset leaves their weights near
    2^-50, still exact in fp32 and bf16; at 200 their row sums underflow, the
    pass reports it and the block is redone with per-row maxima."""
    torch.manual_seed(6)
    n = 200
    m = layers.TriangleAttention().to(gpu).eval()
    x = torch.randn(1, n, n, 128, device=gpu)
    ws = ops.new_workspace(n, gpu)
    with torch.inference_mode():
        ops.triattn(m, x[0], None, True, ops.OUT_BF16, None, ws, stages=1)
        npad, q, k, vt, o, tb, mb = _views(ws, n)
        q[0:n:2, :, :n] = 1.0
        k[0:n:2, :, :n] = -gap / D
        ops.triattn(m, x[0], None, True, ops.OUT_BF16, None, ws, stages=2)
        want = _reference(n, npad, q, k, vt, tb, mb)
        got = o.float()
    assert torch.isfinite(got).all()
    for rows in (slice(0, n, 2), slice(1, n, 2)):
        err = ((got[rows] - want[rows]).abs().max() / want[rows].abs().max()).item()
        assert err < 2e-2, err


@pytest.mark.parametrize("n,masked,boost", [(200, "last31", 1.0), (200, "last140", 1.0), (256, "last51", 1.0),
                                            (200, "last31", 3000.0), (200, "random10", 1.0)])
def test_core_token_padding(gpu, n, masked, boost):
    """Token masks (pair mask m_i m_k).  Rows of unmasked tokens have their
    masked keys as a suffix when the padding is at the end: those blocks run
    the speculative pass with the mask bias added from the first stage that
    holds a padded key and skip the stages past the last open key (last31:
    the mask starts inside a stage; last140: every row has fewer than 64 open
    keys, so one stage).  Rows of padded tokens have no open key and take the
    masked path (uniform weights), as do rows whose masked keys are not a
    suffix (random10).  boost 3000 makes the speculative pass overflow after
    its first stage, so those blocks are redone on the masked path."""
    torch.manual_seed(7)
    m = layers.TriangleAttention().to(gpu).eval()
    x = torch.randn(1, n, n, 128, device=gpu)
    tok = torch.ones(n, device=gpu)
    if masked.startswith("last"):
        tok[n - int(masked[4:]):] = 0
    else:
        tok[torch.randperm(n, generator=torch.Generator().manual_seed(8))[:int(masked[6:]) * n // 100].to(gpu)] = 0
    mask = (tok[:, None] * tok[None, :]).contiguous()
    ws = ops.new_workspace(n, gpu)
    with torch.inference_mode():
        ops.triattn(m, x[0], mask, True, ops.OUT_BF16, None, ws, stages=1)
        npad, q, k, vt, o, tb, mb = _views(ws, n)
        if boost != 1.0:
            k[:, :, 64:n] = (k[:, :, 64:n].float() * boost).bfloat16()
        ops.triattn(m, x[0], mask, True, ops.OUT_BF16, None, ws, stages=2)
        want = _reference(n, npad, q, k, vt, tb, mb)
        got = o.float()
    assert torch.isfinite(got).all()
    # open rows, and the padded rows (uniform weights; with boosted keys their
    # scores no longer vanish next to the 1e9 mask bias in fp32, so only the
    # open rows are compared there)
    for rows in (tok.bool(), ~tok.bool()) if boost == 1.0 else (tok.bool(),):
        if rows.any():
            err = ((got[rows] - want[rows]).abs().max() / want[rows].abs().max()).item()
            assert err < 2e-2, err


def test_core_fractional_mask_rows(gpu):
    """Masks that are neither 0 nor 1 (mask bias between 0 and -1e9 log2 e):
    rows whose every key is fractional have no open key but are not uniform,
    so they must take the masked path, not the closed-row mean; rows mixing
    open, closed and fractional keys likewise."""
    torch.manual_seed(9)
    n = 160
    m = layers.TriangleAttention().to(gpu).eval()
    x = torch.randn(1, n, n, 128, device=gpu)
    g = torch.Generator().manual_seed(10)
    mask = torch.ones(n, n)
    mask[:64] = 1.0 - (torch.rand(64, n, generator=g) * 9e-7 + 2e-7)  # fractional everywhere, just below 1
    mask[64:96, 100:] = 0.0                                   # open keys then a closed suffix
    mask[64:96, 120:130] = 0.9999999                         # ... with fractional keys inside it
    mask = mask.to(gpu)
    ws = ops.new_workspace(n, gpu)
    with torch.inference_mode():
        ops.triattn(m, x[0], mask, True, ops.OUT_BF16, None, ws, stages=3)
        npad, q, k, vt, o, tb, mb = _views(ws, n)
        want = _reference(n, npad, q, k, vt, tb, mb)
        got = o.float()
    assert torch.isfinite(got).all()
    err = ((got - want).abs().max() / want.abs().max()).item()
    assert err < 2e-2, err
