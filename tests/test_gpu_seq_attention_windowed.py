"""bmx_seq_attention_windowed_fwd (the atom transformer's attention with the
to_keys gather done by addressing) against float64 upstream math: keys
gathered through the oracle's single_to_keys / get_indexing_matrix (upstream
encodersv2, zero rows past the ends), the per-structure window bias repeated
over the samples (upstream repeat_interleave) and read in place as one
layer's heads of the [B, windows, W, H, layers * heads] atom bias, the key
mask gathered the same way (pair_bias.py:21-36 math).  Cases: the bias in
upstream's layout and channel-major (prepare_window_bias), first and last
windows with absent keys, padded atoms at the end of a sample (every window
keeps a valid key: a fully masked row's softmax of -1e6-shifted logits is
quantised by fp32 in upstream too), two structures with two samples each, head
widths 24, 32 and 48.  Also the to_keys probe that gates the path."""

import functools

import pytest
import torch

from boltz_lumi_amd import diffusion, ops
from boltz_lumi_amd.pair_bias import prepare_window_bias, window_bias_prepared
from oracle import boltz_ref as R

pytestmark = pytest.mark.gpu


def reference(q, k, v, bias5, mask, g, index, w, h, mult, heads, layer, inf):
    """float64 upstream: window keys by single_to_keys, bias repeated per sample."""
    e, _, width = q.shape
    b = mask.shape[0]
    n = mask.shape[1]
    nw = n // w
    d = width // heads
    kw = R.single_to_keys(k.double().view(b, n, width), index.double(), w, h).view(e, h, width)
    vw = R.single_to_keys(v.double().view(b, n, width), index.double(), w, h).view(e, h, width)
    mw = R.single_to_keys(mask.double().view(b, n, 1), index.double(), w, h).view(e, h)
    bias = bias5.double().repeat_interleave(mult, 0).view(e, w, h, -1)[..., layer * heads:(layer + 1) * heads]
    qh = q.double().view(e, w, heads, d).transpose(1, 2)
    kh, vh = (t.view(e, h, heads, d).transpose(1, 2) for t in (kw, vw))
    logits = qh @ kh.transpose(-1, -2) / d ** 0.5 + bias.permute(0, 3, 1, 2)
    logits = logits + (1 - mw[:, None, None]) * -inf
    o = (torch.softmax(logits, -1) @ vh).transpose(1, 2).reshape(e, w, width)
    return torch.sigmoid(g.double()) * o


CASES = [  # structures, samples each, atoms, heads, head dim, padded atoms at the end, bias channel-major
    (1, 2, 8 * 32, 4, 32, 0, True),
    (1, 2, 8 * 32, 4, 32, 0, False),
    (2, 2, 6 * 32, 4, 32, 40, True),
    (2, 2, 6 * 32, 4, 32, 40, False),
    (1, 3, 5 * 32, 2, 24, 7, True),
    (1, 1, 4 * 32, 2, 48, 0, False),
]


@pytest.mark.parametrize("structures,mult,n,heads,d,pad,prepared", CASES)
def test_windowed_attention_matches_gathered_fp64(gpu, structures, mult, n, heads, d, pad, prepared):
    w, h, layers, layer, inf = 32, 128, 3, 1, 1e6
    g_ = torch.Generator().manual_seed(n + heads + pad)
    b, nw, width = structures * mult, n // 32, heads * d
    proj = torch.randn(b * n, 4 * width, generator=g_)  # q | k | v | g of the atom rows
    bias5 = torch.randn(structures, nw, w, h, layers * heads, generator=g_) * 2
    mask = torch.ones(b, n)
    if pad:
        mask[:, -pad:] = 0
    index = R.get_indexing_matrix(nw, w, h)
    q, k, v, g = proj.split(width, dim=-1)
    e = b * nw
    want = reference(q.reshape(e, w, width), k, v, bias5, mask, g.reshape(e, w, width), index, w, h, mult, heads,
                     layer, inf)
    pd, bd, md = proj.to(gpu), bias5.to(gpu), mask.reshape(-1).to(gpu)
    if prepared:  # the layout optimized_sample hands the atom transformers
        bd = prepare_window_bias(bd)
        assert window_bias_prepared(bd) and torch.equal(bd, bias5.to(gpu))
    qd, kd, vd, gd = pd.split(width, dim=-1)
    with torch.inference_mode():
        got = ops.seq_attention_windowed(qd.view(e, w, width), kd, vd, bd[..., layer * heads:(layer + 1) * heads], md,
                                         gd.view(e, w, width), inf, windows=nw, key_offset=(w - h) // 2,
                                         bias_group=mult * nw)
    torch.cuda.synchronize()
    assert torch.isfinite(got).all()
    err = ((got.double().cpu() - want).abs().max() / want.abs().max()).item()
    assert err < 1e-4


def test_window_probe_accepts_the_gather_only(gpu):
    """window_key_offset accepts upstream's single_to_keys partial (the offset
    (W - H) / 2) and rejects a to_keys with another window layout."""
    n, w, h = 8 * 32, 32, 128
    index = R.get_indexing_matrix(n // w, w, h, device=gpu)
    good = functools.partial(R.single_to_keys, indexing_matrix=index, w=w, h=h)
    shifted = functools.partial(R.single_to_keys, indexing_matrix=torch.roll(index, 1, 0), w=w, h=h)
    assert diffusion.window_key_offset(good, n, w, h, gpu) == (w - h) // 2
    assert diffusion.window_key_offset(shifted, n, w, h, gpu) is None
    assert diffusion.window_key_offset(lambda x: x[:, :1].expand(1, n // w * h, 1), n, w, h, gpu) is None
