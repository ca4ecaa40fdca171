"""GPU tests of the installed Pairformer layers (``pairformer.py``): after
``install`` an upstream-structured ``PairformerLayer`` (the oracle class, with
Boltz's names, parameters and dropout draws) runs the fused composition under
bf16 autocast.  Checked here:

* at N = 1024 (the headline shape, 24 padded tokens) against the fp32 CPU
  oracle, and bit for bit against this package's own ``layers.PairformerLayer``
  on the same weights (the benchmarked layer: the same kernels); at the
  reference's published N = 1134 and 2511 against the oracle layer in fp32
  on the GPU;
* the dropout masks: the generator ends in the state upstream's forward leaves
  it in, and masks with zeros (forced on both sides) drop the same rows and
  columns as the oracle's;
* fallbacks to the class forward, values and gradients equal: a hook on a
  child module, grad mode, ``use_kernels``, fp32 mode;
* ``PairformerNoSeqLayer`` (the MSA stack) against the oracle;
* the fused modules and the layer on a non-default stream (reference
  tests/test_pair_transition.py:68-78);
* the weight-pack cache after in-place parameter updates, including
  parameters made under ``torch.inference_mode`` (reference
  tests/test_operator_additions.py:131-138);
* grad-mode fallback of triangle multiplication and the pair transition with
  equal gradients (reference tests/test_operator_additions.py:139-147,
  tests/test_pair_transition.py:79-93);
* the output kernels' row scale (``row_scale``) composed exactly.
"""

import copy

import pytest
import torch
from torch import nn

from boltz_lumi_amd import adapters, layers, ops, pairformer
from oracle import boltz_ref as R

pytestmark = pytest.mark.gpu

TOL = 2e-2


class Boltz2(nn.Module):
    def __init__(self, layer):
        super().__init__()
        self.pairformer_module = nn.Module()
        self.pairformer_module.layers = nn.ModuleList([layer])


def rel(got, want, base=None):
    got, want = got.double().cpu(), want.double().cpu()
    if base is not None:
        base = base.double().cpu()
        got, want = got - base, want - base
    return ((got - want).abs().max() / want.abs().max()).item()


def inputs(n, padded, seed, c_s=384):
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(1, n, n, 128, generator=g)
    s = torch.randn(1, n, c_s, generator=g)
    mask = torch.ones(1, n)
    if padded:
        mask[:, -padded:] = 0
    return s, z, mask, mask[:, :, None] * mask[:, None, :]


def installed(seed, gpu):
    ref = R.randomize(R.PairformerLayer(), generator=torch.Generator().manual_seed(seed)).eval()
    host = Boltz2(copy.deepcopy(ref).to(gpu))
    assert adapters.install(host, require_boltz2=False) == 6
    layer = host.pairformer_module.layers[0]
    assert "forward" in vars(layer)
    return ref, layer


def test_installed_layer_at_n1024_matches_oracle_and_benchmarked_layer(gpu):
    n = 1024
    print(f"installed PairformerLayer n={n} padded=24", flush=True)
    ref, layer = installed(0, gpu)
    s, z, mask, pm = inputs(n, 24, 1)
    mine = layers.PairformerLayer()
    mine.load_state_dict(ref.state_dict())
    mine = mine.to(gpu).eval()
    sg, zg, mg, pmg = (t.to(gpu) for t in (s, z, mask, pm))
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
        s_got, z_got = layer(sg, zg, mg, pmg, 128)
        # the reference's composition: upstream's layer forward over the patched modules
        _, z_modules = type(layer).forward(layer, sg, zg, mg, pmg, 128)
    with torch.inference_mode():
        s_mine, z_mine = mine(sg, zg, mg, pmg)
    torch.cuda.synchronize()
    assert z_got.dtype == torch.float32 and s_got.dtype == torch.float32
    assert torch.equal(zg.cpu(), z)  # the caller's z is not modified
    # same kernels, masks of ones: bit for bit the benchmarked layer
    assert torch.equal(z_got, z_mine) and torch.equal(s_got, s_mine)
    # every branch adds its bf16 output in fp32, in place or by torch: the same z
    assert torch.equal(z_got, z_modules)
    with torch.no_grad():
        s_ref, z_ref = ref(s, z, mask, pm)
    err_z, err_s = rel(z_got, z_ref, z), rel(s_got, s_ref, s)
    print(f"  z update {err_z:.2e}  s update {err_s:.2e}", flush=True)
    assert err_z < TOL and err_s < TOL


@pytest.mark.parametrize("n", [1134, 2511])
def test_installed_layer_at_the_reference_token_counts(gpu, n):
    """The installed layer at the token counts the reference publishes (3
    padded tokens) against upstream's fp32 composition, the oracle layer,
    evaluated on the same GPU (on the CPU it would take minutes); both calls
    start from the same generator state, so they draw the same dropout masks."""
    print(f"installed PairformerLayer n={n} against the fp32 oracle layer on the GPU", flush=True)
    ref, layer = installed(7, gpu)
    ref_gpu = copy.deepcopy(ref).to(gpu)  # not installed: upstream's forward in fp32
    sg, zg, mg, pmg = (t.to(gpu) for t in inputs(n, 3, 2))
    with torch.inference_mode():
        torch.manual_seed(11)
        s_ref, z_ref = ref_gpu(sg, zg, mg, pmg, chunk_size_tri_attn=128)
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
        torch.manual_seed(11)
        s_got, z_got = layer(sg, zg, mg, pmg, 128)
    assert z_got.dtype == torch.float32 and torch.isfinite(z_got).all() and torch.isfinite(s_got).all()

    def rel_gpu(got, want, base):
        d, w = got - base, want - base
        return ((d - w).abs().max() / w.abs().max()).item()

    err_z, err_s = rel_gpu(z_got, z_ref, zg), rel_gpu(s_got, s_ref, sg)
    print(f"  z update {err_z:.2e}  s update {err_s:.2e}", flush=True)
    assert err_z < TOL and err_s < TOL


@pytest.mark.parametrize("n,padded", [(1, 0), (2, 1), (5, 2)])
def test_installed_layer_at_the_smallest_sizes(gpu, n, padded):
    """The installed layer (fused pair stack and sequence stack) at one, two
    and five tokens, the last ones padded, against the fp32 oracle layer:
    the kernels' tiles hold almost nothing but padding."""
    print(f"installed PairformerLayer n={n} padded={padded}", flush=True)
    ref, layer = installed(3, gpu)
    s, z, mask, pm = inputs(n, padded, 4)
    sg, zg, mg, pmg = (t.to(gpu) for t in (s, z, mask, pm))
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
        s_got, z_got = layer(sg, zg, mg, pmg, 128)
    with torch.no_grad():
        s_ref, z_ref = ref(s, z, mask, pm)
    assert z_got.shape == z.shape and s_got.shape == s.shape
    assert torch.isfinite(z_got).all() and torch.isfinite(s_got).all()
    err_z, err_s = rel(z_got, z_ref, z), rel(s_got, s_ref, s)
    print(f"  z update {err_z:.2e}  s update {err_s:.2e}", flush=True)
    assert err_z < TOL and err_s < TOL


def test_generator_state_follows_upstream(gpu):
    ref, layer = installed(2, gpu)
    s, z, mask, pm = (t.to(gpu) for t in inputs(96, 5, 3))
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
        torch.cuda.manual_seed(11)
        layer(s, z, mask, pm)
        after_fused = torch.cuda.get_rng_state()
        next_fused = torch.rand(4, device=gpu)
        torch.cuda.manual_seed(11)
        type(layer).forward(layer, s, z, mask, pm)  # upstream composition (its modules patched)
        after_upstream = torch.cuda.get_rng_state()
        next_upstream = torch.rand(4, device=gpu)
    assert torch.equal(after_fused, after_upstream)
    assert torch.equal(next_fused, next_upstream)


def test_forced_dropout_zeros_drop_the_same_rows_and_columns(gpu, monkeypatch):
    """Draws that are exactly 0 (probability ~2^-24 each) drop a row of a
    branch update (a column for the ending node); forced on both sides, the
    installed layer follows the oracle's masks."""
    n = 96
    ref, layer = installed(4, gpu)
    s, z, mask, pm = inputs(n, 3, 5)
    drops = [[1, 17, 50], [2, 33], [0, 64, 95], [5, 40, 41]]

    def masks(counter):
        def fake(z_, columnwise=False):
            k = counter[0] % 4
            counter[0] += 1
            shape = (z_.shape[0], 1, z_.shape[2], 1) if columnwise else (z_.shape[0], z_.shape[1], 1, 1)
            d = torch.ones(shape, dtype=z_.dtype, device=z_.device)
            d.view(-1)[drops[k]] = 0
            assert (k == 3) == columnwise
            return d
        return fake

    oracle_fake, fused_fake = masks([0]), masks([0])
    monkeypatch.setattr(R, "get_dropout_mask", lambda p, z_, training, columnwise=False: oracle_fake(z_, columnwise))
    monkeypatch.setattr(pairformer, "dropout_mask", lambda lay, z_, columnwise=False: fused_fake(z_, columnwise))
    with torch.no_grad():
        s_ref, z_ref = ref(s, z, mask, pm)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            s_got, z_got = layer(*(t.to(gpu) for t in (s, z, mask, pm)))
    assert rel(z_got, z_ref, z) < TOL and rel(s_got, s_ref, s) < TOL
    # without the masks the updates differ at the dropped rows: the check above has teeth
    with torch.no_grad():
        monkeypatch.setattr(R, "get_dropout_mask", lambda p, z_, training, columnwise=False: torch.ones_like(
            z_[:, 0:1, :, 0:1] if columnwise else z_[:, :, 0:1, 0:1]))
        _, z_plain = ref(s, z, mask, pm)
    assert rel(z_plain, z_ref, z) > 3 * TOL


def test_fallbacks_match_the_class_forward(gpu, monkeypatch):
    ref, layer = installed(6, gpu)
    s, z, mask, pm = (t.to(gpu) for t in inputs(64, 4, 7))
    fused_calls = []
    real = pairformer.pair_stack
    monkeypatch.setattr(pairformer, "pair_stack", lambda *a, **k: fused_calls.append(1) or real(*a, **k))

    def run(fn, *args, **kw):
        torch.cuda.manual_seed(3)
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
            return fn(*args, **kw)

    upstream = run(type(layer).forward, layer, s, z, mask, pm)
    assert fused_calls == []
    fused = run(layer, s, z, mask, pm)
    assert fused_calls == [1]  # the fused path ran
    assert torch.equal(fused[1], upstream[1]) and rel(fused[0], upstream[0], s) < TOL
    seen = []
    handle = layer.tri_att_start.register_forward_hook(lambda *a: seen.append(1))
    try:
        hooked = run(layer, s, z, mask, pm)
    finally:
        handle.remove()
    assert seen == [1] and fused_calls == [1]  # the hook fired: the class forward ran
    assert all(torch.equal(a, b) for a, b in zip(hooked, upstream))
    kernels = run(layer, s, z, mask, pm, None, False, True, False)  # use_cuequiv_mul requested
    assert all(torch.equal(a, b) for a, b in zip(kernels, run(type(layer).forward, layer, s, z, mask, pm, None,
                                                                 False, True, False)))
    assert fused_calls == [1]
    # fp32 mode (autocast off): the class forward, whose triangle attention runs natively in fp32
    torch.cuda.manual_seed(3)
    with torch.no_grad():
        f32 = layer(s, z, mask, pm)
        torch.cuda.manual_seed(3)
        f32_up = type(layer).forward(layer, s, z, mask, pm)
    assert all(torch.equal(a, b) for a, b in zip(f32, f32_up))
    # grad mode: upstream values and gradients (every child falls back too)
    zr = z.clone().requires_grad_(True)
    sr = s.clone().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        torch.cuda.manual_seed(3)
        s_g, z_g = layer(sr, zr, mask, pm)
        grads = torch.autograd.grad((s_g.float().sum() + z_g.float().sum()), (sr, zr))
        adapters.uninstall(layer)
        torch.cuda.manual_seed(3)
        s_u, z_u = layer(sr, zr, mask, pm)
        grads_u = torch.autograd.grad((s_u.float().sum() + z_u.float().sum()), (sr, zr))
    assert torch.equal(s_g, s_u) and torch.equal(z_g, z_u)
    assert all(torch.equal(a, b) for a, b in zip(grads, grads_u))


def test_noseq_layer_matches_oracle(gpu):
    n = 160
    ref = R.randomize(R.PairformerNoSeqLayer(128), generator=torch.Generator().manual_seed(8)).eval()
    host = nn.Module()
    host.msa_module = nn.Module()
    host.msa_module.layer = copy.deepcopy(ref).to(gpu)
    assert adapters.install(host, require_boltz2=False) == 6
    _, z, _, pm = inputs(n, 9, 9)
    with torch.no_grad():
        want = ref(z, pm)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            got = host.msa_module.layer(z.to(gpu), pm.to(gpu))
    assert got.dtype == torch.float32 and rel(got, want, z) < TOL


def test_layer_and_modules_on_a_side_stream(gpu):
    ref, layer = installed(10, gpu)
    s, z, mask, pm = (t.to(gpu) for t in inputs(130, 6, 11))
    side = torch.cuda.Stream()
    x = z[0]
    mb = pm[0].contiguous()

    def all_ops():
        return [ops.trimul(layer.tri_mul_out, x, mb, True), ops.trimul(layer.tri_mul_in, x, mb, False),
                ops.triattn(layer.tri_att_start, x, mb, True), ops.triattn(layer.tri_att_end, x, mb, False),
                ops.pair_transition(layer.transition_z, x)]

    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
        torch.cuda.manual_seed(1)
        want = layer(s, z, mask, pm)
        want_ops = all_ops()
        torch.cuda.synchronize()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            torch.cuda.manual_seed(1)
            got = layer(s, z, mask, pm)
            got_ops = all_ops()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
    assert all(torch.equal(a, b) for a, b in zip(got, want))
    assert all(torch.equal(a, b) for a, b in zip(got_ops, want_ops))


@pytest.mark.parametrize("inference_params", [False, True])
def test_weight_packs_follow_in_place_updates(gpu, inference_params):
    """Every cached bf16 pack is rebuilt after an in-place parameter update:
    the fused modules then equal freshly built ones (for parameters made
    under inference mode, which carry no version counter, nothing is cached)."""
    torch.manual_seed(12)
    if inference_params:
        with torch.inference_mode():
            lay = R.randomize(R.PairformerLayer()).to(gpu).eval()
    else:
        lay = R.randomize(R.PairformerLayer()).to(gpu).eval()
    x = torch.randn(70, 70, 128, device=gpu)
    mb = torch.ones(70, 70, device=gpu)
    mods = ("tri_mul_out", "tri_att_start", "transition_z")

    def run(lay_):
        return [ops.trimul(lay_.tri_mul_out, x, mb, True), ops.triattn(lay_.tri_att_start, x, mb, True),
                ops.pair_transition(lay_.transition_z, x)]

    with torch.inference_mode():
        before = run(lay)
        for name in mods:
            for p in getattr(lay, name).parameters():
                p.mul_(0.75).add_(0.01)
        after = run(lay)
    fresh = R.PairformerLayer().to(gpu).eval()
    with torch.no_grad():
        for name in mods:
            for p_new, p in zip(getattr(fresh, name).parameters(), getattr(lay, name).parameters()):
                p_new.copy_(p)
    with torch.inference_mode():
        want = run(fresh)
    for a, b, w in zip(before, after, want):
        assert not torch.equal(a, b)
        assert torch.equal(b, w)


def test_grad_fallback_trimul_and_transition_equal_gradients(gpu):
    torch.manual_seed(13)
    host = nn.Module()
    host.layer = R.randomize(R.PairformerLayer()).to(gpu).eval()
    adapters.install(host, require_boltz2=False)
    lay = host.layer
    x = (torch.randn(1, 9, 9, 128, device=gpu) * 0.5).requires_grad_(True)
    mask = torch.ones(1, 9, 9, device=gpu)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        for mod, call in ((lay.tri_mul_out, lambda m, f: f(m, x, mask)), (lay.tri_mul_in, lambda m, f: f(m, x, mask)),
                          (lay.transition_z, lambda m, f: f(m, x))):
            got = call(mod, lambda m, *a: m(*a))
            g_got = torch.autograd.grad(got.float().square().sum(), x)[0]
            want = call(mod, lambda m, *a: type(m).forward(m, *a))
            g_want = torch.autograd.grad(want.float().square().sum(), x)[0]
            assert torch.equal(got, want) and torch.equal(g_got, g_want), type(mod).__name__


@pytest.mark.parametrize("module", ["trimul", "triattn_start", "triattn_end"])
def test_row_scale_is_exact(gpu, module):
    """``row_scale`` multiplies the bf16 module output of each frame row before
    the residual add: equal, bit for bit, to the unscaled bf16 output scaled
    and added in fp32 (frame rows are z's columns for the ending node)."""
    torch.manual_seed(14)
    lay = R.randomize(R.PairformerLayer()).to(gpu).eval()
    n = 77
    x = torch.randn(n, n, 128, device=gpu)
    mb = torch.ones(n, n, device=gpu)
    mb[-3:, :] = 0
    mb[:, -3:] = 0
    scale = torch.ones(n, device=gpu)
    scale[[0, 9, 40]] = 0
    scale[[3, 70]] = 0.5
    scale[11] = 2.0
    with torch.inference_mode():
        if module == "trimul":
            y = ops.trimul(lay.tri_mul_in, x, mb, False)
            got = ops.trimul(lay.tri_mul_in, x, mb, False, ops.OUT_RESIDUAL, torch.empty_like(x), row_scale=scale)
            acc = x.clone()
            ops.trimul(lay.tri_mul_in, acc, mb, False, ops.OUT_ACCUMULATE, acc, row_scale=scale)
            want = x + scale[:, None, None] * y.float()
        else:
            starting = module == "triattn_start"
            mod = lay.tri_att_start if starting else lay.tri_att_end
            y = ops.triattn(mod, x, mb, starting)
            got = ops.triattn(mod, x, mb, starting, ops.OUT_RESIDUAL, torch.empty_like(x), row_scale=scale)
            acc = x.clone()
            ops.triattn(mod, acc, mb, starting, ops.OUT_ACCUMULATE, acc, row_scale=scale)
            sc = scale[:, None, None] if starting else scale[None, :, None]
            want = x + sc * y.float()
    assert torch.equal(got, want) and torch.equal(acc, want)
