"""GPU tests of the drop-in boundary: after ``install``, the stand-in Boltz
modules (oracle classes with Boltz names and parameters) run the native
kernels under bf16 autocast and match the upstream fp32 math within the north
star's 2e-2; in fp32 mode triangle attention runs natively within 1e-4 and
the other pair modules fall back to the upstream forward bit for bit, as does
grad mode; the diffusion blocks run natively in fp32 within 1e-4; the
conditioning cache computes each projection once."""

import copy
from types import SimpleNamespace

import pytest
import torch
from torch import nn

from boltz_lumi_amd import adapters, diffusion, ops
from boltz_lumi_amd.atom_conditioning import atom_conditioning_cache
from oracle import boltz_ref as R

pytestmark = pytest.mark.gpu


class Boltz2(nn.Module):
    def __init__(self):
        super().__init__()
        self.pairformer_module = nn.Module()
        self.pairformer_module.layers = nn.ModuleList([R.PairformerLayer()])
        self.structure_module = nn.Module()
        self.structure_module.score_model = nn.Module()
        sm = self.structure_module.score_model
        sm.adaln = R.AdaLN(768, 768)
        sm.transition = R.ConditionedTransitionBlock(128, 128)


def max_rel(got, want):
    got, want = got.double(), want.double()
    return ((got - want).abs().max() / want.abs().max()).item()


@pytest.fixture()
def model(gpu):
    torch.manual_seed(732991)
    m = R.randomize(Boltz2()).to(gpu).eval()
    yield m
    adapters.uninstall(m)


def test_install_on_gfx950(model):
    assert adapters.install(model) == 9  # the Pairformer layer, its 5 pair modules, AdaLN, CTB and its AdaLN


@pytest.mark.parametrize("n", [7, 17, 64, 117, 312, 576])  # the reference test's sizes (tests/test_operator_additions.py)
def test_patched_pair_modules_match_upstream(model, gpu, n):
    layer = model.pairformer_module.layers[0]
    x = torch.randn(1, n, n, 128, device=gpu) * 0.3
    mask = torch.ones(1, n, n, device=gpu)
    mask[:, -3:, :] = 0
    mask[:, :, -3:] = 0
    calls = {
        "tri_mul_out": lambda m: m(x, mask),
        "tri_mul_in": lambda m: m(x, mask),
        "tri_att_start": lambda m: m(x, mask, chunk_size=32),
        "tri_att_end": lambda m: m(x, mask, chunk_size=32),
        "transition_z": lambda m: m(x),
    }
    with torch.inference_mode():
        want = {k: f(getattr(layer, k)) for k, f in calls.items()}  # upstream fp32
    assert adapters.install(model) == 9  # the Pairformer layer, its 5 pair modules, AdaLN, CTB and its AdaLN
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
        for k, f in calls.items():
            got = f(getattr(layer, k))
            assert got.dtype == torch.bfloat16, k
            assert max_rel(got, want[k]) < 2e-2, k
    with torch.inference_mode():  # fp32 mode
        for k, f in calls.items():
            got = f(getattr(layer, k))
            if k.startswith("tri_att"):  # native fp32 attention: the north star's fp32 bar
                assert got.dtype == torch.float32 and max_rel(got, want[k]) < 1e-4, k
            else:  # upstream math, bit for bit
                assert torch.equal(got, want[k]), k


@pytest.mark.parametrize("n", [17, 117, 312, 576])
def test_patched_transition_dense_and_strided_input(model, gpu, n):
    """The installed pair transition on a dense x and on the strided view
    x[:, ::2] (the reference test's two layouts) against upstream's fp32
    forward on the same input."""
    layer = model.pairformer_module.layers[0]
    x = torch.randn(1, n, n, 128, device=gpu) * 0.3
    for inp in (x, x[:, ::2]):
        with torch.inference_mode():
            want = layer.transition_z(inp)
        assert adapters.install(model) == 9
        with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
            got = layer.transition_z(inp)
        adapters.uninstall(model)
        assert got.shape == inp.shape and got.dtype == torch.bfloat16
        assert max_rel(got, want) < 2e-2


@pytest.mark.parametrize("n", [1134, 2511])
def test_patched_triangle_attention_at_the_reference_token_counts(model, gpu, n):
    """The installed triangle attention, both nodes, at the token counts the
    reference publishes (partial mask: the last 3 tokens), against upstream's
    fp32 forward on the same GPU (chunk 32, as the reference test)."""
    layer = model.pairformer_module.layers[0]
    g = torch.Generator(device=gpu).manual_seed(n)
    x = torch.randn(1, n, n, 128, device=gpu, generator=g) * 0.3
    mask = torch.ones(1, n, n, device=gpu)
    mask[:, -3:, :] = 0
    mask[:, :, -3:] = 0
    print(f"installed triangle attention n={n}", flush=True)
    for name in ("tri_att_start", "tri_att_end"):
        mod = getattr(layer, name)
        with torch.inference_mode():
            want = mod(x, mask, chunk_size=32)  # upstream fp32 (not installed yet)
        assert adapters.install(model) == 9
        with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
            got = mod(x, mask, chunk_size=32)
        adapters.uninstall(model)
        assert got.dtype == torch.bfloat16 and torch.isfinite(got).all(), name
        assert max_rel(got, want) < 2e-2, name
        del want, got


def test_grad_mode_falls_back(model, gpu):
    adapters.install(model)
    layer = model.pairformer_module.layers[0]
    x = torch.randn(1, 5, 5, 128, device=gpu, requires_grad=True)
    mask = torch.ones(1, 5, 5, device=gpu)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        got = layer.tri_att_start(x, mask)
        g_got = torch.autograd.grad(got.float().sum(), x)[0]
        want = type(layer.tri_att_start).forward(layer.tri_att_start, x, mask)
        g_want = torch.autograd.grad(want.float().sum(), x)[0]
    assert torch.equal(got, want) and torch.equal(g_got, g_want)


def test_diffusion_blocks_native_fp32(model, gpu):
    sm = model.structure_module.score_model
    a, s = torch.randn(2, 300, 768, device=gpu), torch.randn(2, 300, 768, device=gpu)
    a2, s2 = torch.randn(5, 500, 128, device=gpu), torch.randn(5, 500, 128, device=gpu)
    with torch.inference_mode():
        want1, want2 = sm.adaln(a, s), sm.transition(a2, s2)
    adapters.install(model)
    assert "forward" in vars(sm.adaln)
    with torch.inference_mode():
        assert max_rel(sm.adaln(a, s), want1) < 1e-4
        assert max_rel(sm.transition(a2, s2), want2) < 1e-4


def test_conditioning_cache_computes_once(gpu):
    torch.manual_seed(317)
    layers = [R.randomize(R.DiffusionTransformerLayer(4, 32, 32), std=0.07).to(gpu).eval() for _ in range(4)]
    score = SimpleNamespace(
        atom_attention_encoder=SimpleNamespace(atom_encoder=SimpleNamespace(
            diffusion_transformer=SimpleNamespace(layers=layers[:2]))),
        atom_attention_decoder=SimpleNamespace(atom_decoder=SimpleNamespace(
            diffusion_transformer=SimpleNamespace(layers=layers[2:]))),
    )
    s = torch.randn(2, 17, 32, device=gpu)
    bias = torch.randn(2, 17, 17, 4, device=gpu)
    mask = torch.ones(2, 17, device=gpu)
    mask[:, -3:] = 0
    acts = [torch.randn(2, 17, 32, device=gpu) for _ in range(3)]
    with torch.inference_mode():
        want = [[layer(a, s, bias, mask) for layer in layers] for a in acts]
    calls = []
    norm = layers[0].adaln.s_norm
    original = norm.forward
    norm.forward = lambda x: (calls.append(1), original(x))[1]
    with torch.inference_mode(), atom_conditioning_cache(score):
        got = [[layer(a, s, bias, mask) for layer in layers] for a in acts]
    assert len(calls) == 1
    for gw, ww in zip(got, want):
        for g_, w_ in zip(gw, ww):
            assert torch.equal(g_, w_)


def test_conditioning_cache_recomputes_per_context_and_stays_off_under_autocast_or_grad(gpu):
    """A new cache context computes the projections again; under bf16 autocast
    or with grad enabled the cache does not memoise (every call computes),
    and the results equal the uncached layer's (the reference's cases,
    tests/test_atom_conditioning.py:100-130)."""
    torch.manual_seed(99)
    layers = [R.randomize(R.DiffusionTransformerLayer(4, 32, 32), std=0.07).to(gpu).eval() for _ in range(2)]
    score = SimpleNamespace(
        atom_attention_encoder=SimpleNamespace(atom_encoder=SimpleNamespace(
            diffusion_transformer=SimpleNamespace(layers=layers[:1]))),
        atom_attention_decoder=SimpleNamespace(atom_decoder=SimpleNamespace(
            diffusion_transformer=SimpleNamespace(layers=layers[1:]))),
    )
    s = torch.randn(1, 17, 32, device=gpu)
    bias = torch.randn(1, 17, 17, 4, device=gpu)
    mask = torch.ones(1, 17, device=gpu)
    a = torch.randn(1, 17, 32, device=gpu)
    calls = []
    norm = layers[0].adaln.s_norm
    original = norm.forward
    norm.forward = lambda x: (calls.append(1), original(x))[1]
    with torch.inference_mode():
        want = layers[0](a, s, bias, mask)
        for _ in range(2):  # two contexts, two calls each: one computation per context
            with atom_conditioning_cache(score):
                for _ in range(2):
                    assert torch.equal(layers[0](a, s, bias, mask), want)
    assert len(calls) == 1 + 2
    calls.clear()
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16), atom_conditioning_cache(score):
        for _ in range(2):
            layers[0](a, s, bias, mask)
    assert len(calls) == 2  # not memoised under autocast
    calls.clear()
    with torch.enable_grad(), atom_conditioning_cache(score):
        for _ in range(2):
            got = layers[0](a, s, bias, mask)
    assert len(calls) == 2  # not memoised with grad
    assert torch.equal(got.detach(), want)


def test_diffusion_widths_off_the_kernels_fall_back(gpu):
    """The fused epilogues take widths that are multiples of 4: a block of
    another width runs its class forward, bit for bit, instead of raising."""
    from boltz_lumi_amd.diffusion import adaln_forward, transition_forward

    ctb = R.randomize(R.ConditionedTransitionBlock(6, 8), generator=torch.Generator().manual_seed(3)).to(gpu).eval()
    a, s = torch.randn(2, 5, 6, device=gpu), torch.randn(2, 5, 8, device=gpu)
    with torch.inference_mode():
        assert torch.equal(transition_forward(ctb, a, s), type(ctb).forward(ctb, a, s))
        assert torch.equal(adaln_forward(ctb.adaln, a, s), type(ctb.adaln).forward(ctb.adaln, a, s))


@pytest.mark.parametrize("width,heads,n,windows", [(768, 16, 300, False), (128, 4, 256, True)])
def test_diffusion_layer_fused_gates_match_upstream(gpu, width, heads, n, windows):
    """An installed DiffusionTransformerLayer (token shape, and atom shape
    with 32-query windows over 128 to_keys rows) fuses both output gates with
    their residual adds and matches the fp32 upstream layer within 1e-4; with a
    forward hook on its transition the layer calls ``a + transition(a, s)``
    instead, with the same result."""
    torch.manual_seed(41 + width)
    ref = R.randomize(R.DiffusionTransformerLayer(heads, width, width), std=0.05).to(gpu).eval()
    host = nn.Module()
    host.structure_module = nn.Module()
    host.structure_module.score_model = nn.Module()
    host.structure_module.score_model.layer = R.DiffusionTransformerLayer(heads, width, width).to(gpu).eval()
    layer = host.structure_module.score_model.layer
    layer.load_state_dict(ref.state_dict())
    assert adapters.install(host, require_boltz2=False) >= 5  # the layer, its AdaLNs, attention, transition
    assert "forward" in vars(layer)
    g = torch.Generator().manual_seed(5)
    a = torch.randn(2, n, width, generator=g).to(gpu)
    s = torch.randn(2, n, width, generator=g).to(gpu)
    mask = torch.ones(2, n, device=gpu)
    mask[:, -7:] = 0
    if windows:  # as the atom transformer calls its layers: [B * N / W, W, D] windows over to_keys rows
        nw, w, h = n // 32, 32, 128
        index = R.get_indexing_matrix(nw, w, h, device=gpu)

        def to_keys(x):
            return R.single_to_keys(x.view(2, nw * w, -1), index, w, h).view(2 * nw, h, -1)

        a, s, mask = a.view(2 * nw, w, width), s.view(2 * nw, w, width), mask.view(2 * nw, w)
        bias = torch.randn(2 * nw, w, h, heads, generator=g).to(gpu)
    else:
        to_keys = None
        bias = torch.randn(2, n, n, heads, generator=g).to(gpu)
    with torch.inference_mode():
        want = ref(a, s, bias, mask, to_keys)
        got = layer(a, s, bias, mask, to_keys)
        handle = layer.transition.register_forward_hook(lambda *args: None)
        try:
            hooked = layer(a, s, bias, mask, to_keys)
        finally:
            handle.remove()
    assert max_rel(got, want) < 1e-4
    assert max_rel(hooked, want) < 1e-4
    adapters.uninstall(host)


@pytest.mark.parametrize("width,heads,n,windows", [(768, 16, 300, False), (128, 4, 256, True)])
def test_diffusion_stack_shared_conditioning_matches_upstream(gpu, width, heads, n, windows):
    """An installed DiffusionTransformer (3 layers; token shape, and atom shape
    with windows over to_keys rows) builds the operands of s once and runs each
    layer's six conditioning projections as two GEMMs with the s_norm affine
    folded into the weights; it matches the fp32 upstream stack within 1e-4.
    Covered on the way: an s_norm with a bias (folded as W b), a layer whose
    s_scale has an instance forward (a memo: that layer calls its projections
    one by one), exact fp32 linears at the token width, and at the token width
    the chained layer boundaries (bit for bit the unchained stack)."""
    torch.manual_seed(43 + width)
    depth = 3
    ref = R.DiffusionTransformer(depth, heads, width, width)
    ref.layers[1].adaln.s_norm = nn.LayerNorm(width)  # affine with a bias
    ref = R.randomize(ref, std=0.05).to(gpu).eval()
    host = nn.Module()
    host.structure_module = nn.Module()
    host.structure_module.score_model = nn.Module()
    host.structure_module.score_model.stack = copy.deepcopy(ref)
    stack = host.structure_module.score_model.stack
    assert adapters.install(host, require_boltz2=False) == 5 * depth + 1
    assert "forward" in vars(stack)
    g = torch.Generator().manual_seed(9)
    a = torch.randn(2, n, width, generator=g).to(gpu)
    s = torch.randn(2, n, width, generator=g).to(gpu)
    mask = torch.ones(2, n, device=gpu)
    mask[:, -5:] = 0
    if windows:
        nw, w, h = n // 32, 32, 128
        index = R.get_indexing_matrix(nw, w, h, device=gpu)

        def to_keys(x):
            return R.single_to_keys(x.view(2, nw * w, -1), index, w, h).view(2 * nw, h, -1)

        a, s, mask = a.view(2 * nw, w, width), s.view(2 * nw, w, width), mask.view(2 * nw, w)
        bias = torch.randn(2 * nw, w, h, depth * heads, generator=g).to(gpu)
    else:
        to_keys = None
        bias = torch.randn(2, n, n, depth * heads, generator=g).to(gpu)
    calls = []
    real = ops.layernorm_split3 if width >= ops.X3_MIN_K else ops.layer_norm
    name = "layernorm_split3" if width >= ops.X3_MIN_K else "layer_norm"
    with torch.inference_mode():
        want = ref(a, s, bias, mask, to_keys)
        with pytest.MonkeyPatch.context() as mp:
            mp.setattr(ops, name, lambda *args: calls.append(1) or real(*args))
            got = stack(a, s, bias, mask, to_keys)
        lin = stack.layers[2].adaln.s_scale
        lin.forward = lambda x, f=type(lin).forward, m=lin: f(m, x)  # an instance forward, as a memo installs
        try:
            memo = stack(a, s, bias, mask, to_keys)
        finally:
            del lin.forward
        if width >= ops.X3_MIN_K:
            before = ops.exact_fp32_linears(True)
            try:
                exact = stack(a, s, bias, mask, to_keys)
            finally:
                ops.exact_fp32_linears(before)
            assert max_rel(exact, want) < 1e-5
    assert len(calls) == 1  # LayerNorm(s) once for the three layers
    assert max_rel(got, want) < 1e-4
    assert max_rel(memo, want) < 1e-4
    if not windows:  # token layers chain their boundaries: layer i's last pass writes layer i + 1's operand
        fused = []
        real_f = ops.gated_residual_adaln_split3
        with torch.inference_mode(), pytest.MonkeyPatch.context() as mp:
            mp.setattr(ops, "gated_residual_adaln_split3", lambda *args, **kw: fused.append(1) or real_f(*args, **kw))
            chained = stack(a, s, bias, mask, to_keys)
            n_chained = len(fused)
            mp.setattr(diffusion, "_operand_path", lambda *args, **kw: False)
            unchained = stack(a, s, bias, mask, to_keys)
        assert n_chained == 2 * depth - 1 and len(fused) - n_chained == depth
        assert torch.equal(chained, unchained) and torch.equal(chained, got)
    adapters.uninstall(host)
