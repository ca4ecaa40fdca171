"""CPU tests of the drop-in boundary: install gating, idempotency, fallback to
the upstream forward (values and gradients), uninstall, and the conditioning
cache's restore-on-exception (reference tests/test_operator_additions.py:97-105,
139-147 and tests/test_atom_conditioning.py:106-111)."""

from types import SimpleNamespace

import pytest
import torch
from torch import nn

import boltz_lumi_amd
from boltz_lumi_amd import adapters
from boltz_lumi_amd.atom_conditioning import atom_conditioning_cache
from oracle import boltz_ref as R


class AtomDiffusion(nn.Module):
    """Stand-in for the structure module: ``sample`` records its keyword arguments."""

    def __init__(self):
        super().__init__()
        self.score_model = nn.Module()
        self.score_model.block = R.ConditionedTransitionBlock(16, 8)
        self.score_model.token_transformer = nn.Module()
        self.score_model.token_transformer.layers = nn.ModuleList([R.DiffusionTransformerLayer(2, 48, 8)])

    def sample(self, *args, **kwargs):
        self.seen = kwargs
        return "sampled"


class Boltz2(nn.Module):
    """Stand-in with the module paths adapters.install walks."""

    def __init__(self):
        super().__init__()
        self.pairformer_module = nn.Module()
        self.pairformer_module.layers = nn.ModuleList([R.PairformerLayer(token_s=32, token_z=128, num_heads=4)])
        self.structure_module = AtomDiffusion()


def test_version_pin():
    assert boltz_lumi_amd.SUPPORTED_BOLTZ_VERSION == "2.2.1"
    assert boltz_lumi_amd.__version__.startswith("2.2.1.")


def test_install_requires_boltz2_and_gfx950():
    assert adapters.install(nn.Linear(2, 2)) == 0
    model = Boltz2()
    if not torch.cuda.is_available():
        assert adapters.install(model) == 0  # no gfx950 device: no-op
        assert not getattr(model, adapters.FLAG, False)


def test_install_patches_by_class_and_path_and_is_idempotent():
    model = Boltz2()
    n = adapters.install(model, require_device=False)
    # the Pairformer layer and its tri_mul_out, tri_mul_in, tri_att_start, tri_att_end, transition_z; score
    # model: block (CTB) and its AdaLN, the token-transformer layer itself, its AdaLN, AttentionPairBias, CTB
    # and its AdaLN; structure_module.sample
    assert n == 14
    layer = model.pairformer_module.layers[0]
    assert "forward" in vars(layer)  # the fused composition (pairformer.pairformer_layer_forward)
    assert "forward" in vars(layer.tri_att_start) and "forward" in vars(layer.tri_att_start.layer_norm)
    assert "forward" in vars(layer.transition_z) and "forward" not in vars(layer.transition_s)
    assert "forward" not in vars(layer.attention)  # the trunk's AttentionPairBias stays upstream
    token_layer = model.structure_module.score_model.token_transformer.layers[0]
    assert "forward" in vars(token_layer.pair_bias_attn) and "sample" in vars(model.structure_module)
    assert "forward" in vars(token_layer)
    assert adapters.install(model, require_device=False) == 0
    assert adapters.uninstall(model) >= 14
    assert "forward" not in vars(layer.tri_att_start) and "sample" not in vars(model.structure_module)
    assert "forward" not in vars(layer)


def test_prepare_token_bias_keeps_values_and_packs_each_layer_densely():
    from boltz_lumi_amd.pair_bias import prepare_token_bias

    g = torch.Generator().manual_seed(4)
    bias = torch.randn(2, 5, 7, 3 * 4, generator=g)  # [B, Q, K, layers * heads]
    packed = prepare_token_bias(bias)
    assert packed.shape == bias.shape and packed.dtype == torch.float32 and torch.equal(packed, bias)
    for layer in range(3):
        per_layer = packed[..., 4 * layer:4 * (layer + 1)].movedim(-1, 1)  # upstream proj_z (Rearrange)
        assert all(per_layer[b].is_contiguous() for b in range(2))
    assert torch.equal(prepare_token_bias(bias.bfloat16()), bias.bfloat16().float())


def test_sample_wrapper_packs_the_token_bias_and_passes_through_under_grad():
    model = Boltz2().eval()
    adapters.install(model, require_device=False)
    sm = model.structure_module
    bias = torch.randn(1, 4, 4, 6)
    cond = {"token_trans_bias": bias, "c": torch.zeros(2, 3)}
    with torch.no_grad():
        assert sm.sample(diffusion_conditioning=cond, multiplicity=2) == "sampled"
    seen = sm.seen["diffusion_conditioning"]["token_trans_bias"]
    assert torch.equal(seen, bias) and seen.movedim(-1, 1)[0].is_contiguous()
    assert cond["token_trans_bias"] is bias  # the caller's dict is not modified
    assert sm.sample(diffusion_conditioning=cond, multiplicity=2) == "sampled"  # grad on: untouched
    assert sm.seen["diffusion_conditioning"] is cond


def test_cpu_tensors_fall_back_to_upstream_exactly():
    torch.manual_seed(0)
    model = Boltz2()
    R.randomize(model)
    layer = model.pairformer_module.layers[0]
    n = 6
    z = torch.randn(1, n, n, 128)
    s = torch.randn(1, n, 32)
    mask = torch.ones(1, n)
    mask[:, -1] = 0
    pm = mask[:, :, None] * mask[:, None, :]
    for training in (False, True):  # in training the dropout masks are live: same seed, same draws
        model.train(training)
        adapters.uninstall(model)
        with torch.no_grad():
            torch.manual_seed(7)
            want = layer(s, z, mask, pm)
            adapters.install(model, require_device=False)
            torch.manual_seed(7)
            got = layer(s, z, mask, pm)
        assert all(torch.equal(a, b) for a, b in zip(got, want))


def test_grad_mode_falls_back_with_equal_gradients():
    torch.manual_seed(1)
    tm = R.randomize(R.TriangleMultiplicationOutgoing(128))
    x = torch.randn(1, 3, 3, 128, requires_grad=True)
    mask = torch.ones(1, 3, 3)
    want = tm(x, mask)
    gw = torch.autograd.grad(want.sum(), x)[0]
    from boltz_lumi_amd.multiplication import normalized_forward

    got = normalized_forward(tm, x, mask)
    gg = torch.autograd.grad(got.sum(), x)[0]
    assert torch.equal(got, want) and torch.equal(gg, gw)


def test_conditioning_cache_restores_forwards_after_exception():
    layers = [R.DiffusionTransformerLayer(2, 16, 8) for _ in range(2)]
    score = SimpleNamespace(
        atom_attention_encoder=SimpleNamespace(atom_encoder=SimpleNamespace(
            diffusion_transformer=SimpleNamespace(layers=layers[:1]))),
        atom_attention_decoder=SimpleNamespace(atom_decoder=SimpleNamespace(
            diffusion_transformer=SimpleNamespace(layers=layers[1:]))),
    )
    before = [vars(m).get("forward") for m in (layers[0].adaln.s_norm, layers[1].transition.output_projection[0])]
    with pytest.raises(RuntimeError, match="boom"):
        with atom_conditioning_cache(score):
            assert "forward" in vars(layers[0].adaln.s_norm)
            raise RuntimeError("boom")
    after = [vars(m).get("forward") for m in (layers[0].adaln.s_norm, layers[1].transition.output_projection[0])]
    assert before == after == [None, None]


def test_conditioning_cache_is_inert_on_cpu():
    layer = R.DiffusionTransformerLayer(2, 16, 8)
    score = SimpleNamespace(
        atom_attention_encoder=SimpleNamespace(atom_encoder=SimpleNamespace(
            diffusion_transformer=SimpleNamespace(layers=[layer]))),
        atom_attention_decoder=SimpleNamespace(atom_decoder=SimpleNamespace(
            diffusion_transformer=SimpleNamespace(layers=[]))),
    )
    calls = []
    original = layer.adaln.s_norm.forward

    def counting(x):
        calls.append(1)
        return original(x)

    layer.adaln.s_norm.forward = counting
    s = torch.randn(3, 8)
    with torch.no_grad(), atom_conditioning_cache(score):
        layer.adaln.s_norm(s)
        layer.adaln.s_norm(s)
    assert len(calls) == 2  # CPU inputs are never cached
    assert layer.adaln.s_norm.forward is counting


def test_msa_template_and_confidence_stacks_are_patched_by_class_and_suffix():
    """The reference selects pair modules by class name anywhere in the model
    and transitions by the ``.transition_z`` suffix (adapters.py:24-45), so
    the MSA, template and confidence stacks are patched like the trunk; the
    MSA module's own ``msa_transition`` is not.  On CPU every patched forward
    falls back to the upstream one bit for bit."""
    model = nn.Module()
    model.msa_module = nn.Module()
    msa_layer = nn.Module()
    msa_layer.pairformer_layer = R.PairformerNoSeqLayer(16, pairwise_head_width=8, pairwise_num_heads=2)
    msa_layer.msa_transition = R.Transition(8, 32)
    model.msa_module.layers = nn.ModuleList([msa_layer])
    model.template_module = nn.Module()
    model.template_module.pairformer = nn.Module()
    model.template_module.pairformer.layers = nn.ModuleList(
        [R.PairformerNoSeqLayer(8, pairwise_head_width=8, pairwise_num_heads=2)])
    model.confidence_module = nn.Module()
    model.confidence_module.pairformer_stack = nn.Module()
    model.confidence_module.pairformer_stack.layers = nn.ModuleList(
        [R.PairformerLayer(token_s=32, token_z=16, num_heads=4, pairwise_head_width=8, pairwise_num_heads=2)])
    R.randomize(model, generator=torch.Generator().manual_seed(3)).eval()
    z = torch.randn(2, 6, 6, 8)
    pm = torch.ones(2, 6, 6)
    pm[:, -1] = 0
    template = model.template_module.pairformer.layers[0]
    with torch.inference_mode():
        want = template(z, pm)
    # 15 pair modules and the three layers (MSA and template PairformerNoSeqLayer, confidence PairformerLayer)
    assert adapters.install(model, require_boltz2=False, require_device=False) == 18
    assert "forward" in vars(msa_layer.pairformer_layer) and "forward" in vars(template)
    assert "forward" in vars(msa_layer.pairformer_layer.transition_z)
    assert "forward" not in vars(msa_layer.msa_transition)
    with torch.inference_mode():
        assert torch.equal(template(z, pm), want)
    adapters.uninstall(model)


def test_window_probe_on_cpu():
    """The to_keys probe that gates the atom transformer's addressed key
    windows: upstream's single_to_keys partial passes with offset (W - H) / 2;
    another window layout, or a to_keys of another shape, does not."""
    import functools

    from boltz_lumi_amd.diffusion import window_key_offset

    n, w, h = 6 * 32, 32, 128
    index = R.get_indexing_matrix(n // w, w, h)
    good = functools.partial(R.single_to_keys, indexing_matrix=index, w=w, h=h)
    assert window_key_offset(good, n, w, h, "cpu") == -48
    assert window_key_offset(functools.partial(R.single_to_keys, indexing_matrix=index.flip(0), w=w, h=h),
                             n, w, h, "cpu") is None
    assert window_key_offset(lambda x: torch.zeros(1, n // w, h - 1, 1), n, w, h, "cpu") is None


def test_split_bf16_threshold_follows_width_and_rows():
    """fp32 linears run split-bf16 from 512 input channels (the token
    transformer), or from 128 with at least 16384 rows (the atom transformer's
    5 x 8192 atoms) when their operand is shared or they have 512+ outputs;
    never for widths that are not multiples of 4 or in exact fp32 mode; the
    Pairformer sequence stack's 1024 rows of 384 stay fp32."""
    from boltz_lumi_amd import ops

    assert ops.use_split(768) and ops.use_split(768, 10) and ops.use_split(1536, 5120)
    assert ops.use_split(128, 40960) and ops.use_split(256, 16384) and ops.use_split(128, 40960, 512)
    assert not ops.use_split(128, 40960, 128) and not ops.use_split(256, 40960, 256) and ops.use_split(768, 64, 128)
    assert not ops.use_split(384, 1024) and not ops.use_split(128, 512) and not ops.use_split(128)
    assert not ops.use_split(64, 10 ** 6) and not ops.use_split(770, 5120)
    before = ops.exact_fp32_linears(True)
    try:
        assert not ops.use_split(768, 5120) and not ops.use_split(128, 40960)
    finally:
        ops.exact_fp32_linears(before)


def test_fp32_triangle_attention_one_pass_or_row_blocks_by_working_set():
    """fp32-mode triangle attention holds up to 4.6 KB per pair for all N rows
    at once: one pass up to about N = 5300 on a 288 GB MI355X; above, blocks
    of frame rows whose working set fits beside the full-frame output, bias
    and mask (532 bytes per pair), e.g. at the kernels' N = 8192 limit; the
    class forward only where not one row fits."""
    from boltz_lumi_amd.triangle import (FP32_BYTES_PER_PAIR, FP32_FRAME_BYTES_PER_PAIR, FP32_MEMORY_SHARE,
                                         fp32_block_rows, fp32_native_fits)

    mi355x = 288 * 1024 ** 3
    assert fp32_native_fits(1024, mi355x) and fp32_native_fits(4096, mi355x) and fp32_native_fits(5300, mi355x)
    assert not fp32_native_fits(6500, mi355x) and not fp32_native_fits(8192, mi355x)
    assert not fp32_native_fits(4096, 64 * 1024 ** 3)  # a smaller device caps earlier
    assert FP32_BYTES_PER_PAIR * 8192 ** 2 > 288e9  # all rows at once would not fit at N = 8192
    assert fp32_block_rows(5300, mi355x) == 5300
    for n in (6500, 8192):
        rows = fp32_block_rows(n, mi355x)
        assert 0 < rows < n
        held = FP32_FRAME_BYTES_PER_PAIR * n * n + FP32_BYTES_PER_PAIR * rows * n
        assert held <= FP32_MEMORY_SHARE * mi355x < held + FP32_BYTES_PER_PAIR * n  # the most rows that fit
    assert fp32_block_rows(8192, 96 * 1024 ** 3) > 0
    assert fp32_block_rows(8192, 64 * 1024 ** 3) == 0  # the frame alone would not fit: class forward


@pytest.mark.parametrize("training", [False, True])
@pytest.mark.parametrize("columnwise", [False, True])
def test_dropout_masks_match_upstream_draws(training, columnwise):
    """The installed layer's dropout masks (one in-place comparison in eval)
    are upstream's get_dropout_mask values, dtype and shape, and leave the
    generator where upstream's leave it."""
    from boltz_lumi_amd import pairformer

    layer = SimpleNamespace(dropout=0.25, training=training)
    z = torch.randn(2, 37, 37, 128)
    torch.manual_seed(5)
    got = pairformer.dropout_mask(layer, z, columnwise)
    state_got = torch.get_rng_state()
    torch.manual_seed(5)
    want = R.get_dropout_mask(0.25, z, training, columnwise)
    assert got.dtype == want.dtype and got.shape == want.shape
    assert torch.equal(got, want)
    assert torch.equal(state_got, torch.get_rng_state())
