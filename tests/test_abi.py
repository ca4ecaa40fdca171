"""CPU checks of the C ABI: the library loads and exports every symbol that
include/bmx.h declares, and argument validation fails loudly without a GPU
(no kernel is launched by these tests)."""

import ctypes
import re
from pathlib import Path

import pytest

from boltz_lumi_amd import _native as N

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    text = (ROOT / "include" / "bmx.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(bmx_\w+)\(", text, re.M)))


def test_header_matches_binding_table():
    assert declared_symbols() == sorted(N.SIGNATURES)


def test_every_entry_point_is_documented():
    """Each declaration's comment names the reference interface it replaces
    (a file:line citation) or says it has no reference counterpart, and the
    integration guide's ABI table lists it."""
    text = (ROOT / "include" / "bmx.h").read_text()
    guide = (ROOT / "INTEGRATION.md").read_text()
    decl = re.compile(r"(/\*(?:(?!\*/).)*\*/)\s*((?:(?:int|size_t|const char\*)\s+bmx_\w+\([^;]*;\s*)+)", re.S)
    seen = set()
    for m in decl.finditer(text):
        comment = " ".join(m.group(1).split())
        names = re.findall(r"(bmx_\w+)\(", m.group(2))
        cited = re.search(r"\.(py|cu|hip):\d", comment) or "no reference counterpart" in comment.lower() \
            or "no counterpart in the reference" in comment.lower() or "no reference kernel" in comment.lower()
        for name in names:
            seen.add(name)
            assert cited, f"{name}: its comment cites no reference interface: {comment[:120]}"
            assert re.search(rf"\b{name}\b", guide), f"{name} is missing from the integration guide's ABI table"
    assert seen == set(declared_symbols())


@pytest.fixture(scope="module")
def lib():
    if not N.lib_path().exists():
        pytest.skip("libbmx.so not built")
    return N.lib()


def test_library_exports_every_declared_symbol(lib):
    for name in declared_symbols():
        assert hasattr(lib, name), name
    assert lib.bmx_abi_version() == 2


def test_workspace_queries(lib):
    assert lib.bmx_trimul_workspace_bytes(0) == 0
    assert lib.bmx_trimul_workspace_bytes(1024) == 3 * 128 * 1024 * 1024 * 2
    assert lib.bmx_trimul_workspace_bytes(100) == 3 * 128 * 256 * 256 * 2  # planes padded to 256
    assert lib.bmx_triattn_workspace_bytes(1024) > 3 * 1024 * 1024 * 128 * 2
    assert lib.bmx_triattn_proj_rows() == 3 * 128 + 32
    # split K (hi, lo) and split V^T (hi, lo), keys padded to the 64-key stage: 5 x 1024 x 768 -> 4 x 7.5 MiB
    # K hi / lo and V^T hi / lo (bf16, keys padded to 64, 256-byte aligned) and the fp32 mask terms
    assert lib.bmx_seq_attention_x3_workspace_bytes(5, 1024, 16, 48) == 4 * 5 * 1024 * 768 * 2 + 5 * 1024 * 4
    assert lib.bmx_seq_attention_x3_workspace_bytes(1, 17, 4, 32) == 4 * 64 * 128 * 2 + 64 * 4
    assert lib.bmx_seq_attention_x3_workspace_bytes(0, 17, 4, 32) == 0


def test_argument_validation_needs_no_gpu(lib):
    # Rejected before any launch: bad dtype code, bad out_mode, empty input.
    rc = lib.bmx_layernorm128(None, 7, 0, None, None, 1e-5, None, 0, 4, None)
    assert rc == N.BMX_EINVAL and b"dtypes" in lib.bmx_last_error()
    rc = lib.bmx_trimul_fwd(None, None, 4, 1, None, None, 1e-5, None, None, None, 1e-5, None, None, None, 9, None, None,
                            0, 7, None)
    assert rc == N.BMX_EINVAL and b"out_mode" in lib.bmx_last_error()
    rc = lib.bmx_trimul_fwd(None, None, 4, 1, None, None, 1e-5, None, None, None, 1e-5, None, None, None, 0, None, None,
                            0, 7, None)
    assert rc == N.BMX_EINVAL and b"null pointer" in lib.bmx_last_error()
    rc = lib.bmx_trimul_fwd(None, None, 4, 1, None, None, 1e-5, None, None, None, 1e-5, None, None, None, 0, None, None,
                            0, 8, None)
    assert rc == N.BMX_EINVAL and b"stages" in lib.bmx_last_error()
    assert lib.bmx_gate(None, None, None, 0, None) == N.BMX_OK
    rc = lib.bmx_diffusion_epilogue(2, None, None, None, None, 0, 1, 4, None)
    assert rc == N.BMX_EINVAL and b"kind" in lib.bmx_last_error()
    rc = lib.bmx_triattn_fwd(None, 0, None, 8, 1, 1e9, None, None, 1e-5, None, None, None, None, None, None, 0,
                             None, None, 0, 7, None)
    assert rc == N.BMX_EINVAL and b"null pointer" in lib.bmx_last_error()
    rc = lib.bmx_pair_transition_fwd(None, 1, 8, None, None, 1e-5, None, None, None, 2, None)
    assert rc == N.BMX_EINVAL and b"residual" in lib.bmx_last_error()
    rc = lib.bmx_pack_mfma_weights(None, 48, 128, None, None)
    assert rc == N.BMX_EINVAL and b"multiple of 32" in lib.bmx_last_error()
    rc = lib.bmx_pack_mfma_weights(None, 32, 128, None, None)
    assert rc == N.BMX_EINVAL and b"null pointer" in lib.bmx_last_error()
    assert lib.bmx_pack_mfma_weights(None, 0, 128, None, None) == N.BMX_OK
    rc = N.lib().bmx_pair_transition_bias_fwd(None, 0, 8, None, None, ctypes.c_float(1e-5), None, None, None, 0,
                                              None, ctypes.c_float(1e-5), None, None)
    assert rc == N.BMX_EINVAL and b"out_mode" in lib.bmx_last_error()
    rc = lib.bmx_pair_bias_fold(None, None, None, 8, None, None)
    assert rc == N.BMX_EINVAL and b"16 heads" in lib.bmx_last_error()
    rc = lib.bmx_seq_attention_fwd(None, None, None, None, None, None, 8, 100, 16, 24, 1e6, None, None)
    assert rc == N.BMX_EINVAL and b"row stride" in lib.bmx_last_error()
    assert lib.bmx_pair_bias_fold_bytes() == 2 * 4 * 64 * 8 * 2 + 16 * 4
    # the split attention checks its workspace before anything is launched
    fake = ctypes.c_void_p(256)
    args = [fake] * 6 + [1, 16, 1024, 768, 768, 0, 0, 0, 0, 1, 16, 48, 1e6, fake]
    rc = lib.bmx_seq_attention_x3_batched_fwd(*args, fake, 1024, None)
    assert rc == N.BMX_EINVAL and b"workspace" in lib.bmx_last_error()
    rc = lib.bmx_seq_attention_x3_batched_fwd(*args[:17], 40, 1e6, fake, fake, 1 << 30, None)
    assert rc == N.BMX_EINVAL and b"head_dim" in lib.bmx_last_error()
    assert lib.bmx_seq_attention_x3_batched_fwd(*args[:6], 0, *args[7:], None, 0, None) == N.BMX_OK
    rc = lib.bmx_seq_attention_x3_batched_split_fwd(*args[:19], ctypes.c_void_p(264), fake, 1 << 30, None)
    assert rc == N.BMX_EINVAL and b"out_op must be 16-byte aligned" in lib.bmx_last_error()
    # split-bf16 operand writers and the strided modulation kernels
    assert lib.bmx_split3_bf16(None, 0, 768, 768, None, None) == N.BMX_OK
    rc = lib.bmx_split3_bf16(fake, 4, 768, 700, fake, None)
    assert rc == N.BMX_EINVAL and b"ldx >= k" in lib.bmx_last_error()
    rc = lib.bmx_layernorm_split3_bf16(fake, 4, 1028, 1028, ctypes.c_float(1e-5), fake, None)
    assert rc == N.BMX_EINVAL and b"dim <= 1024" in lib.bmx_last_error()
    assert lib.bmx_layernorm_split3_t_bf16(None, 0, 128, 128, ctypes.c_float(1e-5), None, None) == N.BMX_OK
    rc = lib.bmx_layernorm_split3_t_bf16(fake, 1 << 16, 128, 128, ctypes.c_float(1e-5), fake, None)
    assert rc == N.BMX_EINVAL and b"n must be < 65536" in lib.bmx_last_error()
    rc = lib.bmx_adaln_split3_bf16(fake, fake, fake, 512, 4, 768, ctypes.c_float(1e-5), fake, None)
    assert rc == N.BMX_EINVAL and b"ld_mod >= dim" in lib.bmx_last_error()
    rc = lib.bmx_adaln_split3_bf16(fake, ctypes.c_void_p(260), fake, 768, 4, 768, ctypes.c_float(1e-5), fake, None)
    assert rc == N.BMX_EINVAL and b"aligned" in lib.bmx_last_error()
    rc = lib.bmx_swiglu_split3_bf16(fake, 2000, 4, 768, fake, None)
    assert rc == N.BMX_EINVAL and b"ldu >= 3 cols" in lib.bmx_last_error()
    rc = lib.bmx_adaln_strided(fake, fake, fake, 100, fake, 0, 4, 128, ctypes.c_float(1e-5), None)
    assert rc == N.BMX_EINVAL and b"ld_mod" in lib.bmx_last_error()
    rc = lib.bmx_gated_residual(fake, fake, 768, None, fake, 4, 768, None)
    assert rc == N.BMX_EINVAL and b"null pointer" in lib.bmx_last_error()
    rc = lib.bmx_gated_residual_adaln_split3_bf16(fake, fake, 700, fake, fake, fake, fake, 768, 4, 768,
                                                  ctypes.c_float(1e-5), fake, None)
    assert rc == N.BMX_EINVAL and b"ld_gate" in lib.bmx_last_error()
    # windowed attention: the windows must tile the batch and see their own queries
    wargs = [fake] * 6 + [10, 32, 128, 512, 512, 4, -48, 8, 0, 0, 1, 1536, 12]
    rc = lib.bmx_seq_attention_windowed_fwd(*wargs, 4, 32, ctypes.c_float(1e6), fake, None)
    assert rc == N.BMX_EINVAL and b"dividing batch" in lib.bmx_last_error()
    wargs[6], wargs[12] = 8, -120
    rc = lib.bmx_seq_attention_windowed_fwd(*wargs, 4, 32, ctypes.c_float(1e6), fake, None)
    assert rc == N.BMX_EINVAL and b"own queries" in lib.bmx_last_error()
    wargs[12], wargs[13] = -48, 6
    rc = lib.bmx_seq_attention_windowed_fwd(*wargs, 4, 32, ctypes.c_float(1e6), fake, None)
    assert rc == N.BMX_EINVAL and b"bias_group" in lib.bmx_last_error()
    wargs[6], wargs[13] = 0, 8
    assert lib.bmx_seq_attention_windowed_fwd(*wargs, 4, 32, ctypes.c_float(1e6), fake, None) == N.BMX_OK


def test_operator_set_entry_points_reject_bad_arguments(lib):
    # The reference's unfused operator set (gate / split / pack / silu_mul / bias softmax) and the
    # stand-alone pair bias: every rejection happens before a launch.
    fake, odd = ctypes.c_void_p(256), ctypes.c_void_p(264)  # 16-byte aligned / only 8-byte aligned
    assert lib.bmx_silu_mul(None, None, None, 0, None) == N.BMX_OK  # empty input: nothing to do
    rc = lib.bmx_silu_mul(None, fake, fake, 64, None)
    assert rc == N.BMX_EINVAL and b"null pointer" in lib.bmx_last_error()
    rc = lib.bmx_trimul_split(fake, fake, fake, fake, fake, 4, 384, None)
    assert rc == N.BMX_EINVAL and b"row stride must be 256 or 512" in lib.bmx_last_error()
    rc = lib.bmx_trimul_split(fake, fake, fake, odd, fake, 4, 256, None)
    assert rc == N.BMX_EINVAL and b"16-byte aligned" in lib.bmx_last_error()
    rc = lib.bmx_trimul_pack(fake, fake, fake, fake, fake, -1, 256, 1, None)
    assert rc == N.BMX_EINVAL and b"bad n" in lib.bmx_last_error()
    rc = lib.bmx_trimul_pack(odd, fake, fake, fake, fake, 8, 512, 0, None)
    assert rc == N.BMX_EINVAL and b"p and g must be 16-byte aligned" in lib.bmx_last_error()
    shape = (ctypes.c_int64 * 5)(1, 1, 4, 4, 4097)
    strides = (ctypes.c_int64 * 5)(0, 0, 0, 4097, 1)
    rc = lib.bmx_bias_softmax(fake, fake, fake, fake, 0, shape, strides, strides, strides, None)
    assert rc == N.BMX_EINVAL and b"at most 4096 keys" in lib.bmx_last_error()
    rc = lib.bmx_bias_softmax(fake, fake, fake, fake, 2, shape, strides, strides, strides, None)
    assert rc == N.BMX_EINVAL and b"dtype must be fp32 or bf16" in lib.bmx_last_error()
    shape[4] = 64
    rc = lib.bmx_bias_softmax(fake, None, fake, fake, 1, shape, strides, strides, strides, None)
    assert rc == N.BMX_EINVAL and b"null pointer" in lib.bmx_last_error()
    rc = lib.bmx_pair_bias_fwd(fake, 0, 4, fake, fake, ctypes.c_float(1e-5), fake, 8, fake, None)
    assert rc == N.BMX_EINVAL and b"16 heads" in lib.bmx_last_error()
    rc = lib.bmx_pair_bias_fwd(odd, 0, 4, fake, fake, ctypes.c_float(1e-5), fake, 16, fake, None)
    assert rc == N.BMX_EINVAL and b"z must be 16-byte aligned" in lib.bmx_last_error()


def test_call_raises_with_message(lib):
    with pytest.raises(N.BmxError, match="eps must be positive"):
        N.call("bmx_layernorm", None, None, None, 0.0, None, 0, 1, 4, None)
