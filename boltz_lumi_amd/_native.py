"""ctypes binding of libbmx.so (the gfx950 C ABI declared in include/bmx.h).

The library is built ahead of time (``python -m boltz_lumi_amd.build``) and
loaded once per process.  ``torch`` is imported first so that the HIP runtime
torch ships (soname ``libamdhip64.so.7``) is the one the library binds to:
device pointers and streams from torch are then valid inside the library.

A missing library is an error, never a silent fallback.
"""

from __future__ import annotations

import ctypes
from ctypes import c_float, c_int, c_int64, c_size_t, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("libbmx.so")

BMX_OK, BMX_EINVAL, BMX_EUNSUPPORTED, BMX_ELAUNCH = 0, 1, 2, 3
F32, BF16 = 0, 1

_P = c_void_p
_I64P = ctypes.POINTER(c_int64)

# name -> (restype, argtypes); mirrors include/bmx.h
SIGNATURES = {
    "bmx_last_error": (ctypes.c_char_p, []),
    "bmx_abi_version": (c_int, []),
    "bmx_layernorm128": (c_int, [_P, c_int, c_int, _P, _P, c_float, _P, c_int, c_int64, _P]),
    "bmx_layernorm": (c_int, [_P, _P, _P, c_float, _P, c_int, c_int64, c_int, _P]),
    "bmx_adaln": (c_int, [_P, _P, _P, _P, c_int, c_int64, c_int, c_float, _P]),
    "bmx_gate": (c_int, [_P, _P, _P, c_int64, _P]),
    "bmx_trimul_split": (c_int, [_P, _P, _P, _P, _P, c_int64, c_int, _P]),
    "bmx_trimul_pack": (c_int, [_P, _P, _P, _P, _P, c_int64, c_int, c_int, _P]),
    "bmx_silu_mul": (c_int, [_P, _P, _P, c_int64, _P]),
    "bmx_split3_bf16": (c_int, [_P, c_int64, c_int64, c_int64, _P, _P]),
    "bmx_layernorm_split3_bf16": (c_int, [_P, c_int64, c_int, c_int64, c_float, _P, _P]),
    "bmx_layernorm_split3_t_bf16": (c_int, [_P, c_int64, c_int, c_int64, c_float, _P, _P]),
    "bmx_adaln_split3_bf16": (c_int, [_P, _P, _P, c_int64, c_int64, c_int, c_float, _P, _P]),
    "bmx_swiglu_split3_bf16": (c_int, [_P, c_int64, c_int64, c_int64, _P, _P]),
    "bmx_gated_residual_adaln_split3_bf16": (c_int, [_P, _P, c_int64, _P, _P, _P, _P, c_int64, c_int64, c_int, c_float,
                                                     _P, _P]),
    "bmx_adaln_strided": (c_int, [_P, _P, _P, c_int64, _P, c_int, c_int64, c_int, c_float, _P]),
    "bmx_gated_residual": (c_int, [_P, _P, c_int64, _P, _P, c_int64, c_int64, _P]),
    "bmx_diffusion_epilogue": (c_int, [c_int, _P, _P, _P, _P, c_int, c_int64, c_int64, _P]),
    "bmx_bias_softmax": (c_int, [_P, _P, _P, _P, c_int, _I64P, _I64P, _I64P, _I64P, _P]),
    "bmx_trimul_workspace_bytes": (c_size_t, [c_int64]),
    "bmx_trimul_fwd": (c_int, [_P, _P, c_int64, c_int, _P, _P, c_float, _P, _P, _P, c_float, _P, _P, _P, c_int, _P,
                               _P, c_size_t, c_int, _P]),
    "bmx_trimul_fwd_noalloc": (c_int, [_P, _P, c_int64, c_int, _P, _P, c_float, _P, _P, _P, c_float, _P, _P, _P,
                                       c_int, _P]),
    "bmx_triattn_workspace_bytes": (c_size_t, [c_int64]),
    "bmx_triattn_proj_rows": (c_int, []),
    "bmx_triattn_fwd": (c_int, [_P, c_int, _P, c_int64, c_int, c_float, _P, _P, c_float, _P, _P, _P, _P, _P, _P, c_int,
                                _P, _P, c_size_t, c_int, _P]),
    "bmx_pack_mfma_weights": (c_int, [_P, c_int64, c_int64, _P, _P]),
    "bmx_pair_transition_fwd": (c_int, [_P, c_int, c_int64, _P, _P, c_float, _P, _P, _P, c_int, _P]),
    "bmx_pair_bias_fwd": (c_int, [_P, c_int, c_int64, _P, _P, c_float, _P, c_int, _P, _P]),
    "bmx_pair_bias_fold_bytes": (c_size_t, []),
    "bmx_pair_bias_fold": (c_int, [_P, _P, _P, c_int, _P, _P]),
    "bmx_pair_transition_bias_fwd": (c_int, [_P, c_int, c_int64, _P, _P, c_float, _P, _P, _P, c_int, _P, c_float, _P,
                                             _P]),
    "bmx_seq_attention_fwd": (c_int, [_P, _P, _P, _P, _P, _P, c_int64, c_int64, c_int, c_int, c_float, _P, _P]),
    "bmx_seq_attention_batched_fwd": (c_int, [_P, _P, _P, _P, _P, _P] + [c_int64] * 10 + [c_int, c_int, c_float, _P, _P]),
    "bmx_seq_attention_windowed_fwd": (c_int, [_P, _P, _P, _P, _P, _P] + [c_int64] * 13
                                       + [c_int, c_int, c_float, _P, _P]),
    "bmx_seq_attention_x3_workspace_bytes": (c_size_t, [c_int64, c_int64, c_int, c_int]),
    "bmx_seq_attention_x3_batched_fwd": (c_int, [_P, _P, _P, _P, _P, _P] + [c_int64] * 10
                                         + [c_int, c_int, c_float, _P, _P, c_size_t, _P]),
    "bmx_seq_attention_x3_batched_split_fwd": (c_int, [_P, _P, _P, _P, _P, _P] + [c_int64] * 10
                                               + [c_int, c_int, c_float, _P, _P, c_size_t, _P]),
}


class BmxError(RuntimeError):
    """A libbmx entry point rejected its arguments or failed to launch."""


_lib = None


def lib_path() -> Path:
    return LIB_PATH


def lib():
    """Load (once) and return the library; raises if it has not been built."""
    global _lib
    if _lib is None:
        import torch  # noqa: F401  -- bind torch's HIP runtime first

        if not LIB_PATH.exists():
            raise BmxError(f"{LIB_PATH} is missing: build it with `python -m boltz_lumi_amd.build`")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def last_error() -> str:
    msg = lib().bmx_last_error()
    return msg.decode() if msg else ""


def call(name: str, *args) -> None:
    """Call a status-returning entry point; raise BmxError on failure."""
    rc = getattr(lib(), name)(*args)
    if rc != BMX_OK:
        raise BmxError(f"{name} failed ({rc}): {last_error()}")


def int64_array(values):
    arr = (c_int64 * len(values))(*[int(v) for v in values])
    return arr
