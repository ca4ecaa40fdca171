"""Triangle attention forwards patched onto Boltz modules.

Reference: src/boltz_lumi/triangle.py (contiguous_mask_chunk :18-22,
ordered_triangle_forward :32-104, normalization_forward :107-146).  Here the
whole ``TriangleAttention.forward`` is replaced: LayerNorm, the q/k/v/gate/
triangle-bias projections, the attention and the output projection run in
the three fused gfx950 kernels, so the ``[I, H, N, N]`` scores are never
materialised and ``chunk_size`` needs no chunk loop.  Every forward falls back
to the module's own class forward when a guard fails, as the reference does.
"""

from __future__ import annotations

import torch

from . import ops
from ._guards import autocast_off, bf16_autocast, fp32_contiguous_on, gfx950_tensor, inference


def _native_shape_ok(module, x) -> bool:
    return (
        getattr(module, "c_in", None) == 128
        and getattr(module, "c_hidden", None) == 32
        and getattr(module, "no_heads", None) == 4
        and x.ndim == 4
        and x.shape[1] == x.shape[2]
        and x.shape[-1] == 128
        and x.shape[1] <= 8192
    )


# fp32 mode holds at most this many bytes per pair at its peak (``ops.triattn_fp32``:
# the [N^2, 576] fp32 projection, the split-bf16 attention's K / V workspace,
# the attention output and the linear_o result), all N rows at once.  Measured
# at N = 1024: 3860-3864 bytes per pair by default, 3088-3604 with exact fp32
# linears (tests/test_gpu_fp32_triattn.py); the bound keeps a margin.
FP32_BYTES_PER_PAIR = 4608
# ... and runs in one pass while that fits in this share of the device memory
# (N up to about 5500 on a 288 GiB MI355X).  Larger N run in blocks of frame
# rows, which hold the output frame, the triangle bias and the mask (this many
# bytes per pair) for the whole frame and the rest for one block at a time.
FP32_MEMORY_SHARE = 0.45
FP32_FRAME_BYTES_PER_PAIR = 532


def fp32_native_fits(n: int, device_bytes: int) -> bool:
    """Whether fp32-mode triangle attention at size ``n`` runs in one pass on
    a device of ``device_bytes`` (its working set within ``FP32_MEMORY_SHARE``)."""
    return FP32_BYTES_PER_PAIR * n * n <= FP32_MEMORY_SHARE * device_bytes


def fp32_block_rows(n: int, device_bytes: int) -> int:
    """Frame rows per block for fp32-mode triangle attention at size ``n``:
    ``n`` when one pass fits, otherwise the most rows whose working set fits
    beside the full-frame output, bias and mask; 0 when not one row fits."""
    if fp32_native_fits(n, device_bytes):
        return n
    budget = FP32_MEMORY_SHARE * device_bytes - FP32_FRAME_BYTES_PER_PAIR * n * n
    return max(0, min(n, int(budget // (FP32_BYTES_PER_PAIR * n))))


def triangle_attention_forward(self, x, mask=None, chunk_size=None, use_kernels=False):
    """Drop-in for ``TriangleAttention{,EndingNode}.forward(x, mask, chunk_size, use_kernels)``.

    Native in inference under bf16 autocast (or for bf16 x), with a bf16
    result like the upstream autocast path; and in fp32 mode (autocast off,
    fp32 x; reference triangle.py:38-52), with an fp32 result
    (``ops.triattn_fp32``): by default one split-bf16 GEMM of
    LayerNorm-without-affine(x) for q | k | v | g and the triangle bias (the
    LayerNorm affine folded into the weights) and the fused split-bf16
    attention, about 2^-16 relative per product; with
    ``BMX_EXACT_FP32_LINEARS=1`` the fp32 LN128 kernel, fp32 GEMMs and the
    fp32-MFMA attention.  fp32 mode runs all N rows in one pass while that
    working set fits (``fp32_native_fits``) and in blocks of rows above
    (``fp32_block_rows``); only a device on which not one row fits takes the
    class forward, which chunks the rows."""
    base = (
        not use_kernels
        and inference(self)
        and gfx950_tensor(x)
        and _native_shape_ok(self, x)
        and (mask is None or tuple(mask.shape) == tuple(x.shape[:-1]))
    )
    starting = getattr(self, "starting", True)
    if base and autocast_off() and x.dtype == torch.float32 and self.layer_norm.weight.dtype == torch.float32:
        rows = fp32_block_rows(x.shape[1], torch.cuda.get_device_properties(x.device).total_memory)
        if rows == 0:
            return type(self).forward(self, x, mask, chunk_size=chunk_size, use_kernels=use_kernels)
        outs = [ops.triattn_fp32(self, x[b], None if mask is None else mask[b], starting, block_rows=rows)
                for b in range(x.shape[0])]
        # one batch element: its result as a view (the ending node's is a transposed one, as upstream's)
        return outs[0].unsqueeze(0) if len(outs) == 1 else torch.stack(outs)
    supported = base and (bf16_autocast() or x.dtype == torch.bfloat16) and x.dtype in (torch.float32, torch.bfloat16)
    if not supported:
        return type(self).forward(self, x, mask, chunk_size=chunk_size, use_kernels=use_kernels)
    out = torch.empty(x.shape, device=x.device, dtype=torch.bfloat16)
    ws = ops.new_workspace(x.shape[1], x.device)
    for b in range(x.shape[0]):
        mb = None if mask is None else mask[b].to(torch.float32).contiguous()
        ops.triattn(self, x[b].contiguous(), mb, starting, ops.OUT_BF16, out[b], ws)
    return out


def normalization_forward(module, x):
    """Drop-in for the triangle ``LayerNorm.forward`` (c_in (128,)): the
    native LN128 with a bf16 result under bf16 autocast (the next op casts to
    bf16 anyway; reference triangle.py:133-145)."""
    eligible = (
        inference(module)
        and gfx950_tensor(x)
        and x.dtype == torch.float32
        and x.shape[-1] == 128
        and getattr(module, "c_in", None) == (128,)
        and fp32_contiguous_on(x.device, module.weight, module.bias)
        and bf16_autocast()
    )
    if not eligible:
        return type(module).forward(module, x)
    flat = x.contiguous().reshape(-1, 128)
    return ops.norm(flat, module.weight, module.bias, module.eps, False, bf16_output=True).reshape(x.shape)


def contiguous_mask_chunk(self, x, tri_bias, mask_bias, mask, chunk_size, use_kernels=False):
    """Ending-node ``_chunk`` with a dense ``mask_bias`` (reference triangle.py:18-22)."""
    if x.shape[-3] > 384:  # upstream const.chunk_size_threshold
        mask_bias = mask_bias.contiguous()
    # The patch is an instance attribute; the class attribute is upstream's.
    return type(self)._chunk(self, x, tri_bias, mask_bias, mask, chunk_size, use_kernels)
