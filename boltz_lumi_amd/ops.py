"""Torch-facing wrappers of the libbmx C ABI.

Two groups:

* the reference's native operator set, same names and argument meaning as
  the reference's extension functions (``norm``, ``gate``, ``split``,
  ``pack``, ``silu_mul``, ``epilogue``, ``ordered_softmax``), each raising
  ``RuntimeError`` on bad input like the reference's ``TORCH_CHECK``s;
* the fused hot-path modules (``trimul``, ``triattn``, ``pair_transition``,
  ``adaln``) that take a module with Boltz's parameter names.

Every call launches on torch's current stream of the input's device, allocates
outputs and workspaces through torch's caching allocator and never
synchronises.  There is no fallback: without the built library every call
raises.
"""

from __future__ import annotations

import os

import torch

from . import _native as N

C = 128

# ---------------------------------------------------------------- helpers


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _code(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return N.F32
    if dtype == torch.bfloat16:
        return N.BF16
    raise RuntimeError(f"unsupported dtype {dtype}; expected float32 or bfloat16")


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _cuda(*tensors: torch.Tensor) -> None:
    dev = tensors[0].device
    for t in tensors:
        _check(t.is_cuda, "expected CUDA (HIP) tensors")
        _check(t.device == dev, "all tensors must be on the same device")


def _inference_only() -> None:
    _check(not torch.is_grad_enabled(), "Inference only")


def cached_weight(module, name: str, sources, build):
    """Derived weight (e.g. a bf16 concatenation) cached on ``module``.

    Reused only while every source parameter keeps its identity, version
    counter, storage, device and dtype (the rule of the reference's joint
    projection cache, multiplication.py:29-40, plus the storage address, which
    a ``param.data = ...`` swap changes).  Inference tensors (parameters made
    or loaded under ``torch.inference_mode``) carry no version counter, so an
    in-place update of one cannot be seen: with such a source the weight is
    rebuilt on every call and never cached."""
    if any(p.is_inference() for p in sources):
        with torch.no_grad():
            return build(*sources).contiguous()
    key = tuple((id(p), p._version, p.data_ptr(), p.device, p.dtype) for p in sources)
    cache = module.__dict__.setdefault("_bmx_weight_cache", {})
    hit = cache.get(name)
    if hit is None or hit[0] != key:
        with torch.no_grad():
            value = build(*sources).contiguous()
        hit = (key, value)
        cache[name] = hit
    return hit[1]


def _bf16(*ws):
    return torch.cat([w.detach() for w in ws], 0).to(torch.bfloat16)


def _f32(t):
    return t.detach().to(torch.float32).contiguous()


def pack_mfma_weights(w):
    """bf16 copy of the row-major matrix ``w`` in MFMA A-operand order
    (``bmx_pack_mfma_weights``): each 32-row x 16-column operand tile becomes
    one contiguous 1 KB run."""
    _cuda(w)
    w = w.detach().to(torch.bfloat16).contiguous()
    rows, cols = w.shape
    out = torch.empty_like(w)
    N.call("bmx_pack_mfma_weights", w.data_ptr(), rows, cols, out.data_ptr(), _stream(w))
    return out


def _bf16_packed(*ws):
    return pack_mfma_weights(_bf16(*ws))


def _workspace(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


# ------------------------------------------------- reference operator set


def norm(x, weight, bias, eps, channel_first=False, waves=None, rows=None, bf16_output=True):
    """LayerNorm over 128 channels (reference ``multiplication_norm``,
    kernels/multiplication_hip.cu:105-156).  ``waves``/``rows`` were gfx90a
    launch-table knobs and are accepted for signature compatibility only."""
    _cuda(x, weight, bias)
    _check(x.is_contiguous() and weight.is_contiguous() and bias.is_contiguous(), "expected contiguous tensors")
    _check(x.dim() == 2 and (x.size(0) == C if channel_first else x.size(1) == C), "expected 128 channels")
    _check(weight.numel() == C and bias.numel() == C and weight.dtype == torch.float32
           and bias.dtype == torch.float32, "expected fp32 weight/bias of 128 elements")
    _inference_only()
    _check(eps > 0, "eps must be positive")
    m = x.size(1) if channel_first else x.size(0)
    out = torch.empty((m, C), device=x.device, dtype=torch.bfloat16 if bf16_output else torch.float32)
    if m:
        N.call("bmx_layernorm128", x.data_ptr(), _code(x.dtype), int(channel_first), weight.data_ptr(),
               bias.data_ptr(), float(eps), out.data_ptr(), _code(out.dtype), m, _stream(x))
    return out


def layer_norm(x, weight, bias, eps):
    """LayerNorm over the last axis (<= 1024 channels) with optional weight/bias."""
    _cuda(x)
    _check(x.is_contiguous(), "expected a contiguous input")
    d = x.shape[-1]
    out = torch.empty_like(x)
    rows = x.numel() // d if d else 0
    w = None if weight is None else _f32(weight)
    b = None if bias is None else _f32(bias)
    if rows:
        N.call("bmx_layernorm", x.data_ptr(), None if w is None else w.data_ptr(), None if b is None else b.data_ptr(),
               float(eps), out.data_ptr(), _code(x.dtype), rows, d, _stream(x))
    return out


def gate(p, g):
    """``bf16(p * bf16(sigmoid(g)))`` (reference ``multiplication_gate``)."""
    _cuda(p, g)
    _check(p.shape == g.shape, "shape mismatch")
    _check(p.dtype == torch.bfloat16 and g.dtype == torch.bfloat16, "expected bf16 inputs")
    _inference_only()
    _check(p.is_contiguous() and g.is_contiguous(), "expected contiguous tensors")
    out = torch.empty_like(p)
    if p.numel():
        N.call("bmx_gate", p.data_ptr(), g.data_ptr(), out.data_ptr(), p.numel(), _stream(p))
    return out


def _check_projection(p, g, mask):
    _cuda(p, g, mask)
    _check(p.shape == g.shape and p.dtype == torch.bfloat16 and g.dtype == torch.bfloat16, "expected bf16 p, g")
    _inference_only()
    _check(p.dim() == 4 and p.size(0) == 1 and p.size(1) == p.size(2) and p.size(3) == 2 * C,
           "expected [1, N, N, 256] projections")
    s = p.stride()
    _check(s[3] == 1 and s[2] in (2 * C, 4 * C) and s[1] == p.size(2) * s[2] and g.stride() == s,
           "Expected dense or joint-projection rows")
    _check(mask.dtype == torch.float32 and mask.is_contiguous() and mask.numel() * 2 * C == p.numel(),
           "expected an fp32 contiguous [1, N, N] mask")
    return s[2]


def split(p, g, mask):
    """Gate and mask into channel-last a, b (reference ``multiplication_gate_split``)."""
    stride = _check_projection(p, g, mask)
    n = p.size(1)
    a = torch.empty((1, n, n, C), device=p.device, dtype=torch.bfloat16)
    b = torch.empty_like(a)
    if n:
        N.call("bmx_trimul_split", p.data_ptr(), g.data_ptr(), mask.data_ptr(), a.data_ptr(), b.data_ptr(), n * n,
               stride, _stream(p))
    return a, b


def pack(p, g, mask, outgoing, channels_per_tile=None):
    """Gate, mask and channel-major operand layout (reference ``multiplication_gate_pack``)."""
    stride = _check_projection(p, g, mask)
    n = p.size(1)
    a = torch.empty((C, n, n), device=p.device, dtype=torch.bfloat16)
    b = torch.empty_like(a)
    if n:
        N.call("bmx_trimul_pack", p.data_ptr(), g.data_ptr(), mask.data_ptr(), a.data_ptr(), b.data_ptr(), n, stride,
               int(bool(outgoing)), _stream(p))
    return a, b


def silu_mul(a, b):
    """``bf16(bf16(silu(a)) * b)`` (reference ``pair_silu_mul``)."""
    _cuda(a, b)
    _check(a.shape == b.shape, "shape mismatch")
    _check(a.dtype == torch.bfloat16 and b.dtype == torch.bfloat16 and a.is_contiguous() and b.is_contiguous(),
           "expected contiguous bf16 inputs")
    _check(not a.requires_grad and not b.requires_grad, "Inference only")
    out = torch.empty_like(a)
    if a.numel():
        N.call("bmx_silu_mul", a.data_ptr(), b.data_ptr(), out.data_ptr(), a.numel(), _stream(a))
    return out


SPLIT_TAIL = 64  # operand columns past 3 k: two ones that meet the split bias, then zeros


def split_width(k: int) -> int:
    """Columns of a split-bf16 operand row for ``k`` input channels."""
    return 3 * k + SPLIT_TAIL


def _row_stride(t) -> int:
    """Element stride between consecutive rows of ``t`` (last axis dense, the
    leading axes collapsing to one row index), e.g. a column slice of a wider
    projection; raises otherwise."""
    _check(t.dim() >= 1 and (t.shape[-1] <= 1 or t.stride(-1) == 1), "the last axis must be dense")
    lead = [(t.shape[i], t.stride(i)) for i in range(t.dim() - 1) if t.shape[i] != 1]
    if not lead:
        return max(t.shape[-1], 1)
    for (_, outer), (n, inner) in zip(lead, lead[1:]):
        _check(outer == inner * n, "the leading axes must collapse to one row index")
    return lead[-1][1]


def _split_out(x, k):
    return torch.empty(x.shape[:-1] + (split_width(k),), device=x.device, dtype=torch.bfloat16)


def split3(x):
    """Split-bf16 operand of fp32 ``x`` (``bmx_split3_bf16``): bf16 [..., 3 k + 64],
    rows [bf16(x) | bf16(x) | bf16(x - bf16(x)) | 1 1 0 ... 0].  ``x`` may be a
    column slice (rows at a stride)."""
    _cuda(x)
    _check(x.dtype == torch.float32 and x.shape[-1] % 4 == 0 and x.shape[-1] > 0,
           "expected fp32 x with a positive multiple of 4 columns")
    k = x.shape[-1]
    out = _split_out(x, k)
    rows = x.numel() // k
    if rows:
        N.call("bmx_split3_bf16", x.data_ptr(), rows, k, _row_stride(x), out.data_ptr(), _stream(x))
    return out


def layernorm_split3(x, eps):
    """Split-bf16 operand of LayerNorm-without-affine(x) (``bmx_layernorm_split3_bf16``)."""
    _cuda(x)
    _check(x.dtype == torch.float32 and 0 < x.shape[-1] <= 1024 and x.shape[-1] % 4 == 0,
           "expected fp32 x with a multiple of 4 columns, at most 1024")
    k = x.shape[-1]
    out = _split_out(x, k)
    rows = x.numel() // k
    if rows:
        N.call("bmx_layernorm_split3_bf16", x.data_ptr(), rows, k, _row_stride(x), float(eps), out.data_ptr(),
               _stream(x))
    return out


def layernorm_split3_t(x, eps):
    """``layernorm_split3`` of the rows of ``x.transpose(0, 1)`` for a square
    pair frame x [N, N, k] with dense rows, without the transposed copy
    (``bmx_layernorm_split3_t_bf16``); bf16 [N, N, 3 k + 64]."""
    _cuda(x)
    _check(x.dim() == 3 and x.shape[0] == x.shape[1] and x.dtype == torch.float32 and x.is_contiguous()
           and 0 < x.shape[-1] <= 1024 and x.shape[-1] % 4 == 0,
           "expected contiguous fp32 x [N, N, k] with a multiple of 4 columns, at most 1024")
    n, k = x.shape[0], x.shape[-1]
    out = _split_out(x, k)
    if n:
        N.call("bmx_layernorm_split3_t_bf16", x.data_ptr(), n, k, k, float(eps), out.data_ptr(), _stream(x))
    return out


def _same_rows(a, *mods):
    """Row stride shared by ``mods`` (column slices of one projection, or dense
    tensors of a's shape)."""
    _check(all(m.shape == a.shape and m.dtype == a.dtype and m.device == a.device for m in mods),
           "shape/dtype mismatch")
    lds = {_row_stride(m) for m in mods}
    _check(len(lds) == 1, "the modulation operands must share one row stride")
    return lds.pop()


def adaln_split3(a, scale, shift, eps):
    """Split-bf16 operand of ``sigmoid(scale) * LN_noaffine(a) + shift``
    (``bmx_adaln_split3_bf16``); scale and shift may be column slices of one
    wider fp32 projection (rows at one stride)."""
    _cuda(a, scale, shift)
    _check(a.dtype == torch.float32 and a.is_contiguous(), "expected contiguous fp32 a")
    d = a.shape[-1]
    _check(0 < d <= 1024 and d % 4 == 0, "expected a multiple of 4 channels, at most 1024")
    ld = _same_rows(a, scale, shift)
    out = _split_out(a, d)
    rows = a.numel() // d
    if rows:
        N.call("bmx_adaln_split3_bf16", a.data_ptr(), scale.data_ptr(), shift.data_ptr(), ld, rows, d, float(eps),
               out.data_ptr(), _stream(a))
    return out


def gated_residual_adaln_split3(a, gate, c, scale, shift, eps, out=None):
    """``r = c + sigmoid(gate) * a`` (fp32, into ``out``, which may be ``c``) and
    the split-bf16 operand of ``sigmoid(scale) * LN_noaffine(r) + shift`` in one
    pass (``bmx_gated_residual_adaln_split3_bf16``); gate, scale and shift may
    be column slices.  Returns (r, operand)."""
    _cuda(a, gate, c, scale, shift)
    _check(a.dtype == c.dtype == torch.float32 and a.is_contiguous() and c.is_contiguous() and a.shape == c.shape,
           "expected contiguous fp32 a and c of one shape")
    d = a.shape[-1]
    _check(0 < d <= 1024 and d % 4 == 0, "expected a multiple of 4 channels, at most 1024")
    ldg = _same_rows(a, gate)
    ldm = _same_rows(a, scale, shift)
    if out is None:
        out = torch.empty_like(a)
    _check(out.shape == a.shape and out.is_contiguous() and out.dtype == torch.float32, "bad out")
    op = _split_out(a, d)
    rows = a.numel() // d
    if rows:
        N.call("bmx_gated_residual_adaln_split3_bf16", a.data_ptr(), gate.data_ptr(), ldg, c.data_ptr(), out.data_ptr(),
               scale.data_ptr(), shift.data_ptr(), ldm, rows, d, float(eps), op.data_ptr(), _stream(a))
    return out, op


def swiglu_split3(u, cols):
    """Split-bf16 operand of ``silu(g) * x * b`` for rows [x | g | b | ...] of
    fp32 ``u`` (``cols`` values each; ``bmx_swiglu_split3_bf16``)."""
    _cuda(u)
    _check(u.dtype == torch.float32 and cols > 0 and cols % 4 == 0 and u.shape[-1] >= 3 * cols,
           "expected fp32 u with at least 3 cols columns, cols a multiple of 4")
    out = torch.empty(u.shape[:-1] + (split_width(cols),), device=u.device, dtype=torch.bfloat16)
    rows = u.numel() // u.shape[-1]
    if rows:
        N.call("bmx_swiglu_split3_bf16", u.data_ptr(), _row_stride(u), rows, cols, out.data_ptr(), _stream(u))
    return out


def gated_residual(a, gate, c, out=None):
    """``c + sigmoid(gate) * a`` (fp32, ``bmx_gated_residual``; the MODULATION
    epilogue) with ``gate`` possibly a column slice of a wider projection;
    ``out`` may be ``c``."""
    _cuda(a, gate, c)
    _check(a.dtype == gate.dtype == c.dtype == torch.float32, "expected fp32 operands")
    _check(a.is_contiguous() and c.is_contiguous() and a.shape == c.shape == gate.shape, "shape mismatch")
    if out is None:
        out = torch.empty_like(a)
    _check(out.shape == a.shape and out.is_contiguous() and out.dtype == torch.float32, "bad out")
    cols = a.shape[-1]
    rows = a.numel() // cols if cols else 0
    if rows:
        N.call("bmx_gated_residual", a.data_ptr(), gate.data_ptr(), _row_stride(gate), c.data_ptr(), out.data_ptr(),
               rows, cols, _stream(a))
    return out


def _x3_weight(w, b=None):
    """Weight rows [Wh | Wl | Wh | bh bl 0 ... 0] (Wh = bf16(W), Wl = bf16(W - Wh),
    likewise for the bias), bf16 [N, 3 K + 64], for W [N, K] and bias b [N] or None."""
    w = w.detach().float()
    hi = w.to(torch.bfloat16)
    lo = (w - hi.float()).to(torch.bfloat16)
    tail = torch.zeros(w.shape[0], SPLIT_TAIL, device=w.device, dtype=torch.bfloat16)
    if b is not None:
        b = b.detach().float()
        bh = b.to(torch.bfloat16)
        tail[:, 0] = bh
        tail[:, 1] = (b - bh.float()).to(torch.bfloat16)
    return torch.cat([hi, lo, hi, tail], dim=1)


def x3_weight(module, name, weights, biases=None):
    """Split weight of ``mm_split`` for the row concatenation of ``weights``
    ([N_i, K] each) with the biases ``biases`` (one per weight, None for none),
    cached on ``module`` under ``name``."""
    weights = tuple(weights)
    biases = tuple(biases) if biases is not None else (None,) * len(weights)
    _check(len(biases) == len(weights), "one bias (or None) per weight")
    present = tuple(b for b in biases if b is not None)

    def build(*srcs):
        ws = srcs[:len(weights)]
        b = None
        if present:
            it = iter(srcs[len(weights):])
            b = torch.cat([next(it).detach().float() if bb is not None else w.new_zeros(w.shape[0], dtype=torch.float32)
                           for bb, w in zip(biases, ws)])
        return _x3_weight(torch.cat(ws, 0), b)

    return cached_weight(module, name, weights + present, build)


def mm_split(op, w3):
    """``x @ W^T + b`` from the split operand ``op`` of x ([M, 3 K + 64] bf16)
    and ``w3 = x3_weight(..W.., ..b..)``: one hipBLASLt bf16 GEMM with fp32
    accumulation (x W + b up to about 2^-16 relative per product); fp32 [M, N]."""
    _check(op.dim() == 2 and op.shape[1] == w3.shape[1], "operand does not match the split weight")
    return torch.mm(op, w3.t(), out_dtype=torch.float32)


def mm_x3(x, w3):
    """``mm_split(split3(x), w3)`` for fp32 x [M, K]."""
    _check(x.dim() == 2 and w3.shape[1] == split_width(x.shape[1]), "x does not match the split weight")
    return mm_split(split3(x.float()), w3)


# fp32 linears run as split-bf16 GEMMs from 512 input channels up (the token
# transformer's 768 / 1536: ~1.5x faster per block), and from 128 up when
# they are tall (the atom transformer's 5 x 8192 rows at 128 / 256 channels:
# 46.5 against 65.3 us at N = 512, 53 against 89 us at N = 768, 0.23 ms per
# configs[4] step).  Short narrow ones (the Pairformer sequence stack's 1024
# rows of 384) stay on hipBLASLt's fp32 GEMM, and so do tall narrow ones with
# fewer than 512 outputs whose operand needs a split pass of its own (40 960 x
# 128: 12 us for the pass + 27 us against 29 us in fp32 at N = 128).
X3_MIN_K = 512
X3_TALL_MIN_K, X3_TALL_MIN_ROWS, X3_TALL_MIN_N = 128, 16384, 512

# Set BMX_EXACT_FP32_LINEARS=1 (or call exact_fp32_linears(True)) to run every
# fp32 linear of the diffusion blocks and of fp32-mode triangle attention as a
# true fp32 GEMM and fp32-mode attention on fp32 MFMA, as the reference does,
# instead of the split-bf16 form (about 2^-16 relative per product).
_EXACT_FP32 = [os.environ.get("BMX_EXACT_FP32_LINEARS", "0") not in ("", "0")]


def exact_fp32_linears(enabled: bool = True) -> bool:
    """Switch ``linear_fp32`` between the split-bf16 GEMM (False, default) and
    the plain fp32 GEMM (True) for the whole process; returns the previous
    setting."""
    before = _EXACT_FP32[0]
    _EXACT_FP32[0] = bool(enabled)
    return before


def use_split(k: int, rows: int = 0, n: int | None = None) -> bool:
    """Whether fp32 linears of ``k`` input channels over ``rows`` rows run as
    split-bf16 GEMMs (never in exact fp32 mode).  ``n``: the GEMM's outputs
    when its operand is split for it alone (None: a shared split operand)."""
    if _EXACT_FP32[0] or k % 4:
        return False
    return k >= X3_MIN_K or (k >= X3_TALL_MIN_K and rows >= X3_TALL_MIN_ROWS and (n is None or n >= X3_TALL_MIN_N))


def linear_fp32(x, linear):
    """``linear(x)`` for fp32 x: ``linear_x3`` where ``use_split`` says so
    (never with exact fp32 linears switched on), else the fp32 GEMM."""
    if use_split(x.shape[-1], x.numel() // max(x.shape[-1], 1), linear.weight.shape[0]):
        return linear_x3(x, linear)
    return torch.nn.functional.linear(x, linear.weight, linear.bias)


def linear_x3(x, linear):
    """``linear(x)`` for fp32 x through ``mm_x3``, the bias folded into the GEMM."""
    _cuda(x)
    k = x.shape[-1]
    _check(linear.weight.shape[1] == k, "x does not match the linear's input width")
    w = x3_weight(linear, "x3", (linear.weight,), (linear.bias,))
    y = mm_x3(x.reshape(-1, k), w)
    return y.view(x.shape[:-1] + (w.shape[0],))


MODULATION, GATE, GATED_SWIGLU = 0, 1, 3


def epilogue(a, b, c, kind):
    """Diffusion epilogues (reference ``diffusion_epilogue``, op codes diffusion.py:27)."""
    _check(kind in (MODULATION, GATE, GATED_SWIGLU), "unknown epilogue kind")
    _cuda(a, b)
    _check(a.dtype == b.dtype and a.dtype in (torch.float32, torch.bfloat16), "expected fp32 or bf16 inputs")
    _check(a.is_contiguous() and b.is_contiguous(), "expected contiguous inputs")
    shape = list(a.shape)
    cols = shape[-1]
    if kind == GATED_SWIGLU:
        _check(cols % 2 == 0, "SwiGLU input needs an even last dimension")
        cols //= 2
        shape[-1] = cols
    _check(list(b.shape) == shape, "b must match the output shape")
    if kind == MODULATION:
        _check(c is not None and list(c.shape) == shape and c.dtype == a.dtype and c.is_contiguous()
               and c.device == a.device, "MODULATION needs c of the output shape")
    out = torch.empty(shape, device=a.device, dtype=a.dtype)
    n = out.numel()
    if n:
        N.call("bmx_diffusion_epilogue", kind, a.data_ptr(), b.data_ptr(), None if c is None else c.data_ptr(),
               out.data_ptr(), _code(a.dtype), n // cols, cols, _stream(a))
    return out


def ordered_softmax(scores, bias, mask, *, rows=None, waves_per_eu=None, allow_large=False):
    """``softmax(round(round(scores + mask) + bias))`` over keys
    (reference ``ordered_softmax``, kernels/triangle_softmax.py:117-161).
    scores [B,I,H,Q,K], bias [B,1,H,Q,K] (broadcast over I), mask [B,I,1,1,K]."""
    if torch.is_grad_enabled() or scores.dtype not in (torch.float32, torch.bfloat16) or scores.ndim != 5:
        raise ValueError("Expected inference-only FP32/BF16 triangle scores")
    bt, i, h, q, k = scores.shape
    if q <= 0 or k != q:
        raise ValueError("Expected nonempty square score matrices")
    _cuda(scores, bias, mask)
    if bias.dtype != scores.dtype or mask.dtype != torch.float32:
        raise ValueError("bias must match the score dtype and mask must be fp32")
    out = torch.empty(scores.shape, device=scores.device, dtype=scores.dtype)
    N.call("bmx_bias_softmax", scores.data_ptr(), bias.data_ptr(), mask.data_ptr(), out.data_ptr(),
           _code(scores.dtype), N.int64_array(scores.shape), N.int64_array(scores.stride()),
           N.int64_array(bias.stride()), N.int64_array(mask.stride()), _stream(scores))
    return out


# ----------------------------------------------------- fused hot-path ops

# out_mode: write bf16 / write fp32 / out += y (in-place residual) / out = x + y
OUT_BF16, OUT_F32, OUT_ACCUMULATE, OUT_RESIDUAL = 0, 1, 2, 3
ALL_STAGES = 7


def _out_tensor(x, out, out_mode):
    if out_mode == OUT_ACCUMULATE:
        _check(out is not None and out.dtype == torch.float32 and out.shape == x.shape and out.is_contiguous(),
               "accumulate mode needs an fp32 contiguous `out` of x's shape")
        return out
    dtype = torch.bfloat16 if out_mode == OUT_BF16 else torch.float32
    if out is None:
        return torch.empty(x.shape, device=x.device, dtype=dtype)
    _check(out.dtype == dtype and out.shape == x.shape and out.is_contiguous(), "bad `out` tensor")
    if out_mode == OUT_RESIDUAL:
        _check(out.data_ptr() != x.data_ptr(), "residual-write mode needs `out` distinct from x")
    return out


def _row_scale(row_scale, x, n):
    """Checked fp32 [n] row scale (or None) for the fused modules' output kernels."""
    if row_scale is None:
        return None
    _cuda(x, row_scale)
    _check(row_scale.dtype == torch.float32 and row_scale.numel() == n and row_scale.is_contiguous(),
           "expected a contiguous fp32 row scale of n values")
    return row_scale


def trimul(module, x, mask, outgoing, out_mode=OUT_BF16, out=None, workspace=None, stages=ALL_STAGES,
           row_scale=None):
    """Fused TriangleMultiplication{Outgoing,Incoming} for x [N, N, 128] fp32.

    ``stages`` selects the kernels (1 projection, 2 contraction, 4 output);
    separate calls must share ``workspace``.  ``row_scale`` (fp32 [N] or None)
    multiplies output row i (before the residual add): PairformerLayer's
    row-wise dropout mask."""
    _cuda(x, mask)
    _check(x.dim() == 3 and x.size(0) == x.size(1) and x.size(2) == C, "expected x of shape [N, N, 128]")
    _check(x.dtype == torch.float32 and x.is_contiguous(), "expected contiguous fp32 x")
    _check(mask.shape == x.shape[:2] and mask.dtype == torch.float32 and mask.is_contiguous(),
           "expected a contiguous fp32 [N, N] mask")
    n = x.size(0)
    w_in = cached_weight(module, "w_in", (module.p_in.weight, module.g_in.weight), _bf16)
    w_pout = cached_weight(module, "w_pout", (module.p_out.weight,), _bf16)
    w_gout = cached_weight(module, "w_gout", (module.g_out.weight,), _bf16)
    ni, no = module.norm_in, module.norm_out
    niw, nib = cached_weight(module, "ni_w", (ni.weight,), _f32), cached_weight(module, "ni_b", (ni.bias,), _f32)
    now, nob = cached_weight(module, "no_w", (no.weight,), _f32), cached_weight(module, "no_b", (no.bias,), _f32)
    out = _out_tensor(x, out, out_mode)
    rs = _row_scale(row_scale, x, n)
    nbytes = N.lib().bmx_trimul_workspace_bytes(n)
    ws = workspace if workspace is not None and workspace.numel() >= nbytes else _workspace(nbytes, x.device)
    if n:
        N.call("bmx_trimul_fwd", x.data_ptr(), mask.data_ptr(), n, int(bool(outgoing)), niw.data_ptr(),
               nib.data_ptr(), float(ni.eps), w_in.data_ptr(), now.data_ptr(), nob.data_ptr(), float(no.eps),
               w_pout.data_ptr(), w_gout.data_ptr(), out.data_ptr(), out_mode, None if rs is None else rs.data_ptr(),
               ws.data_ptr(), ws.numel(), stages, _stream(x))
    return out


def workspace_bytes(n: int) -> int:
    """Workspace that serves both fused triangle ops at size n."""
    lib = N.lib()
    return max(lib.bmx_trimul_workspace_bytes(n), lib.bmx_triattn_workspace_bytes(n))


def new_workspace(n: int, device) -> torch.Tensor:
    return _workspace(workspace_bytes(n), device)


def _triattn_proj_weight(wq, wk, wv, wb):
    rows = N.lib().bmx_triattn_proj_rows()
    w = torch.zeros((rows, C), dtype=torch.bfloat16, device=wq.device)
    used = torch.cat([wq, wk, wv, wb], 0)
    w[: used.shape[0]] = used.to(torch.bfloat16)
    return w


def triattn(module, x, mask, starting, out_mode=OUT_BF16, out=None, workspace=None, stages=ALL_STAGES,
            row_scale=None):
    """Fused TriangleAttention (starting or ending node) for x [N, N, 128].

    ``module`` carries Boltz's TriangleAttention parameters: ``layer_norm``,
    ``linear`` (triangle bias), ``mha.linear_{q,k,v,g,o}``, ``inf``.
    ``stages`` selects the kernels (1 projection, 2 attention core, 4 output).
    ``row_scale`` (fp32 [N] or None) multiplies the output of x's row i
    (starting) or column i (ending) before the residual add:
    PairformerLayer's dropout mask (row-wise / column-wise)."""
    _cuda(x)
    _check(x.dim() == 3 and x.size(0) == x.size(1) and x.size(2) == C, "expected x of shape [N, N, 128]")
    _check(x.dtype in (torch.float32, torch.bfloat16) and x.is_contiguous(), "expected contiguous fp32/bf16 x")
    n = x.size(0)
    if mask is not None:
        _cuda(x, mask)
        _check(mask.shape == x.shape[:2] and mask.dtype == torch.float32 and mask.is_contiguous(),
               "expected a contiguous fp32 [N, N] mask")
    mha = module.mha
    w_proj = cached_weight(module, "w_proj", (mha.linear_q.weight, mha.linear_k.weight, mha.linear_v.weight,
                                              module.linear.weight), _triattn_proj_weight)
    w_g = cached_weight(module, "w_g", (mha.linear_g.weight,), _bf16)
    w_o = cached_weight(module, "w_o", (mha.linear_o.weight,), _bf16)
    b_g = cached_weight(module, "b_g", (mha.linear_g.bias,), _f32)
    b_o = cached_weight(module, "b_o", (mha.linear_o.bias,), _f32)
    ln = module.layer_norm
    lnw, lnb = cached_weight(module, "ln_w", (ln.weight,), _f32), cached_weight(module, "ln_b", (ln.bias,), _f32)
    out = _out_tensor(x, out, out_mode)
    rs = _row_scale(row_scale, x, n)
    nbytes = N.lib().bmx_triattn_workspace_bytes(n)
    ws = workspace if workspace is not None and workspace.numel() >= nbytes else _workspace(nbytes, x.device)
    if n:
        N.call("bmx_triattn_fwd", x.data_ptr(), _code(x.dtype), None if mask is None else mask.data_ptr(), n,
               int(bool(starting)), float(module.inf), lnw.data_ptr(), lnb.data_ptr(), float(ln.eps),
               w_proj.data_ptr(), w_g.data_ptr(), b_g.data_ptr(), w_o.data_ptr(), b_o.data_ptr(), out.data_ptr(),
               out_mode, None if rs is None else rs.data_ptr(), ws.data_ptr(), ws.numel(), stages, _stream(x))
    return out


TRIATTN_FP32_PROJ_COLS = 576


def _triattn_fp32_split_weight(module):
    """q | k | v | g and the triangle bias as one split-bf16 weight for
    LayerNorm-without-affine(x), the LayerNorm affine folded in:
    (W diag w) LN0(x) + (bias + W b); bf16 [576, 3 * 128 + 64] (rows 512 ..
    512 + heads the triangle bias, zero rows up to 576)."""
    mha, ln = module.mha, module.layer_norm
    lins = (mha.linear_q, mha.linear_k, mha.linear_v, mha.linear_g, module.linear)

    def fold(*_):
        w = torch.cat([lin.weight.detach().float() for lin in lins])
        b = torch.cat([lin.bias.detach().float() if lin.bias is not None
                       else w.new_zeros(lin.out_features) for lin in lins])
        if ln.bias is not None:
            b = b + w @ ln.bias.detach().float()
        # zero rows up to 576 outputs: the GEMM runs faster than at 516 and output rows stay 128-byte aligned
        pad = TRIATTN_FP32_PROJ_COLS - w.shape[0]
        w = torch.cat([w * ln.weight.detach().float(), w.new_zeros(pad, C)])
        return _x3_weight(w, torch.cat([b, b.new_zeros(pad)]))

    srcs = tuple(t for m_ in (ln,) + lins for t in (m_.weight, m_.bias) if t is not None)
    _check(4 * C + module.no_heads <= TRIATTN_FP32_PROJ_COLS, "too many heads")
    return cached_weight(module, "qkvgb_ln_x3", srcs, fold)


def _triattn_fp32_exact_weights(module):
    """fp32 q | k | v | g weight [512, 128] and bias (linear_g's only)."""
    mha = module.mha
    w = cached_weight(module, "qkvg_f32", (mha.linear_q.weight, mha.linear_k.weight, mha.linear_v.weight,
                                           mha.linear_g.weight), lambda *ws: torch.cat(ws, 0).float())
    b = cached_weight(module, "qkvg_bias_f32", (mha.linear_g.bias,),
                      lambda bg: torch.cat([bg.new_zeros(3 * C), bg]).float())
    return w, b


def triattn_fp32(module, x, mask, starting, block_rows=None):
    """TriangleAttention (starting or ending node) in fp32 for x [N, N, 128]
    fp32, the fp32 mode of the module (autocast off; reference
    triangle.py:38-52 accelerates it too).  The q | k | v | g projection and
    the triangle bias are one split-bf16 GEMM of LayerNorm-without-affine(x),
    the LayerNorm affine folded into its weights (in exact fp32 mode the fp32
    LN128 kernel and fp32 GEMMs);
    the attention, mask bias, softmax, PV product and gate run fused in
    ``bmx_seq_attention_x3_batched_fwd`` (split-bf16 products, about 2^-16
    relative each; ``bmx_seq_attention_batched_fwd`` on fp32 MFMA in exact fp32
    mode), every row i one batch element attending over its N keys, all rows
    sharing the [4, N, N] triangle bias, so the [N, 4, N, N] scores never
    reach HBM; ``linear_o`` is an fp32 GEMM.  Returns fp32 [N, N, 128].

    ``block_rows`` < N processes the rows of the frame (x's rows for the
    starting node, its columns for the ending node) in blocks of that many
    (``_triattn_fp32_blocked``): the same products, with the per-pair working
    set held for one block at a time."""
    _cuda(x)
    _check(x.dim() == 3 and x.size(0) == x.size(1) and x.size(2) == C and x.dtype == torch.float32,
           "expected fp32 x of shape [N, N, 128]")
    n = x.size(0)
    mha, heads, d = module.mha, module.no_heads, module.c_hidden
    _check(heads * d == C, "expected heads x head dim = 128")
    if block_rows is not None and 0 < block_rows < n:
        return _triattn_fp32_blocked(module, x, mask, starting, int(block_rows))
    if not starting:
        mask = None if mask is None else mask.transpose(0, 1)
    ln = module.layer_norm
    split = not _EXACT_FP32[0] and ln.weight is not None
    # the ending node works on x transposed: the split path's LayerNorm reads the transposed rows in
    # place, the exact path transposes x once
    x = x.contiguous() if starting or split else x.transpose(0, 1).contiguous()
    if split:
        w3 = _triattn_fp32_split_weight(module)
        op = (layernorm_split3(x.view(-1, C), ln.eps) if starting
              else layernorm_split3_t(x, ln.eps).view(-1, split_width(C)))
        proj = mm_split(op, w3).view(n, n, TRIATTN_FP32_PROJ_COLS)
        del op  # 0.9 KB per pair, not needed by the attention
        tri_bias = proj[..., 4 * C:4 * C + heads].permute(2, 0, 1).contiguous()  # [H, q, k], shared by every row
    else:
        xn = norm(x.view(-1, C), _f32(ln.weight), _f32(ln.bias), ln.eps, bf16_output=False)
        w, b = _triattn_fp32_exact_weights(module)
        proj = torch.nn.functional.linear(xn, w, b).view(n, n, 4 * C)
        tri_bias = torch.nn.functional.linear(xn, module.linear.weight.float()).view(n, n, heads)
        tri_bias = tri_bias.permute(2, 0, 1).contiguous()  # [H, q, k], shared by every row
    m = x.new_ones(n, n) if mask is None else mask.to(torch.float32).contiguous()
    q, k, v, g = proj[..., :4 * C].split(C, dim=-1)
    # the split-bf16 kernel (about 2^-16 relative per product; 1.8x faster at N = 1024) unless exact
    # fp32 products are asked for
    o = seq_attention_batched(q, k, v, tri_bias[None], m, g, module.inf, bias_div=n, split=not _EXACT_FP32[0])
    del q, k, v, g, proj, tri_bias  # 2.3 KB per pair, before linear_o's output is allocated
    out = torch.nn.functional.linear(o, mha.linear_o.weight.float(), mha.linear_o.bias.float())
    return out if starting else out.transpose(0, 1)


def _triattn_fp32_blocked(module, x, mask, starting, rows):
    """``triattn_fp32`` over blocks of ``rows`` frame rows (x's rows for the
    starting node, x's columns, copied transposed one block at a time, for the
    ending node).  A first pass writes the [H, N, N] triangle bias, which every
    row shares, from each block's LayerNorm operand and only the bias rows of
    the projection weight; a second pass recomputes each block's operand and
    runs its q | k | v | g projection, the fused attention over the block's
    rows and ``linear_o`` into the output frame.  Full-frame memory: the
    output, the bias and the mask (about 532 bytes per pair); the rest is
    per block."""
    n = x.size(0)
    mha, heads, ln = module.mha, module.no_heads, module.layer_norm
    split = not _EXACT_FP32[0] and ln.weight is not None
    if mask is None:
        m = x.new_ones(n, n)
    else:
        m = (mask if starting else mask.transpose(0, 1)).to(torch.float32).contiguous()

    def frame_rows(i0, i1):  # [i1 - i0, N, 128] fp32, contiguous
        return x[i0:i1].contiguous() if starting else x[:, i0:i1].transpose(0, 1).contiguous()

    if split:
        w3 = _triattn_fp32_split_weight(module)
        w3_bias = w3[4 * C:]  # the bias rows and their zero padding: 64 outputs
        features = lambda xb: layernorm_split3(xb.view(-1, C), ln.eps)
        project_bias = lambda f: mm_split(f, w3_bias)
        project = lambda f: mm_split(f, w3)
    else:
        w, b = _triattn_fp32_exact_weights(module)
        w_bias = module.linear.weight.float()
        features = lambda xb: norm(xb.view(-1, C), _f32(ln.weight), _f32(ln.bias), ln.eps, bf16_output=False)
        project_bias = lambda f: torch.nn.functional.linear(f, w_bias)
        project = lambda f: torch.nn.functional.linear(f, w, b)
    blocks = [(i0, min(n, i0 + rows)) for i0 in range(0, n, rows)]
    tri_bias = torch.empty(heads, n, n, device=x.device, dtype=torch.float32)  # [H, q, k]
    for i0, i1 in blocks:
        bias = project_bias(features(frame_rows(i0, i1)))[:, :heads]
        tri_bias[:, i0:i1] = bias.view(i1 - i0, n, heads).permute(2, 0, 1)
        del bias
    out = torch.empty(n, n, C, device=x.device, dtype=torch.float32)  # the output frame
    w_o, b_o = mha.linear_o.weight.float(), mha.linear_o.bias.float()
    for i0, i1 in blocks:
        proj = project(features(frame_rows(i0, i1))).view(i1 - i0, n, -1)
        q, k, v, g = proj[..., :4 * C].split(C, dim=-1)
        o = seq_attention_batched(q, k, v, tri_bias[None], m[i0:i1], g, module.inf, bias_div=i1 - i0,
                                  split=not _EXACT_FP32[0])
        del q, k, v, g, proj
        torch.addmm(b_o, o.view(-1, C), w_o.t(), out=out[i0:i1].view(-1, C))
        del o
    return out if starting else out.transpose(0, 1)


def pair_transition(module, x, out_mode=OUT_BF16, out=None, pair_bias=None):
    """Fused Transition(128, 512) over the rows of x [..., 128].

    ``pair_bias=(proj_z_norm, proj_z_linear, bias_out)`` also writes the
    sequence stack's pair bias of the result (``pair_bias`` below applied to
    ``out``) into ``bias_out`` [16, rows] in the same pass; it needs an fp32
    ``out_mode``."""
    _cuda(x)
    _check(x.shape[-1] == C and x.dtype in (torch.float32, torch.bfloat16) and x.is_contiguous(),
           "expected contiguous fp32/bf16 x with 128 channels")
    _check(module.fc1.weight.shape == (4 * C, C) and module.fc3.weight.shape == (C, 4 * C),
           "expected a 128 -> 512 -> 128 transition")
    w12 = cached_weight(module, "w12p", (module.fc1.weight, module.fc2.weight), _bf16_packed)
    w3 = cached_weight(module, "w3p", (module.fc3.weight,), _bf16_packed)
    lnw = cached_weight(module, "ln_w", (module.norm.weight,), _f32)
    lnb = cached_weight(module, "ln_b", (module.norm.bias,), _f32)
    out = _out_tensor(x, out, out_mode)
    rows = x.numel() // C
    if pair_bias is None:
        if rows:
            N.call("bmx_pair_transition_fwd", x.data_ptr(), _code(x.dtype), rows, lnw.data_ptr(), lnb.data_ptr(),
                   float(module.norm.eps), w12.data_ptr(), w3.data_ptr(), out.data_ptr(), out_mode, _stream(x))
        return out
    norm, lin, bias_out = pair_bias
    _check(out_mode != OUT_BF16, "the fused pair bias needs an fp32 out_mode")
    _check(lin.weight.shape == (16, C), "expected a 128 -> 16 projection")
    _check(bias_out.numel() == 16 * rows and bias_out.dtype == torch.float32 and bias_out.is_contiguous(),
           "bias_out must be a contiguous fp32 tensor of 16 x rows")
    fold = cached_weight(lin, "pair_bias_fold", (norm.weight, norm.bias, lin.weight), pair_bias_fold)
    if rows:
        N.call("bmx_pair_transition_bias_fwd", x.data_ptr(), _code(x.dtype), rows, lnw.data_ptr(), lnb.data_ptr(),
               float(module.norm.eps), w12.data_ptr(), w3.data_ptr(), out.data_ptr(), out_mode, fold.data_ptr(),
               float(norm.eps), bias_out.data_ptr(), _stream(x))
    return out


def pair_bias_fold(ln_w, ln_b, w):
    """Folded pair-bias weights (``bmx_pair_bias_fold``): the LayerNorm affine
    folded into the 128 -> 16 projection, in the fused epilogue's operand order."""
    _cuda(ln_w, ln_b, w)
    _check(ln_w.shape == (C,) and ln_b.shape == (C,) and w.shape == (16, C), "expected a 128 -> 16 projection")
    ln_w, ln_b, w = (_f32(t) for t in (ln_w, ln_b, w))
    out = torch.empty(N.lib().bmx_pair_bias_fold_bytes(), dtype=torch.uint8, device=w.device)
    N.call("bmx_pair_bias_fold", ln_w.data_ptr(), ln_b.data_ptr(), w.data_ptr(), 16, out.data_ptr(), _stream(w))
    return out


def pair_bias(proj_z_norm, proj_z_linear, z, out=None):
    """fp32 ``Linear(LN(z))`` for 16 heads, returned (or written into ``out``)
    head-major as [H, N, N] (the layout AttentionPairBias adds to its logits);
    z is [N, N, 128]."""
    _cuda(z)
    _check(z.dim() == 3 and z.shape[-1] == C and z.dtype in (torch.float32, torch.bfloat16) and z.is_contiguous(),
           "expected contiguous z of shape [N, N, 128]")
    heads = proj_z_linear.weight.shape[0]
    _check(heads == 16 and proj_z_linear.weight.shape[1] == C, "expected a 128 -> 16 projection")
    w = cached_weight(proj_z_linear, "w32", (proj_z_linear.weight,), _f32)
    lnw = cached_weight(proj_z_norm, "w32", (proj_z_norm.weight,), _f32)
    lnb = cached_weight(proj_z_norm, "b32", (proj_z_norm.bias,), _f32)
    shape = (heads, z.shape[0], z.shape[1])
    if out is None:
        out = torch.empty(shape, device=z.device, dtype=torch.float32)
    _check(out.shape == shape and out.dtype == torch.float32 and out.is_contiguous(),
           "out must be a contiguous fp32 [16, N, N]")
    rows = z.shape[0] * z.shape[1]
    if rows:
        N.call("bmx_pair_bias_fwd", z.data_ptr(), _code(z.dtype), rows, lnw.data_ptr(), lnb.data_ptr(),
               float(proj_z_norm.eps), w.data_ptr(), heads, out.data_ptr(), _stream(z))
    return out


def seq_attention(q, k, v, bias, mask, g, inf, out=None):
    """Pair-biased softmax attention of AttentionPairBias, fp32, for one batch
    element: q, k, v and the gate logits g are [N, H * D] (D = 24 or 48) with
    unit column stride and one common row stride (e.g. column slices of a
    fused [N, 4 H D] projection), bias [H, N, N], mask [N].  Returns (or
    writes into ``out``) ``sigmoid(g) * softmax(q k^T / sqrt(D) + bias +
    (1 - mask) * -inf) v`` as a contiguous [N, H * D]."""
    _cuda(q, k, v, bias, mask, g)
    _check(bias.dim() == 3, "expected a [H, N, N] bias")
    heads, n = bias.shape[0], q.shape[0]
    width = q.shape[1] if q.dim() == 2 else -1
    _check(width > 0 and width % heads == 0 and width // heads in (24, 48), "expected H heads of 24 or 48 dims")
    ld = q.stride(0) if n > 1 else width
    for t in (q, k, v, g):
        _check(t.shape == (n, width) and t.dtype == torch.float32 and t.stride(1) == 1
               and (n <= 1 or t.stride(0) == ld), "expected fp32 [N, H * D] q / k / v / g with one row stride")
    _check(bias.shape == (heads, n, n) and bias.dtype == torch.float32 and bias.is_contiguous(),
           "expected a contiguous fp32 [H, N, N] bias")
    _check(mask.shape == (n,) and mask.dtype == torch.float32 and mask.is_contiguous(), "expected an fp32 [N] mask")
    if out is None:
        out = torch.empty((n, width), device=q.device, dtype=torch.float32)
    _check(out.shape == (n, width) and out.dtype == torch.float32 and out.is_contiguous(),
           "out must be a contiguous fp32 [N, H * D]")
    N.call("bmx_seq_attention_fwd", q.data_ptr(), k.data_ptr(), v.data_ptr(), bias.data_ptr(), mask.data_ptr(),
           g.data_ptr(), n, ld, heads, width // heads, float(inf), out.data_ptr(), _stream(q))
    return out


# The token transformer's attention (H * D = 768 >= X3_MIN_K, 1024 keys) runs
# its two products as split-bf16 MFMA (bmx_seq_attention_x3_batched_fwd) like
# its linears, unless exact fp32 is switched on; short key rows (the atom
# windows' 128) and the Pairformer sequence stack (H * D = 384) keep the fp32
# MFMA kernel, where the split pre-pass would cost more than it saves.
X3_ATTN_MIN_KEYS = 256


def seq_attention_split_ok(q, g, nk) -> bool:
    """Whether ``seq_attention_batched`` takes the split-bf16 kernel by default:
    not in exact fp32 mode, width >= ``X3_MIN_K``, >= ``X3_ATTN_MIN_KEYS`` keys,
    and 16-byte g rows."""
    width = q.shape[-1]
    return (not _EXACT_FP32[0] and width >= X3_MIN_K and nk >= X3_ATTN_MIN_KEYS and g.data_ptr() % 16 == 0
            and q.stride(1) % 4 == 0 and q.stride(0) % 4 == 0)


def seq_attention_batched(q, k, v, bias, mask, g, inf, bias_div=1, out=None, split=None, split_out=False):
    """``seq_attention`` for a batch in one launch (``bmx_seq_attention_batched_fwd``):
    q, g [B, NQ, H * D] and k, v [B, NK, H * D] (D = 24, 32 or 48; unit column
    stride; q and g share their strides, k and v theirs), bias
    [B / bias_div, H, NQ, NK] with dense elements (element b uses bias
    b // bias_div), mask [B or 1, NK] with unit stride.  Returns (or writes into
    ``out``) a contiguous fp32 [B, NQ, H * D].  ``split``: True for the
    split-bf16 kernel (``bmx_seq_attention_x3_batched_fwd``, about 2^-16
    relative per product), False for fp32 MFMA, None to choose as above.
    ``split_out``: return the output rows as the split-bf16 operand of the next
    linear instead ([B * NQ, 3 H D + 64] bf16, ``bmx_seq_attention_x3_batched_split_fwd``;
    split-bf16 kernel only)."""
    _cuda(q, k, v, bias, mask, g)
    _check(q.dim() == 3 and k.dim() == 3 and bias.dim() == 4 and mask.dim() == 2, "expected 3-d q/k, 4-d bias, 2-d mask")
    b, nq, width = q.shape
    nk, heads = k.shape[1], bias.shape[1]
    _check(width % heads == 0 and width // heads in (24, 32, 48), "expected H heads of 24, 32 or 48 dims")
    _check(g.shape == q.shape and g.stride() == q.stride() and k.shape == (b, nk, width) and v.shape == k.shape
           and v.stride() == k.stride(), "q / g and k / v must match in shape and strides")
    for t in (q, k, v, g):
        _check(t.dtype == torch.float32 and t.stride(2) == 1, "expected fp32 q / k / v / g with unit column stride")
    _check(bias.dtype == torch.float32 and bias.shape[1:] == (heads, nq, nk) and bias.shape[0] * bias_div == b
           and (bias.shape[0] == 0 or bias[0].is_contiguous()), "expected fp32 [B / bias_div, H, NQ, NK] dense bias")
    _check(mask.dtype == torch.float32 and mask.shape[1] == nk and mask.shape[0] in (1, b) and mask.stride(1) == 1,
           "expected an fp32 [B or 1, NK] mask")
    if split is None:
        split = seq_attention_split_ok(q, g, nk)
    if split_out:
        _check(split and out is None, "split_out needs the split-bf16 kernel and no out")
        out = torch.empty((b * nq, split_width(width)), device=q.device, dtype=torch.bfloat16)
    elif out is None:
        out = torch.empty((b, nq, width), device=q.device, dtype=torch.float32)
    else:
        _check(out.shape == (b, nq, width) and out.dtype == torch.float32 and out.is_contiguous(),
               "out must be a contiguous fp32 [B, NQ, H * D]")
    if b and nq:
        args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), bias.data_ptr(), mask.data_ptr(), g.data_ptr(), b, nq, nk,
                q.stride(1), k.stride(1), q.stride(0), k.stride(0), bias.stride(0),
                mask.stride(0) if mask.shape[0] > 1 else 0, bias_div, heads, width // heads, float(inf),
                out.data_ptr())
        if split:
            nbytes = N.lib().bmx_seq_attention_x3_workspace_bytes(b, nk, heads, width // heads)
            ws = torch.empty(nbytes, device=q.device, dtype=torch.uint8)
            name = "bmx_seq_attention_x3_batched_split_fwd" if split_out else "bmx_seq_attention_x3_batched_fwd"
            N.call(name, *args, ws.data_ptr(), nbytes, _stream(q))
        else:
            N.call("bmx_seq_attention_batched_fwd", *args, _stream(q))
    return out


def seq_attention_windowed(q, k, v, bias, mask, g, inf, *, windows, key_offset, bias_group):
    """The atom transformer's windowed attention (``bmx_seq_attention_windowed_fwd``):
    q, g [E, W, H * D] query windows (E = samples x ``windows`` windows; rows
    at one stride, windows contiguous), k, v [E * W, H * D] (the projected atom
    rows, rows at one stride), mask [E * W] (the atom mask).  Window e reads
    key j from atom row e * W + key_offset + j of its sample; keys past the
    sample's ends are zero keys and values with mask 0 (upstream's zero rows of
    single_to_keys).  bias [B, windows, W, NK, H] (or [B * windows, W, NK, H])
    in any strides (one layer's heads of the atom bias, in place): window e
    uses window e % windows of structure e // bias_group.  Returns a
    contiguous fp32 [E, W, H * D]."""
    _cuda(q, k, v, bias, mask, g)
    if bias.dim() == 4:  # [Eb, W, NK, H]: structures of ``windows`` consecutive elements
        _check(bias.shape[0] % windows == 0, "bias elements must be whole structures")
        bias = bias.unflatten(0, (bias.shape[0] // windows, windows))
    _check(q.dim() == 3 and bias.dim() == 5 and k.dim() == 2 and mask.dim() == 1, "expected 3-d q, 2-d k, 5-d bias")
    e, w, width = q.shape
    nk, heads = bias.shape[3], bias.shape[4]
    _check(width % heads == 0 and width // heads in (24, 32, 48), "expected H heads of 24, 32 or 48 dims")
    _check(g.shape == q.shape and g.stride() == q.stride() and q.stride(2) == 1 and q.stride(0) == w * q.stride(1),
           "q / g must be [E, W, H * D] windows with dense rows, sharing strides")
    _check(k.shape == (e * w, width) and v.shape == k.shape and k.stride() == v.stride() and k.stride(1) == 1,
           "k / v must be [E * W, H * D] with dense rows, sharing strides")
    _check(mask.shape == (e * w,) and mask.is_contiguous() and mask.dtype == torch.float32, "mask must be fp32 [E * W]")
    _check(bias.dtype == torch.float32 and tuple(bias.shape[1:3]) == (windows, w) and bias.shape[0] * bias_group == e
           and e % windows == 0 and bias_group % windows == 0, "bias does not match the windows")
    for t in (q, k, v, g):
        _check(t.dtype == torch.float32, "expected fp32 q / k / v / g")
    out = torch.empty((e, w, width), device=q.device, dtype=torch.float32)
    if e:
        N.call("bmx_seq_attention_windowed_fwd", q.data_ptr(), k.data_ptr(), v.data_ptr(), bias.data_ptr(),
               mask.data_ptr(), g.data_ptr(), e, w, nk, q.stride(1), k.stride(0), windows, key_offset, bias_group,
               bias.stride(0), bias.stride(1), bias.stride(4), bias.stride(2), bias.stride(3), heads, width // heads,
               float(inf), out.data_ptr(), _stream(q))
    return out


def adaln_modulate(a, scale, shift, eps):
    """``sigmoid(scale) * LN_noaffine(a) + shift`` in one pass; scale and shift
    may be column slices of one wider projection (rows at one stride,
    ``bmx_adaln_strided``)."""
    _cuda(a, scale, shift)
    _check(a.is_contiguous(), "expected contiguous a")
    ld = _same_rows(a, scale, shift)
    d = a.shape[-1]
    out = torch.empty_like(a)
    rows = a.numel() // d if d else 0
    if rows:
        N.call("bmx_adaln_strided", a.data_ptr(), scale.data_ptr(), shift.data_ptr(), ld, out.data_ptr(),
               _code(a.dtype), rows, d, float(eps), _stream(a))
    return out
