"""Eligibility predicates shared by the patched forwards."""

from __future__ import annotations

from functools import lru_cache

import torch


@lru_cache(maxsize=None)
def _is_gfx950(index: int) -> bool:
    props = torch.cuda.get_device_properties(index)
    return getattr(props, "gcnArchName", "").startswith("gfx950")


def gfx950_tensor(x: torch.Tensor) -> bool:
    """True for a tensor on a gfx950 (MI355X) device of a ROCm build."""
    return bool(torch.version.hip) and x.is_cuda and _is_gfx950(x.device.index or 0)


def gfx950_available() -> bool:
    return bool(torch.version.hip) and torch.cuda.is_available() and _is_gfx950(torch.cuda.current_device())


def inference(module) -> bool:
    return not module.training and not torch.is_grad_enabled()


def bf16_autocast() -> bool:
    return torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16


def autocast_off() -> bool:
    return not torch.is_autocast_enabled("cuda")


def fp32_contiguous_on(device, *tensors) -> bool:
    return all(t.dtype == torch.float32 and t.is_contiguous() and t.device == device for t in tensors)
