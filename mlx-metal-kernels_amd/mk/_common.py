"""Helpers shared by the op modules: env flags, dtype checks, shape rules."""

from __future__ import annotations

import os

import torch

ACT_DTYPES = (torch.float16, torch.bfloat16)
FLOAT_DTYPES = (torch.float16, torch.bfloat16, torch.float32, torch.float64)


def ci_safe_mode_enabled() -> bool:
    """MLX_METAL_CI_SAFE_MODE=1 routes ops to their ``reference_*`` path, as in
    the reference (ops/quant_ops.py:33-34).  It is an explicit opt-in for hosts
    without a GPU; it is never set implicitly."""
    return os.environ.get("MLX_METAL_CI_SAFE_MODE", "0") == "1"


def env_flag(name: str) -> bool:
    return os.environ.get(name, "0") == "1"


def finfo_max(dtype: torch.dtype) -> float:
    return float(torch.finfo(dtype).max)


def scales_for_kernel(scales: torch.Tensor, zeros: torch.Tensor | None):
    """fp16 scales/zeros go to the kernels as they are; any other float dtype
    is promoted to fp32 (the reference promotes everything to fp32 at the
    kernel boundary, ops/quant_ops.py:424)."""
    use_f16 = scales.dtype == torch.float16 and (zeros is None or zeros.dtype == torch.float16)
    target = torch.float16 if use_f16 else torch.float32
    s = scales.to(target).contiguous()
    z = None if zeros is None else zeros.to(target).contiguous()
    return s, z


def as_u8(t: torch.Tensor) -> torch.Tensor:
    return (t if t.dtype == torch.uint8 else t.to(torch.uint8)).contiguous()
