"""Residual add -- drop-in for the part of ops/fused_ops.py on the MLP path."""

from __future__ import annotations

import torch

from . import _lib
from ._common import ACT_DTYPES, ci_safe_mode_enabled


def reference_residual_add(x, residual):
    """ops/fused_ops.py:149-152."""
    if x.shape != residual.shape:
        raise ValueError(f"x and residual must have identical shapes, got {tuple(x.shape)}, {tuple(residual.shape)}")
    return (x.to(torch.float32) + residual.to(torch.float32)).to(x.dtype)


def residual_add(x, residual, *, backend: str = "auto"):
    """ops/fused_ops.py:155-180."""
    if x.shape != residual.shape:
        raise ValueError(f"x and residual must have identical shapes, got {tuple(x.shape)}, {tuple(residual.shape)}")
    if x.dtype not in ACT_DTYPES:
        raise TypeError(f"x dtype must be float16 or bfloat16, got {x.dtype}")
    backend_name = backend.lower()
    if backend_name == "auto":
        backend_name = "metal"
    if ci_safe_mode_enabled() or backend_name == "reference":
        return reference_residual_add(x, residual)
    if backend_name != "metal":
        raise ValueError("backend must be one of 'reference', 'metal', 'auto'")
    x = x.contiguous()
    r = residual.to(x.dtype).contiguous()
    dev = _lib.require_device(x, r)
    out = torch.empty_like(x)
    _lib.launch("mk_residual_add", dev, _lib.ptr(x), _lib.ptr(r), _lib.ptr(out), x.numel(),
                _lib.dtype_code(x.dtype))
    return out
