"""RMSNorm -- drop-in for ops/norm_ops.py (the MLP-block prologue)."""

from __future__ import annotations

import torch

from . import _lib
from ._common import ci_safe_mode_enabled

_NORM_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def _validate_inputs(x, weight):
    """ops/norm_ops.py:27-44."""
    if x.ndim != 3:
        raise ValueError(f"x must be 3-D [B,S,D], got shape {tuple(x.shape)}")
    if weight.ndim != 1:
        raise ValueError(f"weight must be 1-D [D], got shape {tuple(weight.shape)}")
    B, S, D = x.shape
    if D != weight.shape[0]:
        raise ValueError(f"weight shape must be [D] with D={D}, got {tuple(weight.shape)}")
    if B <= 0 or S <= 0 or D <= 0:
        raise ValueError(f"Invalid x shape: {tuple(x.shape)}")
    if x.dtype not in _NORM_DTYPES:
        raise TypeError(f"x dtype must be float16, bfloat16, or float32, got {x.dtype}")
    if weight.dtype not in _NORM_DTYPES:
        raise TypeError(f"weight dtype must be float16, bfloat16, or float32, got {weight.dtype}")
    return B, S, D


def reference_rms_norm(x, weight, eps: float = 1e-5):
    """ops/norm_ops.py:47-52: x * rsqrt(mean(x^2) + eps) * w in fp32."""
    _, _, D = _validate_inputs(x, weight)
    xf = x.to(torch.float32)
    variance = torch.mean(xf * xf, dim=-1, keepdim=True)
    inv_rms = torch.rsqrt(variance + float(eps))
    out = xf * inv_rms * weight.to(torch.float32).reshape(1, 1, D)
    return out.to(x.dtype)


def rms_norm(x, weight, eps: float = 1e-5, *, backend: str = "auto"):
    """ops/norm_ops.py:55-85."""
    B, S, D = _validate_inputs(x, weight)
    backend_name = backend.lower()
    if backend_name == "auto":
        backend_name = "metal"
    if ci_safe_mode_enabled() or backend_name == "reference":
        return reference_rms_norm(x, weight, eps=eps)
    if backend_name != "metal":
        raise ValueError("backend must be one of 'reference', 'metal', 'auto'")
    x = x.contiguous()
    w = weight.contiguous()
    dev = _lib.require_device(x, w)
    y = torch.empty_like(x)
    _lib.launch("mk_rms_norm", dev, _lib.ptr(x), _lib.ptr(w), _lib.ptr(y), B * S, D, float(eps),
                _lib.dtype_code(x.dtype), _lib.dtype_code(w.dtype))
    return y


def residual_rms_norm(x, residual, weight, eps: float = 1e-5):
    """One-pass ``z = x + residual; y = rms_norm(z)`` returning (z, y): the
    prologue of ops/mlp_block_ops.py:343-344 fused into one HIP launch."""
    if x.shape != residual.shape:
        raise ValueError(f"x and residual must have identical shapes, got {tuple(x.shape)}, {tuple(residual.shape)}")
    B, S, D = _validate_inputs(x, weight)
    x = x.contiguous()
    r = residual.to(x.dtype).contiguous()
    w = weight.contiguous()
    dev = _lib.require_device(x, r, w)
    z = torch.empty_like(x)
    y = torch.empty_like(x)
    _lib.launch("mk_residual_rms_norm", dev, _lib.ptr(x), _lib.ptr(r), _lib.ptr(w), _lib.ptr(z), _lib.ptr(y),
                B * S, D, float(eps), _lib.dtype_code(x.dtype), _lib.dtype_code(w.dtype))
    return z, y
