"""SwiGLU -- drop-in for ops/activation_ops.py (the MLP-block activation)."""

from __future__ import annotations

import torch

from . import _lib
from ._common import ACT_DTYPES, ci_safe_mode_enabled


def _validate_inputs(gate, up):
    """ops/activation_ops.py:41-51."""
    if gate.ndim != 3 or up.ndim != 3:
        raise ValueError(f"gate and up must be 3-D [B,S,D], got {tuple(gate.shape)}, {tuple(up.shape)}")
    if gate.shape != up.shape:
        raise ValueError(f"gate and up must have identical shapes, got {tuple(gate.shape)}, {tuple(up.shape)}")
    B, S, D = gate.shape
    if gate.dtype not in ACT_DTYPES:
        raise TypeError(f"gate dtype must be float16 or bfloat16, got {gate.dtype}")
    if up.dtype not in ACT_DTYPES:
        raise TypeError(f"up dtype must be float16 or bfloat16, got {up.dtype}")
    return B, S, D


def _normalize_fused_inputs(gate, up):
    """ops/activation_ops.py:54-75."""
    if gate.shape != up.shape:
        raise ValueError(f"gate and up must have identical shapes, got {tuple(gate.shape)}, {tuple(up.shape)}")
    if gate.ndim == 2:
        rows, dim = gate.shape
        gate2d, up2d = gate, up
    elif gate.ndim == 3:
        rows = gate.shape[0] * gate.shape[1]
        dim = gate.shape[2]
        gate2d, up2d = gate.reshape(rows, dim), up.reshape(rows, dim)
    else:
        raise ValueError(f"gate and up must have shape [rows,D] or [B,S,D], got {tuple(gate.shape)}, {tuple(up.shape)}")
    if gate.dtype not in ACT_DTYPES:
        raise TypeError(f"gate dtype must be float16 or bfloat16, got {gate.dtype}")
    if up.dtype not in ACT_DTYPES:
        raise TypeError(f"up dtype must be float16 or bfloat16, got {up.dtype}")
    return gate2d, up2d, tuple(gate.shape), rows, dim


def _silu_mul(gate, up):
    g = gate.to(torch.float32)
    return (g / (1.0 + torch.exp(-g)) * up.to(torch.float32)).to(gate.dtype)


def _hip_swiglu(gate, up):
    gate = gate.contiguous()
    up = up.to(gate.dtype).contiguous()
    dev = _lib.require_device(gate, up)
    out = torch.empty_like(gate)
    _lib.launch("mk_swiglu", dev, _lib.ptr(gate), _lib.ptr(up), _lib.ptr(out), gate.numel(),
                _lib.dtype_code(gate.dtype))
    return out


def reference_swiglu(gate, up):
    """ops/activation_ops.py:83-88: g / (1 + exp(-g)) * u in fp32."""
    _validate_inputs(gate, up)
    return _silu_mul(gate, up)


def swiglu(gate, up, *, backend: str = "auto"):
    """ops/activation_ops.py:91-114."""
    _validate_inputs(gate, up)
    backend_name = backend.lower()
    if backend_name == "auto":
        backend_name = "metal"
    if ci_safe_mode_enabled() or backend_name == "reference":
        return reference_swiglu(gate, up)
    if backend_name != "metal":
        raise ValueError("backend must be one of 'reference', 'metal', 'auto'")
    return _hip_swiglu(gate, up)


def fused_swiglu(gate, up, *, backend: str = "metal_fused"):
    """ops/activation_ops.py:117-153 (flattened rows)."""
    gate2d, up2d, original_shape, rows, dim = _normalize_fused_inputs(gate, up)
    backend_name = backend.lower()
    if backend_name == "auto":
        backend_name = "metal_fused"
    if ci_safe_mode_enabled() or backend_name == "reference":
        return _silu_mul(gate2d, up2d).reshape(original_shape)
    if backend_name == "metal":
        if len(original_shape) != 3:
            raise ValueError("backend='metal' for fused_swiglu requires [B,S,D] inputs; use 'metal_fused' for flattened shapes")
        return swiglu(gate, up, backend="metal")
    if backend_name != "metal_fused":
        raise ValueError("backend must be one of 'reference', 'metal', 'metal_fused', 'auto'")
    return _hip_swiglu(gate2d, up2d).reshape(original_shape)
