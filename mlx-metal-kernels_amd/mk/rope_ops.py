"""Interleaved (GPT-J style) RoPE semantics used by the fused
qkv-split + RoPE + paged-update kernels -- ops/rope_ops.py:61-75 and the table
builder of models/llama_config.py:107-124."""

from __future__ import annotations

import torch


def _validate_inputs(x, cos, sin, position_offset: int):
    """ops/rope_ops.py:25-58."""
    if x.ndim != 4:
        raise ValueError(f"x must be 4-D [B,S,H,D], got {tuple(x.shape)}")
    if cos.ndim != 2 or sin.ndim != 2:
        raise ValueError(f"cos and sin must be 2-D [S_total, D/2], got {tuple(cos.shape)}, {tuple(sin.shape)}")
    if cos.shape != sin.shape:
        raise ValueError(f"cos and sin must have identical shapes, got {tuple(cos.shape)}, {tuple(sin.shape)}")
    B, S, H, D = x.shape
    if D % 2 != 0:
        raise ValueError(f"RoPE requires even D, got D={D}")
    if cos.shape[1] != D // 2:
        raise ValueError(f"cos/sin last dim must be D/2={D // 2}, got {cos.shape[1]}")
    if position_offset < 0:
        raise ValueError("position_offset must be non-negative")
    if position_offset + S > cos.shape[0]:
        raise ValueError(
            f"position_offset + S must fit in cos/sin rows, got offset={position_offset}, S={S}, rows={cos.shape[0]}"
        )
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise TypeError(f"x dtype must be float16 or bfloat16, got {x.dtype}")
    return B, S, H, D, cos.shape[0]


def reference_apply_rope(x, cos, sin, position_offset: int = 0):
    """ops/rope_ops.py:61-75: pairs (2i, 2i+1) rotate by the angle of row
    position_offset + s; fp32 math, result in x's dtype.  The tables may sit
    on the host: the rows used move to x's device."""
    _, S, _, D, _ = _validate_inputs(x, cos, sin, position_offset)
    c = cos[position_offset:position_offset + S].to(device=x.device, dtype=torch.float32).reshape(1, S, 1, D // 2)
    s = sin[position_offset:position_offset + S].to(device=x.device, dtype=torch.float32).reshape(1, S, 1, D // 2)
    xe = x[..., 0::2].to(torch.float32)
    xo = x[..., 1::2].to(torch.float32)
    ye = xe * c - xo * s
    yo = xe * s + xo * c
    return torch.stack([ye, yo], dim=-1).reshape(x.shape).to(x.dtype)


def build_rope_tables(seq_len: int, head_dim: int, theta: float = 10000.0, *, device=None):
    """models/llama_config.py:107-124: inv_freq = theta^(-arange(0,D,2)/D),
    returns fp32 cos/sin of shape [seq_len, D/2]."""
    if seq_len <= 0:
        raise ValueError(f"seq_len must be positive, got {seq_len}")
    if head_dim % 2 != 0:
        raise ValueError(f"head_dim must be even for RoPE, got {head_dim}")
    positions = torch.arange(seq_len, dtype=torch.float32, device=device)
    inv_freq = 1.0 / (float(theta) ** (torch.arange(0, head_dim, 2, dtype=torch.float32, device=device) / float(head_dim)))
    freqs = positions.reshape(seq_len, 1) * inv_freq.reshape(1, head_dim // 2)
    return torch.cos(freqs), torch.sin(freqs)
