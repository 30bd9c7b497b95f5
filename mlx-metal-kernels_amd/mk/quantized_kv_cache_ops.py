"""Contiguous symmetric q8/q4 KV cache -- drop-in for
``ops/quantized_kv_cache_ops.py`` (config, cache dataclass, quantize /
dequantize / error, and GQA decode attention) over ``torch.Tensor``.

Format (ops/quantized_kv_cache_ops.py:131-170, the same quantizer as the
paged cache): per (sequence, position, kv head, group of ``group_size``
along D) one fp16 scale s = max(max|v|, 1e-8) / 127 (q8) or / 7 (q4),
computed in fp32 and rounded to fp16 after use; codes
clip(round_half_even(v / s), +-127|7) + 128|8, q4 packed two per byte
(low nibble = even d).  ``quantize_kv_cache`` quantizes positions
j < lengths[b] and leaves codes and scales of the others at 0, as the
reference does (:173-277).

Decode attention backends: ``"reference"`` (tensor ops) and ``"metal_q8"`` /
``"metal_q4"``, which run the paged quantized split-K HIP kernel over an
identity-paged view of the contiguous codes and scales (no copy).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Any

import torch

from . import _contig, _lib
from .gqa_ops import validate_gqa_heads
from .kv_cache_ops import normalize_positions
from .paged_kv_ops import _masked_attention
from .paged_quantized_kv_ops import (
    _dequant_last_dim,
    _hip_quantize_rows,
    _pack_last_dim,
    _quantize_last_dim,
)
from .quant_ops import unpack_q4_reference

_MAX_HEAD_DIM = 128


@dataclass
class QuantizedKVCacheConfig:
    """ops/quantized_kv_cache_ops.py:40-60."""

    bits: int = 8
    group_size: int = 32
    symmetric: bool = True
    with_zeros: bool = False
    scale_dtype: str = "float16"
    layout: str = "contiguous"

    def validate(self) -> "QuantizedKVCacheConfig":
        if self.bits not in (4, 8):
            raise ValueError(f"bits must be 4 or 8, got {self.bits}")
        if self.group_size <= 0:
            raise ValueError(f"group_size must be > 0, got {self.group_size}")
        if not self.symmetric:
            raise NotImplementedError("asymmetric quantization is not implemented yet")
        if self.with_zeros:
            raise NotImplementedError("zero-point quantization is not implemented yet")
        if self.layout != "contiguous":
            raise NotImplementedError(f"layout={self.layout!r} is not implemented yet; use 'contiguous'")
        return self


@dataclass
class QuantizedKVCache:
    """ops/quantized_kv_cache_ops.py:68-123: k_q/v_q [B, MAX_S, Hkv, D]
    (q8) or [..., ceil(D/2)] (q4) uint8, k/v_scales [B, MAX_S, Hkv,
    ceil(D/group_size)] fp16."""

    k_q: Any
    v_q: Any
    k_scales: Any
    v_scales: Any
    k_zeros: Any | None = None
    v_zeros: Any | None = None
    bits: int = 8
    group_size: int = 32
    original_shape: tuple[int, ...] | None = None
    layout: str = "contiguous"
    metadata: dict[str, Any] = field(default_factory=dict)

    def shapes(self) -> dict[str, tuple[int, ...] | None]:
        return {
            "k_q": tuple(self.k_q.shape),
            "v_q": tuple(self.v_q.shape),
            "k_scales": tuple(self.k_scales.shape),
            "v_scales": tuple(self.v_scales.shape),
            "original": None if self.original_shape is None else tuple(self.original_shape),
        }

    def validate(self) -> "QuantizedKVCache":
        if self.bits not in (4, 8):
            raise ValueError(f"bits must be 4 or 8, got {self.bits}")
        if self.k_q.shape != self.v_q.shape:
            raise ValueError(f"k_q and v_q shapes must match, got {tuple(self.k_q.shape)} != {tuple(self.v_q.shape)}")
        if self.k_scales.shape != self.v_scales.shape:
            raise ValueError(f"k_scales and v_scales shapes must match, got {tuple(self.k_scales.shape)} != "
                             f"{tuple(self.v_scales.shape)}")
        if self.layout != "contiguous":
            raise NotImplementedError(f"layout={self.layout!r} is not supported")
        if self.original_shape is not None and len(self.original_shape) != 4:
            raise ValueError(f"original_shape must be 4-D [B,MAX_S,Hkv,D], got {self.original_shape}")
        return self

    def memory_bytes(self) -> int:
        total = 0
        for arr in (self.k_q, self.v_q, self.k_scales, self.v_scales, self.k_zeros, self.v_zeros):
            if arr is not None:
                total += arr.numel() * arr.element_size()
        return total

    def compression_ratio(self, fp_bytes_per_value: int = 2) -> float | None:
        if self.original_shape is None:
            return None
        B, S, H, D = self.original_shape
        q_bytes = self.memory_bytes()
        return None if q_bytes == 0 else 2 * B * S * H * D * fp_bytes_per_value / q_bytes


def _geometry(cache: QuantizedKVCache):
    """(B, MAX_S, Hkv, D) of a cache, from original_shape or the code tensor."""
    if cache.original_shape is not None:
        return tuple(int(v) for v in cache.original_shape)
    B, S, H, Dq = cache.k_q.shape
    return B, S, H, (Dq if cache.bits == 8 else 2 * Dq)


def quantize_kv_cache(K_cache, V_cache, config: QuantizedKVCacheConfig, *, lengths=None) -> QuantizedKVCache:
    """ops/quantized_kv_cache_ops.py:173-277: positions j < lengths[b]
    (default: all) are quantized, the others keep zero codes and scales.
    Device tensors run ``mk_quantize_kv``; host tensors the tensor-op path."""
    config = config.validate()
    if K_cache.shape != V_cache.shape:
        raise ValueError(f"K_cache and V_cache must match, got {tuple(K_cache.shape)} != {tuple(V_cache.shape)}")
    if K_cache.ndim != 4:
        raise ValueError(f"K_cache must be 4-D [B,MAX_S,Hkv,D], got {tuple(K_cache.shape)}")
    B, MAX_S, Hkv, D = K_cache.shape
    g, bits = config.group_size, config.bits
    if K_cache.device.type == "cuda":
        kq, ks = _hip_quantize_rows(K_cache, g, bits)
        vq, vs = _hip_quantize_rows(V_cache, g, bits)
    else:
        kq, ks = _quantize_last_dim(K_cache.to(torch.float32), g, bits)
        vq, vs = _quantize_last_dim(V_cache.to(torch.float32), g, bits)
        if bits == 4:
            kq, vq = _pack_last_dim(kq), _pack_last_dim(vq)
    if lengths is not None:
        ln = normalize_positions(lengths, B, MAX_S + 1, device=K_cache.device)
        keep = (torch.arange(MAX_S, device=K_cache.device).reshape(1, MAX_S)
                < ln.to(K_cache.device).long().reshape(B, 1)).reshape(B, MAX_S, 1, 1)
        kq, vq = kq * keep, vq * keep
        ks, vs = ks * keep, vs * keep
    return QuantizedKVCache(k_q=kq, v_q=vq, k_scales=ks, v_scales=vs, bits=bits, group_size=g,
                            original_shape=tuple(K_cache.shape), layout=config.layout)


def _codes(cache: QuantizedKVCache, which: str, D: int) -> torch.Tensor:
    codes = cache.k_q if which == "k" else cache.v_q
    if cache.bits == 8:
        return codes
    return unpack_q4_reference(codes.reshape(-1, codes.shape[-1]), K=D).reshape(*codes.shape[:-1], D)


def dequantize_kv_cache(qkv_cache: QuantizedKVCache):
    """ops/quantized_kv_cache_ops.py:280-313: (code - 128|8) * |s| in fp32,
    rounded to fp16, for every position."""
    qkv_cache = qkv_cache.validate()
    B, S, H, D = _geometry(qkv_cache)
    g, bits = qkv_cache.group_size, qkv_cache.bits
    K = _dequant_last_dim(_codes(qkv_cache, "k", D), qkv_cache.k_scales, g, bits, D).to(torch.float16)
    V = _dequant_last_dim(_codes(qkv_cache, "v", D), qkv_cache.v_scales, g, bits, D).to(torch.float16)
    return K, V


def quantized_kv_error(K_cache, V_cache, qkv_cache: QuantizedKVCache) -> dict[str, float]:
    """ops/quantized_kv_cache_ops.py:316-341."""
    K_deq, V_deq = dequantize_kv_cache(qkv_cache)
    kd = K_cache.to(torch.float32) - K_deq.to(torch.float32).to(K_cache.device)
    vd = V_cache.to(torch.float32) - V_deq.to(torch.float32).to(V_cache.device)
    cr = qkv_cache.compression_ratio(fp_bytes_per_value=2)
    return {
        "k_max_abs_error": float(kd.abs().max()),
        "k_mean_abs_error": float(kd.abs().mean()),
        "k_rmse": float(torch.sqrt(torch.mean(kd ** 2))),
        "v_max_abs_error": float(vd.abs().max()),
        "v_mean_abs_error": float(vd.abs().mean()),
        "v_rmse": float(torch.sqrt(torch.mean(vd ** 2))),
        "compression_ratio": float(cr) if cr is not None else 0.0,
    }


def _validate_quantized_decode_inputs(q, qkv_cache: QuantizedKVCache, lengths):
    """ops/quantized_kv_cache_ops.py:348-374."""
    if q.ndim != 4:
        raise ValueError(f"q must be 4-D [B,1,Hq,D], got {tuple(q.shape)}")
    if q.shape[1] != 1:
        raise ValueError(f"q must have shape [B,1,Hq,D], got {tuple(q.shape)}")
    B, _, Hq, D = q.shape
    cache_B, MAX_S, Hkv, D_cache = _geometry(qkv_cache)
    if B != cache_B:
        raise ValueError(f"batch mismatch: q batch={B}, cache batch={cache_B}")
    if D != D_cache:
        raise ValueError(f"head_dim mismatch: q D={D}, cache D={D_cache}")
    validate_gqa_heads(Hq, Hkv)
    lengths_arr = normalize_positions(lengths if lengths is not None else MAX_S, B, MAX_S + 1, device=q.device)
    lengths_arr = torch.clamp(lengths_arr, max=MAX_S)
    return lengths_arr, B, MAX_S, Hq, Hkv, D


def reference_quantized_kv_gqa_decode_attention(q, qkv_cache: QuantizedKVCache, lengths=None, *, scale=None):
    """ops/quantized_kv_cache_ops.py:377-406: dequantize, then fp32 masked
    softmax attention per query head on kv head h // (Hq/Hkv)."""
    lengths_arr, B, MAX_S, Hq, Hkv, D = _validate_quantized_decode_inputs(q, qkv_cache, lengths)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    K_deq, V_deq = dequantize_kv_cache(qkv_cache)
    valid = torch.ones((B, MAX_S), dtype=torch.bool, device=q.device)
    out = _masked_attention(q[:, 0], K_deq.to(q.device), V_deq.to(q.device), lengths_arr, valid, scale)
    return out.unsqueeze(1).to(q.dtype)


def _check_kernel_layout(cache: QuantizedKVCache, B: int, S: int, Hkv: int, D: int):
    """The kernel reads codes and scales from (B, MAX_S, Hkv, D, bits,
    group_size) alone: the tensors must have exactly that layout."""
    g = int(cache.group_size)
    if g <= 0:
        raise ValueError(f"group_size must be positive, got {g}")
    want_codes = (B, S, Hkv, D if cache.bits == 8 else (D + 1) // 2)
    want_scales = (B, S, Hkv, (D + g - 1) // g)
    for name, t, want in (("k_q", cache.k_q, want_codes), ("v_q", cache.v_q, want_codes),
                          ("k_scales", cache.k_scales, want_scales), ("v_scales", cache.v_scales, want_scales)):
        if tuple(t.shape) != want:
            raise ValueError(f"{name} must have shape {want} for bits={cache.bits}, D={D}, group_size={g}; "
                             f"got {tuple(t.shape)}")


def _hip_quantized_attention(q, cache: QuantizedKVCache, lengths_arr, scale: float):
    B, _, Hq, D = q.shape
    _, S, Hkv, _ = _geometry(cache)
    _check_kernel_layout(cache, B, S, Hkv, D)
    kq, vq = cache.k_q.contiguous(), cache.v_q.contiguous()
    ks = cache.k_scales.to(torch.float16).contiguous()
    vs = cache.v_scales.to(torch.float16).contiguous()
    dev = _lib.require_device(q, kq, vq, ks, vs)
    if kq.dtype != torch.uint8 or vq.dtype != torch.uint8:
        raise TypeError(f"quantized codes must be uint8, got {kq.dtype}, {vq.dtype}")
    P = _contig.page_size_for(S)
    kp, vp = _contig.as_pages(kq, P), _contig.as_pages(vq, P)
    ksp, vsp = _contig.as_pages(ks, P), _contig.as_pages(vs, P)
    bt = _contig.identity_table(B, S, P, dev)
    q3 = q[:, 0].contiguous()
    ln = lengths_arr.to(device=dev, dtype=torch.int32).contiguous()
    out = torch.empty((B, Hq, D), dtype=q.dtype, device=dev)
    ws, ws_bytes = _lib.attention_workspace(dev, B, Hq, Hkv, D, S // P, P)
    _lib.launch("mk_paged_quantized_decode_attention", dev, _lib.ptr(q3), _lib.ptr(kp), _lib.ptr(vp), _lib.ptr(ksp),
                _lib.ptr(vsp), _lib.ptr(bt), _lib.ptr(ln), _lib.ptr(out), B, Hq, Hkv, D, P, S // P, kp.shape[0],
                cache.group_size, cache.bits, float(scale), _lib.dtype_code(q.dtype), _lib.ptr(ws), ws_bytes)
    return out.unsqueeze(1)


def quantized_kv_gqa_decode_attention(q, qkv_cache: QuantizedKVCache, lengths=None, *, scale=None,
                                      backend: str = "reference"):
    """ops/quantized_kv_cache_ops.py:506-541."""
    lengths_arr, B, MAX_S, Hq, Hkv, D = _validate_quantized_decode_inputs(q, qkv_cache, lengths)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    backend_name = backend.lower()
    if backend_name == "reference":
        return reference_quantized_kv_gqa_decode_attention(q, qkv_cache, lengths=lengths_arr, scale=scale)
    if backend_name == "metal_q8":
        if qkv_cache.bits != 8:
            raise ValueError(f"metal_q8 backend requires bits=8, got bits={qkv_cache.bits}")
        if D > _MAX_HEAD_DIM:
            raise ValueError(f"metal_q8 backend supports D <= {_MAX_HEAD_DIM}, got D={D}")
        return _hip_quantized_attention(q, qkv_cache, lengths_arr, scale)
    if backend_name == "metal_q4":
        if qkv_cache.bits != 4:
            raise ValueError(f"metal_q4 backend requires bits=4, got bits={qkv_cache.bits}")
        if D > _MAX_HEAD_DIM:
            raise ValueError(f"metal_q4 backend supports D <= {_MAX_HEAD_DIM}, got D={D}")
        return _hip_quantized_attention(q, qkv_cache, lengths_arr, scale)
    raise ValueError(f"backend must be one of 'reference', 'metal_q8', 'metal_q4', got {backend_name!r}")
