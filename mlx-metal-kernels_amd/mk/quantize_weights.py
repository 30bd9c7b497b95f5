"""Groupwise weight quantizer (models/quantize_weights.py:93-231).

``quantize_weight_groupwise`` turns an fp32/fp16/bf16 ``[out, in]`` weight on a
ROCm device into the packed codes and per-group scales the matvec kernels
consume, with one HIP launch (``mk_quantize_weight``).  Symmetric absmax per
group of ``group_size`` along ``in``: ``scale = max(max|w| / limit, eps)``
(limit 7 or 127), codes ``clip(rint(w / scale), -limit, limit) + 8 | 128``,
q4 packed two per byte (low nibble = even column).  ``zeros`` stay ``None``;
kernels take the implied zero point 8/128 (``kernel_zeros``,
models/quantized_layer_package.py:27-28).

``backend="reference"`` runs the same algorithm as torch ops on any device.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any

import torch

from . import _lib

_SCALE_DTYPES = {"float16": torch.float16, "bfloat16": torch.bfloat16, "float32": torch.float32}


def _symmetric_zero_point(bits: int) -> float:
    """models/quantize_weights.py:79-84."""
    if bits == 4:
        return 8.0
    if bits == 8:
        return 128.0
    raise ValueError(f"bits must be 4 or 8, got {bits}")


def _scale_dtype(name: str) -> torch.dtype:
    if name not in _SCALE_DTYPES:
        raise ValueError(f"dtype must be one of 'float16', 'bfloat16', 'float32', got {name!r}")
    return _SCALE_DTYPES[name]


@dataclass
class QuantizationConfig:
    """models/quantize_weights.py:93-109."""

    bits: int = 4
    group_size: int = 32
    symmetric: bool = True
    with_zeros: bool = False
    dtype: str = "float16"
    eps: float = 1e-8

    def validate(self) -> "QuantizationConfig":
        if self.bits not in (4, 8):
            raise ValueError(f"bits must be 4 or 8, got {self.bits}")
        if self.group_size <= 0:
            raise ValueError(f"group_size must be positive, got {self.group_size}")
        _scale_dtype(self.dtype)
        if self.eps <= 0:
            raise ValueError(f"eps must be positive, got {self.eps}")
        return self


@dataclass
class QuantizedWeight:
    """models/quantize_weights.py:112-161."""

    name: str | None
    bits: int
    group_size: int
    packed_weight: Any
    scales: Any
    zeros: Any | None = None
    original_shape: tuple[int, int] | None = None
    packed_shape: tuple[int, ...] | None = None
    scale_shape: tuple[int, ...] | None = None
    symmetric: bool = True

    def shapes(self) -> dict:
        return {
            "original_shape": self.original_shape,
            "packed_shape": self.packed_shape or tuple(self.packed_weight.shape),
            "scale_shape": self.scale_shape or tuple(self.scales.shape),
            "zeros_shape": None if self.zeros is None else tuple(self.zeros.shape),
        }

    def to_metadata(self) -> dict:
        return {"name": self.name, "bits": self.bits, "group_size": self.group_size,
                "symmetric": self.symmetric, **self.shapes()}

    def kernel_zeros(self):
        """The zero points the matvec kernels take (models/quantized_layer_package.py:27-28)."""
        if self.zeros is not None:
            return self.zeros
        return torch.full(tuple(self.scales.shape), _symmetric_zero_point(self.bits), dtype=self.scales.dtype,
                          device=self.scales.device)

    def validate(self) -> "QuantizedWeight":
        if self.bits not in (4, 8):
            raise ValueError(f"bits must be 4 or 8, got {self.bits}")
        if self.group_size <= 0:
            raise ValueError(f"group_size must be positive, got {self.group_size}")
        if self.original_shape is None:
            raise ValueError("original_shape must be provided")
        out_dim, in_dim = self.original_shape
        expected_packed = (out_dim, math.ceil(in_dim / 2)) if self.bits == 4 else (out_dim, in_dim)
        packed_shape = self.packed_shape or tuple(self.packed_weight.shape)
        scale_shape = self.scale_shape or tuple(self.scales.shape)
        if packed_shape != expected_packed:
            raise ValueError(f"packed_weight must have shape {expected_packed}, got {packed_shape}")
        groups = math.ceil(in_dim / self.group_size)
        if scale_shape != (out_dim, groups):
            raise ValueError(f"scales must have shape {(out_dim, groups)}, got {scale_shape}")
        if self.zeros is not None and tuple(self.zeros.shape) != (out_dim, groups):
            raise ValueError(f"zeros must have shape {(out_dim, groups)}, got {tuple(self.zeros.shape)}")
        return self


def _reference_quantize(w: torch.Tensor, bits: int, group_size: int, eps: float):
    """Tensor-op statement of models/quantize_weights.py:177-191."""
    w = w.to(torch.float32)
    out_dim, in_dim = w.shape
    groups = math.ceil(in_dim / group_size)
    pad = groups * group_size - in_dim
    wp = torch.nn.functional.pad(w, (0, pad)) if pad else w
    limit = 7 if bits == 4 else 127
    amax = wp.reshape(out_dim, groups, group_size).abs().amax(dim=-1).to(torch.float64)
    scale32 = torch.clamp(amax / float(limit), min=eps).to(torch.float32)
    full = scale32.repeat_interleave(group_size, dim=1)[:, :in_dim]
    q = torch.clamp(torch.round(w / full), -limit, limit).to(torch.int32) + int(_symmetric_zero_point(bits))
    q = q.to(torch.uint8)
    if bits == 4:
        if in_dim % 2:
            q = torch.nn.functional.pad(q, (0, 1))
        q = (q[:, 0::2] | (q[:, 1::2] << 4)).contiguous()
    return q, scale32


def quantize_weight_groupwise(weight, config: QuantizationConfig, *, backend: str = "auto") -> QuantizedWeight:
    """models/quantize_weights.py:164-203 (symmetric only, as the reference)."""
    config = config.validate()
    if not config.symmetric:
        raise NotImplementedError(
            "Asymmetric quantization is not implemented: the kernel path is defined around symmetric packaging.")
    if not isinstance(weight, torch.Tensor):
        raise TypeError(f"weight must be a torch.Tensor, got {type(weight).__name__}")
    if weight.ndim != 2:
        raise ValueError(f"weight must be rank-2 [OUT_DIM, IN_DIM], got {tuple(weight.shape)}")
    out_dim, in_dim = weight.shape
    sdt = _scale_dtype(config.dtype)
    name = backend.lower()
    if name == "reference":
        packed, s32 = _reference_quantize(weight, config.bits, config.group_size, config.eps)
        scales = s32.to(sdt)
    elif name in ("auto", "metal"):
        w = weight if weight.dtype in (torch.float16, torch.bfloat16, torch.float32) else weight.to(torch.float32)
        w = w.contiguous()
        dev = _lib.require_device(w)
        groups = math.ceil(in_dim / config.group_size)
        cols = (in_dim + 1) // 2 if config.bits == 4 else in_dim
        packed = torch.empty((out_dim, cols), dtype=torch.uint8, device=dev)
        scales = torch.empty((out_dim, groups), dtype=sdt, device=dev)
        _lib.launch("mk_quantize_weight", dev, _lib.ptr(w), _lib.ptr(packed), _lib.ptr(scales), out_dim, in_dim,
                    config.group_size, config.bits, float(config.eps), _lib.dtype_code(w.dtype),
                    _lib.dtype_code(sdt))
    else:
        raise ValueError("backend must be one of 'reference', 'metal', 'auto'")
    return QuantizedWeight(
        name=None, bits=config.bits, group_size=config.group_size, packed_weight=packed, scales=scales, zeros=None,
        original_shape=(int(out_dim), int(in_dim)), packed_shape=tuple(packed.shape),
        scale_shape=tuple(scales.shape), symmetric=True,
    ).validate()


def dequantize_quantized_weight(q_weight, scales, zeros=None, *, bits=4, group_size=32, backend: str = "auto"):
    """models/quantize_weights.py:206-231: ``(q - z) * s`` as fp16 (HIP
    dequant kernels on the device; zeros default to 8/128)."""
    from .quant_ops import dequant_q4, dequant_q8

    if bits not in (4, 8):
        raise ValueError(f"bits must be 4 or 8, got {bits}")
    if zeros is None:
        zeros = torch.full(tuple(scales.shape), _symmetric_zero_point(bits), dtype=torch.float32,
                           device=scales.device)
    fn = dequant_q4 if bits == 4 else dequant_q8
    return fn(q_weight, scales, zeros, group_size=group_size, out_dtype=torch.float16, backend=backend)
