"""A quantized Llama-like layer as a package of arrays: the five projections
(codes, scales, optional zeros) and the two norm weights
(models/quantized_layer_package.py), convertible to the kernel weights of
``mk.llama_layer_ops`` and movable to HBM.

Members may be numpy arrays (a package read from disk) or torch tensors.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any

import numpy as np

from .llama_layer_ops import LlamaLayerKernelWeights, LlamaLikeConfig


def _shape_tuple(value: Any) -> tuple[int, ...] | None:
    shape = getattr(value, "shape", None)
    return None if shape is None else tuple(int(d) for d in shape)


def _symmetric_zeros(scales: Any, bits: int):
    """The zero points of a symmetric quantization -- 8 (q4) or 128 (q8) per
    group -- shaped like ``scales`` (models/quantize_weights.py:87-89): float32
    for numpy scales, the scales' dtype and device for torch scales."""
    zp = 8.0 if bits == 4 else 128.0
    try:
        import torch

        if isinstance(scales, torch.Tensor):
            return torch.full_like(scales, zp)
    except ImportError:  # pragma: no cover
        pass
    return np.full(_shape_tuple(scales), zp, dtype=np.float32)


@dataclass
class QuantizedLinearPackage:
    """One quantized projection (models/quantized_layer_package.py:9-26)."""

    name: str
    weight: Any
    scales: Any
    zeros: Any | None
    bits: int
    group_size: int
    original_shape: tuple[int, int]

    def shapes(self) -> dict[str, tuple[int, ...] | None]:
        return {"weight": _shape_tuple(self.weight), "scales": _shape_tuple(self.scales),
                "zeros": _shape_tuple(self.zeros), "original_shape": self.original_shape}

    def kernel_zeros(self):
        """The zero points the matvec kernels take: the stored ones, else the
        symmetric ones (models/quantized_layer_package.py:27-28)."""
        return self.zeros if self.zeros is not None else _symmetric_zeros(self.scales, self.bits)


@dataclass
class QuantizedLlamaLayerPackage:
    """models/quantized_layer_package.py:31-140."""

    layer_idx: int
    input_layernorm_weight: Any
    post_attention_layernorm_weight: Any
    qkv: QuantizedLinearPackage
    o_proj: QuantizedLinearPackage
    gate_proj: QuantizedLinearPackage
    up_proj: QuantizedLinearPackage
    down_proj: QuantizedLinearPackage

    _LINEARS = ("qkv", "o_proj", "gate_proj", "up_proj", "down_proj")

    def shapes(self) -> dict[str, Any]:
        out = {"input_layernorm_weight": _shape_tuple(self.input_layernorm_weight),
               "post_attention_layernorm_weight": _shape_tuple(self.post_attention_layernorm_weight)}
        out.update({k: getattr(self, k).shapes() for k in self._LINEARS})
        return out

    def to_kernel_weights(self, config: LlamaLikeConfig) -> LlamaLayerKernelWeights:
        """The layer's LlamaLayerKernelWeights, validated against ``config``
        (models/quantized_layer_package.py:117-140); zeros default to the
        symmetric ones."""
        p = {}
        for key, short in (("qkv", "qkv"), ("o_proj", "o"), ("gate_proj", "gate"), ("up_proj", "up"),
                           ("down_proj", "down")):
            lin = getattr(self, key)
            p[f"{short}_w"] = lin.weight
            p[f"{short}_scales"] = lin.scales
            p[f"{short}_zeros"] = lin.kernel_zeros()
        weights = LlamaLayerKernelWeights(input_layernorm_weight=self.input_layernorm_weight,
                                          post_attention_layernorm_weight=self.post_attention_layernorm_weight,
                                          bits=self.qkv.bits, group_size=self.qkv.group_size, **p)
        return weights.validate(config)

    def to_device(self, device, *, dtype=None) -> "QuantizedLlamaLayerPackage":
        """A copy whose arrays are torch tensors on ``device`` in the layout the
        HIP kernels take: codes uint8, scales and zeros float16 (symmetric zeros
        materialised), norm weights in ``dtype`` (default float16)."""
        import torch

        act = torch.float16 if dtype is None else dtype

        def dev(a, dt):
            t = a if isinstance(a, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(a))
            return t.to(device=device, dtype=dt).contiguous()

        lins = {}
        for key in self._LINEARS:
            lin = getattr(self, key)
            lins[key] = QuantizedLinearPackage(name=lin.name, weight=dev(lin.weight, torch.uint8),
                                               scales=dev(lin.scales, torch.float16),
                                               zeros=dev(lin.kernel_zeros(), torch.float16), bits=lin.bits,
                                               group_size=lin.group_size, original_shape=tuple(lin.original_shape))
        return QuantizedLlamaLayerPackage(layer_idx=self.layer_idx,
                                          input_layernorm_weight=dev(self.input_layernorm_weight, act),
                                          post_attention_layernorm_weight=dev(self.post_attention_layernorm_weight,
                                                                              act), **lins)
