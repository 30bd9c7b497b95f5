"""Quantized checkpoint package: the ``package.json`` metadata of a q4/q8
Llama-like model and its per-tensor payload files (models/quantized_package_io.py),
plus the loader that brings a written package into HBM as the kernel weights
of ``mk.llama_stack_ops``.

The JSON layout, field names, validation rules and error messages follow the
reference, so a package written by either side loads on the other.
"""

from __future__ import annotations

import json
from dataclasses import asdict, dataclass, field
from pathlib import Path
from typing import Any

from .llama_layer_ops import LlamaLikeConfig
from .quantized_layer_package import QuantizedLinearPackage, QuantizedLlamaLayerPackage
from .tensor_data_io import load_tensor_to_device, validate_tensor_file

_REQUIRED_LAYER_TENSOR_KEYS = ["input_layernorm", "post_attention_layernorm", "qkv", "o_proj", "gate_proj",
                               "up_proj", "down_proj"]
_VALID_ROLES = ["qkv", "o_proj", "gate_proj", "up_proj", "down_proj", "embedding", "lm_head", "norm", "final_norm",
                "other"]
_FORMAT_VERSION = "0.1.0"
_LINEAR_KEYS = ("qkv", "o_proj", "gate_proj", "up_proj", "down_proj")


@dataclass
class QuantizedTensorMetadata:
    """models/quantized_package_io.py:37-85."""

    name: str
    role: str
    bits: int
    group_size: int
    original_shape: tuple[int, ...]
    packed_shape: tuple[int, ...]
    scales_shape: tuple[int, ...]
    zeros_shape: tuple[int, ...] | None = None
    dtype: str = "float16"
    data_file: str | None = None
    scales_file: str | None = None
    zeros_file: str | None = None
    checksum: str | None = None

    def to_dict(self) -> dict[str, Any]:
        d = asdict(self)
        for k in ("original_shape", "packed_shape", "scales_shape"):
            d[k] = list(getattr(self, k))
        if self.zeros_shape is not None:
            d["zeros_shape"] = list(self.zeros_shape)
        return d

    @classmethod
    def from_dict(cls, data: dict[str, Any]) -> "QuantizedTensorMetadata":
        zs = data.get("zeros_shape")
        return cls(name=data["name"], role=data["role"], bits=data["bits"], group_size=data["group_size"],
                   original_shape=tuple(data["original_shape"]), packed_shape=tuple(data["packed_shape"]),
                   scales_shape=tuple(data["scales_shape"]), zeros_shape=tuple(zs) if zs is not None else None,
                   dtype=data.get("dtype", "float16"), data_file=data.get("data_file"),
                   scales_file=data.get("scales_file"), zeros_file=data.get("zeros_file"),
                   checksum=data.get("checksum"))


@dataclass
class QuantizedLayerMetadata:
    """models/quantized_package_io.py:88-101."""

    layer_idx: int
    tensors: dict[str, QuantizedTensorMetadata]

    def to_dict(self) -> dict[str, Any]:
        return {"layer_idx": self.layer_idx, "tensors": {k: t.to_dict() for k, t in self.tensors.items()}}

    @classmethod
    def from_dict(cls, data: dict[str, Any]) -> "QuantizedLayerMetadata":
        return cls(layer_idx=data["layer_idx"],
                   tensors={k: QuantizedTensorMetadata.from_dict(t) for k, t in data.get("tensors", {}).items()})


def _iter_all_tensors(package: "QuantizedCheckpointPackage"):
    for name, tensor in package.global_tensors.items():
        yield f"global_tensors.{name}", tensor
    for layer in package.layers:
        for name, tensor in layer.tensors.items():
            yield f"layers[{layer.layer_idx}].tensors.{name}", tensor


def _resolve(rel: str, base: Path | None) -> Path:
    p = Path(rel)
    return base / p if base is not None and not p.is_absolute() else p


def _payload_path(rel: str, base: Path, tensor_subdir: str) -> Path:
    """Where a payload file of a written package lives.  The writer records
    names relative to the tensor folder (models/quantized_package_writer.py:
    122-130 and 170-175: ``data_file = "layers.0.qkv.weight.npy"`` for a file
    under ``<package>/tensors/``), other tools relative to the package folder;
    both are accepted, the package folder first."""
    direct = _resolve(rel, base)
    if direct.exists():
        return direct
    nested = _resolve(rel, base / tensor_subdir)
    return nested if nested.exists() else direct


@dataclass
class QuantizedCheckpointPackage:
    """models/quantized_package_io.py:104-329."""

    format_version: str = _FORMAT_VERSION
    model_type: str = "llama_like"
    config: dict[str, Any] = field(default_factory=dict)
    quantization: dict[str, Any] = field(default_factory=dict)
    layers: list[QuantizedLayerMetadata] = field(default_factory=list)
    global_tensors: dict[str, QuantizedTensorMetadata] = field(default_factory=dict)
    metadata: dict[str, Any] = field(default_factory=dict)

    def to_dict(self) -> dict[str, Any]:
        return {"format_version": self.format_version, "model_type": self.model_type, "config": dict(self.config),
                "quantization": dict(self.quantization), "layers": [l.to_dict() for l in self.layers],
                "global_tensors": {k: t.to_dict() for k, t in self.global_tensors.items()},
                "metadata": dict(self.metadata)}

    @classmethod
    def from_dict(cls, data: dict[str, Any]) -> "QuantizedCheckpointPackage":
        return cls(format_version=data.get("format_version", _FORMAT_VERSION),
                   model_type=data.get("model_type", "llama_like"), config=data.get("config", {}),
                   quantization=data.get("quantization", {}),
                   layers=[QuantizedLayerMetadata.from_dict(l) for l in data.get("layers", [])],
                   global_tensors={k: QuantizedTensorMetadata.from_dict(t)
                                   for k, t in data.get("global_tensors", {}).items()},
                   metadata=data.get("metadata", {}))

    def save_json(self, path: str | Path) -> None:
        target = Path(path)
        target.parent.mkdir(parents=True, exist_ok=True)
        target.write_text(json.dumps(self.to_dict(), indent=2), encoding="utf-8")

    @classmethod
    def load_json(cls, path: str | Path) -> "QuantizedCheckpointPackage":
        return cls.from_dict(json.loads(Path(path).read_text(encoding="utf-8")))

    def has_tensor_data(self, *, require_all: bool = True) -> bool:
        """Whether every quantized tensor names its data and scales files
        (norm tensors, bits 0, are not required to)."""
        for _, t in _iter_all_tensors(self):
            if t.bits == 0:
                continue
            if (t.data_file is None or t.scales_file is None) and require_all:
                return False
        return True

    def tensor_files(self, base_dir: str | Path | None = None) -> dict[str, str]:
        """``"<tensor>.<data|scales|zeros>_file"`` -> path (joined to
        ``base_dir`` when relative)."""
        out: dict[str, str] = {}
        base = Path(base_dir).resolve() if base_dir is not None else None
        for fname, t in _iter_all_tensors(self):
            for attr in ("data_file", "scales_file", "zeros_file"):
                rel = getattr(t, attr)
                if rel is not None:
                    out[f"{fname}.{attr}"] = str(_resolve(rel, base))
        return out

    def validate_tensor_files(self, base_dir: str | Path | None = None, *, check_checksums: bool = False) -> list[str]:
        """Problems with the payload files, as messages (the checksum, when
        asked for, is the data file's)."""
        issues: list[str] = []
        base = Path(base_dir).resolve() if base_dir is not None else None
        for fname, t in _iter_all_tensors(self):
            if t.bits == 0 and t.data_file is None:
                continue
            for attr in ("data_file", "scales_file", "zeros_file"):
                rel = getattr(t, attr)
                if rel is None:
                    if t.bits != 0 or attr != "data_file":
                        continue
                    issues.append(f"{fname}.{attr}: not set")
                    continue
                want = t.checksum if check_checksums and attr == "data_file" else None
                issues += [f"{fname}.{attr}: {m}" for m in validate_tensor_file(_resolve(rel, base),
                                                                                 expected_checksum=want)]
        return issues

    def validate(self, *, allow_partial: bool = False) -> "QuantizedCheckpointPackage":
        """models/quantized_package_io.py:219-284."""
        if not self.format_version:
            raise ValueError("format_version must be non-empty")
        if not self.model_type:
            raise ValueError("model_type must be non-empty")
        if not self.layers and not allow_partial:
            raise ValueError("package must contain at least one layer unless allow_partial=True")
        seen: set[int] = set()
        for layer in self.layers:
            if layer.layer_idx < 0:
                raise ValueError(f"layer_idx must be non-negative, got {layer.layer_idx}")
            if layer.layer_idx in seen:
                raise ValueError(f"duplicate layer_idx: {layer.layer_idx}")
            seen.add(layer.layer_idx)
            for key in _REQUIRED_LAYER_TENSOR_KEYS:
                if key not in layer.tensors and not allow_partial:
                    raise ValueError(f"layer {layer.layer_idx} missing required tensor key: {key!r}")
            for t in layer.tensors.values():
                if any(d <= 0 for d in t.original_shape):
                    raise ValueError(f"tensor {t.name!r} original_shape contains non-positive dims: "
                                     f"{t.original_shape}")
                if t.role not in _VALID_ROLES:
                    raise ValueError(f"tensor {t.name!r} has invalid role {t.role!r}; expected one of {_VALID_ROLES}")
                if t.role in ("norm", "final_norm"):
                    if t.bits != 0:
                        raise ValueError(f"tensor {t.name!r} is unquantized norm metadata and must use bits=0, "
                                         f"got {t.bits}")
                    if t.group_size != 0:
                        raise ValueError(f"tensor {t.name!r} is unquantized norm metadata and must use "
                                         f"group_size=0, got {t.group_size}")
                    continue
                if t.bits not in (4, 8):
                    raise ValueError(f"tensor {t.name!r} bits must be 4 or 8, got {t.bits}")
                if t.group_size <= 0:
                    raise ValueError(f"tensor {t.name!r} group_size must be positive, got {t.group_size}")
        if not allow_partial and seen:
            lo, hi = min(seen), max(seen)
            missing = sorted(set(range(lo, hi + 1)) - seen)
            if missing:
                raise ValueError(f"layer indices must be contiguous from {lo} to {hi}, missing indices: {missing}")
        return self

    def num_layers(self) -> int:
        return len(self.layers)

    def tensor_count(self) -> int:
        return len(self.global_tensors) + sum(len(l.tensors) for l in self.layers)

    def summary(self) -> dict[str, Any]:
        return {"format_version": self.format_version, "model_type": self.model_type,
                "num_layers": self.num_layers(), "tensor_count": self.tensor_count(),
                "bits": self.quantization.get("bits"), "group_size": self.quantization.get("group_size"),
                "config_keys": list(self.config.keys()),
                "per_layer": {str(l.layer_idx): {n: list(t.original_shape) for n, t in l.tensors.items()}
                              for l in self.layers},
                "global_tensors": list(self.global_tensors.keys())}


def _shape(a) -> tuple[int, ...]:
    return tuple(int(d) for d in a.shape)


def _linear_metadata(name: str, role: str, pkg: QuantizedLlamaLayerPackage, qkv_rows: int | None):
    """models/quantized_package_io.py:332-368: the fused qkv's original shape
    is (q + 2 kv output dims, hidden)."""
    if role not in _LINEAR_KEYS:
        raise ValueError(f"unsupported role for linear tensor: {role!r}")
    lin: QuantizedLinearPackage = getattr(pkg, role)
    shape = (qkv_rows, lin.original_shape[1]) if role == "qkv" else tuple(lin.original_shape)
    return QuantizedTensorMetadata(name=name, role=role, bits=lin.bits, group_size=lin.group_size,
                                   original_shape=shape, packed_shape=_shape(lin.weight),
                                   scales_shape=_shape(lin.scales),
                                   zeros_shape=_shape(lin.zeros) if lin.zeros is not None else None, dtype="float16")


def _norm_metadata(name: str, weight) -> QuantizedTensorMetadata:
    """models/quantized_package_io.py:371-382."""
    shape = _shape(weight) if hasattr(weight, "shape") else (0,)
    return QuantizedTensorMetadata(name=name, role="norm", bits=0, group_size=0, original_shape=shape,
                                   packed_shape=shape, scales_shape=(0,), dtype="float16")


def package_from_quantized_layers(config: LlamaLikeConfig, quantized_layers: list[QuantizedLlamaLayerPackage], *,
                                  bits: int = 4, group_size: int = 32, model_type: str = "llama_like",
                                  symmetric: bool = True, with_zeros: bool = False,
                                  metadata: dict[str, Any] | None = None) -> QuantizedCheckpointPackage:
    """The package metadata of a list of layer packages
    (models/quantized_package_io.py:385-430)."""
    config.validate()
    qkv_rows = config.q_output_dim() + 2 * config.kv_output_dim()
    layers = []
    for pkg in quantized_layers:
        i = pkg.layer_idx
        tensors = {k: _linear_metadata(f"layers.{i}.{k}", k, pkg, qkv_rows) for k in _LINEAR_KEYS}
        if pkg.input_layernorm_weight is not None:
            tensors["input_layernorm"] = _norm_metadata(f"layers.{i}.input_layernorm", pkg.input_layernorm_weight)
        if pkg.post_attention_layernorm_weight is not None:
            tensors["post_attention_layernorm"] = _norm_metadata(f"layers.{i}.post_attention_layernorm",
                                                                 pkg.post_attention_layernorm_weight)
        layers.append(QuantizedLayerMetadata(layer_idx=i, tensors=tensors))
    return QuantizedCheckpointPackage(format_version=_FORMAT_VERSION, model_type=model_type,
                                      config=config.to_dict(),
                                      quantization={"bits": bits, "group_size": group_size, "symmetric": symmetric,
                                                    "with_zeros": with_zeros},
                                      layers=layers, metadata=metadata or {})


# ------------------------------------------------------------- into HBM


def load_layer_package(package: QuantizedCheckpointPackage, base_dir: str | Path, layer_idx: int, device, *,
                       dtype=None, check_checksums: bool = True,
                       tensor_subdir: str = "tensors") -> QuantizedLlamaLayerPackage:
    """Layer ``layer_idx`` of a written package as device tensors in the
    kernels' layout (codes uint8, scales/zeros float16 -- symmetric zeros
    materialised when the package stores none --, norm weights in ``dtype``,
    default float16).  Every payload file is checked against the metadata's
    packed/scales/zeros shapes and, with ``check_checksums``, the data file's
    SHA-256 before it is copied; a mismatch raises ValueError."""
    import torch

    base = Path(base_dir)
    layer = next((l for l in package.layers if l.layer_idx == layer_idx), None)
    if layer is None:
        raise ValueError(f"package has no layer {layer_idx}")
    act = torch.float16 if dtype is None else dtype

    def need(t: QuantizedTensorMetadata, attr: str) -> str:
        rel = getattr(t, attr)
        if rel is None:
            raise ValueError(f"layer {layer_idx} tensor {t.name!r}: {attr} not set (package has no tensor data)")
        return str(_payload_path(rel, base, tensor_subdir))

    lins = {}
    for key in _LINEAR_KEYS:
        t = layer.tensors[key]
        w = load_tensor_to_device(need(t, "data_file"), device, dtype=torch.uint8, expected_shape=t.packed_shape,
                                  expected_checksum=t.checksum if check_checksums else None)
        s = load_tensor_to_device(need(t, "scales_file"), device, dtype=torch.float16, expected_shape=t.scales_shape)
        z = None
        if t.zeros_file is not None:
            z = load_tensor_to_device(need(t, "zeros_file"), device, dtype=torch.float16,
                                      expected_shape=t.zeros_shape)
        lin = QuantizedLinearPackage(name=t.name, weight=w, scales=s, zeros=z, bits=t.bits,
                                     group_size=t.group_size, original_shape=tuple(t.original_shape))
        if lin.zeros is None:
            lin.zeros = lin.kernel_zeros()
        lins[key] = lin
    norms = {}
    for key in ("input_layernorm", "post_attention_layernorm"):
        t = layer.tensors[key]
        norms[key] = load_tensor_to_device(need(t, "data_file"), device, dtype=act, expected_shape=t.packed_shape,
                                           expected_checksum=t.checksum if check_checksums else None)
    return QuantizedLlamaLayerPackage(layer_idx=layer_idx, input_layernorm_weight=norms["input_layernorm"],
                                      post_attention_layernorm_weight=norms["post_attention_layernorm"], **lins)


def load_quantized_stack(package_dir: str | Path, device, *, dtype=None, check_checksums: bool = True,
                         lm_head_bits: int | None = None, lm_head_group_size: int = 32,
                         tensor_subdir: str = "tensors"):
    """A written package (``package_dir/package.json`` + payload) as
    ``(config, LlamaStackWeights)`` on ``device``: every layer through
    load_layer_package and to_kernel_weights; the ``norm`` / ``embedding`` /
    ``lm_head`` global tensors when present, in ``dtype``.  With
    ``lm_head_bits`` (4 or 8) the head is quantized on the device for the
    q4/q8 head matvec; otherwise it stays dense."""
    import torch

    from .llama_stack_ops import LlamaStackWeights, QuantizedHead
    from .quantize_weights import QuantizationConfig, quantize_weight_groupwise

    base = Path(package_dir)
    package = QuantizedCheckpointPackage.load_json(base / "package.json").validate()
    config = LlamaLikeConfig.from_dict(package.config)
    act = torch.float16 if dtype is None else dtype
    layers = [load_layer_package(package, base, l.layer_idx, device, dtype=act, check_checksums=check_checksums,
                                 tensor_subdir=tensor_subdir).to_kernel_weights(config)
              for l in sorted(package.layers, key=lambda l: l.layer_idx)]

    def global_tensor(name):
        t = package.global_tensors.get(name)
        if t is None or t.data_file is None:
            return None
        return load_tensor_to_device(str(_payload_path(t.data_file, base, tensor_subdir)), device, dtype=act,
                                     expected_shape=t.packed_shape,
                                     expected_checksum=t.checksum if check_checksums else None)

    final_norm = global_tensor("norm")
    if final_norm is None:
        final_norm = torch.ones(config.hidden_size, dtype=act, device=device)
    embedding = global_tensor("embedding")
    lm_head = global_tensor("lm_head")
    if lm_head is not None and lm_head_bits is not None:
        q = quantize_weight_groupwise(lm_head, QuantizationConfig(bits=lm_head_bits, group_size=lm_head_group_size))
        lm_head = QuantizedHead(w=q.packed_weight, scales=q.scales, zeros=q.kernel_zeros(), bits=lm_head_bits,
                                group_size=lm_head_group_size)
    stack = LlamaStackWeights(layers=layers, final_norm_weight=final_norm, lm_head=lm_head, embedding=embedding)
    return config, stack.validate(config)
