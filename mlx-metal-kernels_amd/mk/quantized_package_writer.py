"""Writes a quantized package's payload -- one .npy file per array under
``<output>/<tensor_subdir>/`` -- and then its ``package.json``
(models/quantized_package_writer.py).

File names follow the reference: ``layers.<i>.<key>.weight.npy`` /
``.scales.npy`` / ``.zeros.npy`` for the projections,
``layers.<i>.<norm key>.weight.npy`` for the norms and
``<name>.weight.npy`` for global tensors.  The metadata records each
relative path and the SHA-256 of the data (weight) file; ``package.json`` is
written only when every tensor was written.  Arrays may be numpy arrays or
torch tensors (device tensors are copied to the host).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from pathlib import Path
from typing import Any

from .quantized_layer_package import QuantizedLlamaLayerPackage
from .quantized_package_io import QuantizedCheckpointPackage, QuantizedTensorMetadata
from .tensor_data_io import save_tensor_npy


@dataclass
class PackageWriterConfig:
    """models/quantized_package_writer.py:12-24.  ``checksum_algorithm`` is
    validated but, as in the reference, the recorded checksums are SHA-256."""

    tensor_subdir: str = "tensors"
    checksum_algorithm: str = "sha256"

    def validate(self) -> "PackageWriterConfig":
        if not self.tensor_subdir:
            raise ValueError("tensor_subdir must be non-empty")
        if self.checksum_algorithm not in ("sha256", "sha1", "md5"):
            raise ValueError(f"checksum_algorithm must be one of sha256, sha1, md5, got {self.checksum_algorithm!r}")
        return self


@dataclass
class PackageWriterReport:
    """models/quantized_package_writer.py:27-39."""

    ok: bool
    files_written: list[str] = field(default_factory=list)
    errors: list[str] = field(default_factory=list)
    warnings: list[str] = field(default_factory=list)
    tensor_count: int = 0
    total_bytes: int = 0
    package_path: str | None = None

    def raise_for_errors(self) -> None:
        if self.errors:
            raise ValueError("; ".join(self.errors))


@dataclass
class TensorWriteInfo:
    file_path: str
    nbytes: int


class QuantizedPackageWriter:
    """models/quantized_package_writer.py:42-206."""

    def __init__(self, config: PackageWriterConfig | None = None):
        self._config = (config or PackageWriterConfig()).validate()

    def config(self) -> PackageWriterConfig:
        return self._config

    @staticmethod
    def _tensor_rel_path(layer_idx: int | None, name: str, suffix: str) -> str:
        return f"layers.{layer_idx}.{name}{suffix}" if layer_idx is not None else f"{name}{suffix}"

    def write_tensors(self, package: QuantizedCheckpointPackage, layer_packages: list[QuantizedLlamaLayerPackage],
                      output_dir: str | Path, *, global_tensors: dict[str, Any] | None = None) -> PackageWriterReport:
        """Write every layer tensor the metadata lists (from the matching layer
        package) and every global tensor given, filling in the metadata's file
        names and checksums; errors are collected per tensor, not raised."""
        out = Path(output_dir)
        tdir = out / self._config.tensor_subdir
        files, errors = [], []
        total = count = 0
        by_idx = {p.layer_idx: p for p in layer_packages}
        for meta in package.layers:
            pkg = by_idx.get(meta.layer_idx)
            if pkg is None:
                errors.append(f"layer {meta.layer_idx}: no QuantizedLlamaLayerPackage provided")
                continue
            for key, tmeta in meta.tensors.items():
                try:
                    info = self._write_layer_tensor(tdir, meta.layer_idx, key, tmeta, pkg)
                    files.append(info.file_path)
                    total += info.nbytes
                    count += 1
                except Exception as exc:  # noqa: BLE001 - reported per tensor
                    errors.append(f"layer {meta.layer_idx}, tensor {key}: {exc}")
        for name, data in (global_tensors or {}).items():
            try:
                tmeta = package.global_tensors.get(name)
                rel = self._tensor_rel_path(None, name, ".weight.npy")
                info = save_tensor_npy(data, tdir / rel)
                if tmeta:
                    tmeta.data_file = rel
                    tmeta.checksum = info.checksum
                files.append(info.file_path)
                total += info.nbytes
                count += 1
            except Exception as exc:  # noqa: BLE001
                errors.append(f"global tensor {name}: {exc}")
        path = str(out / "package.json")
        if not errors:
            package.save_json(out / "package.json")
        return PackageWriterReport(ok=not errors, files_written=files, errors=errors, warnings=[], tensor_count=count,
                                   total_bytes=total, package_path=path if (not errors or files) else None)

    def _write_layer_tensor(self, tdir: Path, layer_idx: int, key: str, tmeta: QuantizedTensorMetadata,
                            pkg: QuantizedLlamaLayerPackage) -> TensorWriteInfo:
        if tmeta.role in ("norm", "final_norm"):
            attr = key if key.endswith("_weight") else f"{key}_weight"
            weight = getattr(pkg, attr, None)
            if weight is None:
                raise ValueError(f"layer {layer_idx}: no weight attribute for norm {key}")
            rel = self._tensor_rel_path(layer_idx, key, ".weight.npy")
            info = save_tensor_npy(weight, tdir / rel)
            tmeta.data_file = rel
            tmeta.checksum = info.checksum
            return TensorWriteInfo(file_path=info.file_path, nbytes=info.nbytes)
        lin = getattr(pkg, key, None)
        if lin is None:
            raise ValueError(f"layer {layer_idx}: no attribute {key} on QuantizedLlamaLayerPackage")
        rel_w = self._tensor_rel_path(layer_idx, key, ".weight.npy")
        rel_s = self._tensor_rel_path(layer_idx, key, ".scales.npy")
        winfo = save_tensor_npy(lin.weight, tdir / rel_w)
        save_tensor_npy(lin.scales, tdir / rel_s)
        tmeta.data_file = rel_w
        tmeta.scales_file = rel_s
        tmeta.checksum = winfo.checksum
        if lin.zeros is not None:
            rel_z = self._tensor_rel_path(layer_idx, key, ".zeros.npy")
            save_tensor_npy(lin.zeros, tdir / rel_z)
            tmeta.zeros_file = rel_z
        return TensorWriteInfo(file_path=winfo.file_path, nbytes=winfo.nbytes)

    def write_package(self, package: QuantizedCheckpointPackage, layer_packages: list[QuantizedLlamaLayerPackage],
                      output_dir: str | Path, *, global_tensors: dict[str, Any] | None = None,
                      dry_run: bool = False) -> PackageWriterReport:
        """write_tensors, or with ``dry_run`` only the count of tensors it would
        write (nothing touches the disk)."""
        if dry_run:
            n = sum(len(l.tensors) for l in package.layers) + len(global_tensors or {})
            return PackageWriterReport(ok=True, tensor_count=n, package_path=str(Path(output_dir) / "package.json"))
        return self.write_tensors(package, layer_packages, output_dir, global_tensors=global_tensors)
