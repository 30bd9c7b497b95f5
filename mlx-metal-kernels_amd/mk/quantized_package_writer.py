"""Writer of a quantized package's payload and ``package.json``.

What is fixed by the on-disk format (models/quantized_package_writer.py:42-206,
the files and fields the reference's loader and ours read back):

* one ``.npy`` per array under ``<output>/<tensor_subdir>/``, named
  ``layers.<i>.<key>.weight.npy`` / ``.scales.npy`` / ``.zeros.npy`` for a
  projection, ``layers.<i>.<norm key>.weight.npy`` for a norm (taken from the
  layer package's ``<key>_weight`` attribute) and ``<name>.weight.npy`` for a
  global tensor;
* the metadata records those names relative to the tensor folder and the
  SHA-256 of each weight (data) file;
* ``package.json`` is written only when every tensor was written; the report
  carries the same fields, messages and counts.

How it is done here: the writer first turns the metadata into a flat plan --
one entry per tensor, holding the files to write and where each name goes in
the metadata -- without touching the disk (a dry run is that plan's size).  It
then streams every array through a sink that feeds the file and the hash
together, so each payload is written once and never read back to checksum
it, and records a tensor's file names and checksum in the metadata only once
all of that tensor's files are on disk.  Arrays may be numpy arrays or torch
tensors (device tensors are copied to the host).
"""

from __future__ import annotations

import hashlib
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any

import numpy as np

from .quantized_layer_package import QuantizedLlamaLayerPackage
from .quantized_package_io import QuantizedCheckpointPackage, QuantizedTensorMetadata
from .tensor_data_io import _as_numpy

_CHECKSUMS = ("sha256", "sha1", "md5")
_NORM_ROLES = ("norm", "final_norm")


@dataclass
class PackageWriterConfig:
    """models/quantized_package_writer.py:12-24.  ``checksum_algorithm`` is
    validated, but the recorded checksums are SHA-256, the digest the
    package loader verifies."""

    tensor_subdir: str = "tensors"
    checksum_algorithm: str = "sha256"

    def validate(self) -> "PackageWriterConfig":
        if not self.tensor_subdir:
            raise ValueError("tensor_subdir must be non-empty")
        if self.checksum_algorithm not in _CHECKSUMS:
            raise ValueError(f"checksum_algorithm must be one of {', '.join(_CHECKSUMS)}, "
                             f"got {self.checksum_algorithm!r}")
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
    """One written tensor: its data file and the data's size in bytes."""

    file_path: str
    nbytes: int


class _HashSink:
    """File-like target for ``np.lib.format.write_array``: every piece goes to
    the file and into the digest, so the checksum needs no second read."""

    def __init__(self, fh, digest):
        self._fh = fh
        self._digest = digest

    def write(self, data) -> int:
        self._digest.update(data)
        return self._fh.write(data)


def _stream_npy(array: Any, path: Path) -> tuple[int, str]:
    """Write ``array`` as numpy's ``.npy`` encoding (the bytes ``np.save``
    produces) and return (data bytes, SHA-256 of the file)."""
    arr = _as_numpy(array)
    if arr.dtype.hasobject:
        raise TypeError("object arrays cannot be written to a tensor payload")
    path.parent.mkdir(parents=True, exist_ok=True)
    digest = hashlib.sha256()
    with path.open("wb") as fh:
        np.lib.format.write_array(_HashSink(fh, digest), arr, allow_pickle=False)
    return int(arr.nbytes), digest.hexdigest()


# (metadata field, file suffix); the first file of a tensor is its data file
_PROJ_FILES = (("data_file", ".weight.npy"), ("scales_file", ".scales.npy"), ("zeros_file", ".zeros.npy"))
_WEIGHT_ONLY = (("data_file", ".weight.npy"),)


@dataclass
class _Entry:
    """One tensor of the plan: the error label, the files as (metadata
    field, relative name, array), the metadata object to fill in, or the
    reason the tensor cannot be written."""

    label: str
    files: list[tuple[str, str, Any]] = field(default_factory=list)
    meta: QuantizedTensorMetadata | None = None
    problem: str | None = None


def _layer_entry(layer_idx: int, key: str, meta: QuantizedTensorMetadata,
                 pkg: QuantizedLlamaLayerPackage) -> _Entry:
    entry = _Entry(label=f"layer {layer_idx}, tensor {key}", meta=meta)
    stem = f"layers.{layer_idx}.{key}"
    if meta.role in _NORM_ROLES:
        attr = key if key.endswith("_weight") else f"{key}_weight"
        weight = getattr(pkg, attr, None)
        if weight is None:
            entry.problem = f"layer {layer_idx}: no weight attribute for norm {key}"
            return entry
        arrays: tuple[Any, ...] = (weight,)
        spec = _WEIGHT_ONLY
    else:
        lin = getattr(pkg, key, None)
        if lin is None:
            entry.problem = f"layer {layer_idx}: no attribute {key} on QuantizedLlamaLayerPackage"
            return entry
        arrays = (lin.weight, lin.scales, lin.zeros)
        spec = _PROJ_FILES
    for (slot, suffix), arr in zip(spec, arrays):
        if arr is not None:
            entry.files.append((slot, stem + suffix, arr))
    return entry


class QuantizedPackageWriter:
    """models/quantized_package_writer.py:42-206 (the files, metadata fields
    and report it produces)."""

    def __init__(self, config: PackageWriterConfig | None = None):
        self._config = (config or PackageWriterConfig()).validate()

    def config(self) -> PackageWriterConfig:
        return self._config

    # -- plan --------------------------------------------------------------
    def plan(self, package: QuantizedCheckpointPackage, layer_packages: list[QuantizedLlamaLayerPackage],
             global_tensors: dict[str, Any] | None = None) -> list[_Entry]:
        """The tensors a write would produce, in write order, with no I/O.  A
        layer without a package is one entry that cannot be written."""
        found = {p.layer_idx: p for p in layer_packages}
        entries: list[_Entry] = []
        for layer in package.layers:
            pkg = found.get(layer.layer_idx)
            if pkg is None:
                entries.append(_Entry(label=f"layer {layer.layer_idx}", problem="no QuantizedLlamaLayerPackage provided"))
                continue
            entries.extend(_layer_entry(layer.layer_idx, key, meta, pkg) for key, meta in layer.tensors.items())
        for name, data in (global_tensors or {}).items():
            entries.append(_Entry(label=f"global tensor {name}", files=[("data_file", f"{name}.weight.npy", data)],
                                  meta=package.global_tensors.get(name)))
        return entries

    # -- execute -----------------------------------------------------------
    def _write_entry(self, tdir: Path, entry: _Entry) -> TensorWriteInfo:
        if entry.problem is not None:
            raise ValueError(entry.problem)
        written: list[tuple[str, str, int, str]] = []
        for slot, rel, arr in entry.files:
            nbytes, digest = _stream_npy(arr, tdir / rel)
            written.append((slot, rel, nbytes, digest))
        _, data_rel, data_bytes, data_digest = written[0]
        if entry.meta is not None:  # recorded only once every file is on disk
            for slot, rel, _, _ in written:
                setattr(entry.meta, slot, rel)
            entry.meta.checksum = data_digest
        return TensorWriteInfo(file_path=str(tdir / data_rel), nbytes=data_bytes)

    def write_tensors(self, package: QuantizedCheckpointPackage, layer_packages: list[QuantizedLlamaLayerPackage],
                      output_dir: str | Path, *, global_tensors: dict[str, Any] | None = None) -> PackageWriterReport:
        """Write every planned tensor, fill in the metadata's file names and
        checksums, and save ``package.json`` if nothing failed.  Failures are
        reported per tensor, not raised."""
        out = Path(output_dir)
        tdir = out / self._config.tensor_subdir
        report = PackageWriterReport(ok=False)
        for entry in self.plan(package, layer_packages, global_tensors):
            try:
                info = self._write_entry(tdir, entry)
            except Exception as exc:  # noqa: BLE001 - reported per tensor
                report.errors.append(f"{entry.label}: {exc}")
                continue
            report.files_written.append(info.file_path)
            report.total_bytes += info.nbytes
            report.tensor_count += 1
        json_path = out / "package.json"
        report.ok = not report.errors
        if report.ok:
            package.save_json(json_path)
        report.package_path = str(json_path) if (report.ok or report.files_written) else None
        return report

    def write_package(self, package: QuantizedCheckpointPackage, layer_packages: list[QuantizedLlamaLayerPackage],
                      output_dir: str | Path, *, global_tensors: dict[str, Any] | None = None,
                      dry_run: bool = False) -> PackageWriterReport:
        """``write_tensors``; with ``dry_run`` only the number of tensors the
        metadata and ``global_tensors`` name (nothing touches the disk)."""
        if dry_run:
            count = sum(len(layer.tensors) for layer in package.layers) + len(global_tensors or {})
            return PackageWriterReport(ok=True, tensor_count=count, package_path=str(Path(output_dir) / "package.json"))
        return self.write_tensors(package, layer_packages, output_dir, global_tensors=global_tensors)
