"""Tensor payload files of a quantized package: one ``.npy`` file per array,
identified by its SHA-256 -- the on-disk format of models/tensor_data_io.py,
plus a loader that streams a payload file into HBM.

The file format is numpy's own ``.npy`` (np.save of the array as given), so
packages written here and by the reference are byte-identical for the same
arrays and their checksums agree.  Files are read without unpickling
(``allow_pickle=False``).

``load_tensor_to_device`` is the MI355X side: a memory-mapped payload goes to
the GPU through two pinned staging buffers in fixed-size chunks, so a tensor
of any size (a 1 GiB embedding, a 32-layer stack) is never held whole in host
memory and the PCIe copy of one chunk overlaps the file read of the next.
"""

from __future__ import annotations

import hashlib
from dataclasses import dataclass
from pathlib import Path
from typing import Any

import numpy as np

_CHUNK_BYTES = 64 << 20


@dataclass
class TensorDataInfo:
    """models/tensor_data_io.py:9-15."""

    file_path: str
    shape: tuple[int, ...]
    dtype: str
    nbytes: int
    checksum: str


def compute_file_checksum(file_path: str | Path, algorithm: str = "sha256") -> str:
    """Hex digest of a file, read in 64 KiB pieces (models/tensor_data_io.py:22-28)."""
    h = hashlib.new(algorithm)
    with Path(file_path).open("rb") as f:
        for piece in iter(lambda: f.read(65536), b""):
            h.update(piece)
    return h.hexdigest()


def _as_numpy(tensor: Any) -> np.ndarray:
    """numpy view of an array or a torch tensor (device tensors are copied to
    the host; bfloat16 has no numpy type and is refused)."""
    try:
        import torch
    except ImportError:  # pragma: no cover - torch is a dependency of the package
        torch = None
    if torch is not None and isinstance(tensor, torch.Tensor):
        if tensor.dtype == torch.bfloat16:
            raise TypeError("bfloat16 tensors have no .npy representation; convert to float16 or float32 first")
        return tensor.detach().cpu().contiguous().numpy()
    return np.asarray(tensor)


def save_tensor_npy(tensor: Any, file_path: str | Path) -> TensorDataInfo:
    """Write ``tensor`` as .npy (creating parent folders) and describe the
    file (models/tensor_data_io.py:31-46)."""
    path = Path(file_path)
    path.parent.mkdir(parents=True, exist_ok=True)
    arr = _as_numpy(tensor)
    with path.open("wb") as f:
        np.save(f, arr)
    return TensorDataInfo(file_path=str(path), shape=tuple(int(d) for d in arr.shape), dtype=str(arr.dtype),
                          nbytes=int(arr.nbytes), checksum=compute_file_checksum(path))


def load_tensor_npy(file_path: str | Path) -> np.ndarray:
    """The array of a .npy file (models/tensor_data_io.py:49-52); a missing
    file raises FileNotFoundError."""
    with Path(file_path).open("rb") as f:
        return np.load(f, allow_pickle=False)


def _header(file_path: str | Path) -> np.ndarray:
    return np.load(str(file_path), mmap_mode="r", allow_pickle=False)


def tensor_shape(file_path: str | Path) -> tuple[int, ...]:
    """Shape from the .npy header, without reading the data."""
    return tuple(int(d) for d in _header(file_path).shape)


def tensor_dtype(file_path: str | Path) -> str:
    return str(_header(file_path).dtype)


def tensor_nbytes(file_path: str | Path) -> int:
    return int(_header(file_path).nbytes)


def validate_tensor_file(file_path: str | Path, *, expected_shape: tuple[int, ...] | None = None,
                         expected_dtype: str | None = None, expected_checksum: str | None = None) -> list[str]:
    """Problems found with a payload file, as messages (empty when it is
    fine): existence, readable header, shape, dtype, checksum -- in that order,
    stopping at the first that cannot be read (models/tensor_data_io.py:73-113)."""
    issues: list[str] = []
    path = Path(file_path)
    if not path.exists():
        return [f"file not found: {path}"]
    try:
        shape = tensor_shape(path)
    except Exception as exc:  # noqa: BLE001 - any unreadable header is reported, not raised
        return [f"failed to read shape from {path}: {exc}"]
    if expected_shape is not None and shape != tuple(expected_shape):
        issues.append(f"shape mismatch for {path}: expected {tuple(expected_shape)}, got {shape}")
    try:
        dtype = tensor_dtype(path)
    except Exception as exc:  # noqa: BLE001
        issues.append(f"failed to read dtype from {path}: {exc}")
        return issues
    if expected_dtype is not None and dtype != expected_dtype:
        issues.append(f"dtype mismatch for {path}: expected {expected_dtype}, got {dtype}")
    if expected_checksum is not None:
        try:
            actual = compute_file_checksum(path)
        except Exception as exc:  # noqa: BLE001
            issues.append(f"failed to compute checksum for {path}: {exc}")
            return issues
        if actual != expected_checksum:
            issues.append(f"checksum mismatch for {path}: expected {expected_checksum}, got {actual}")
    return issues


def load_tensor_to_device(file_path: str | Path, device, *, dtype=None, expected_shape=None, expected_dtype=None,
                          expected_checksum=None, chunk_bytes: int = _CHUNK_BYTES):
    """A payload file as a torch tensor on ``device``, checked first with
    validate_tensor_file (ValueError listing the problems).

    For a GPU device the file is memory-mapped and copied in ``chunk_bytes``
    pieces through two pinned host buffers: the piece in flight on the copy
    stream and the next one being filled from the page cache.  ``dtype``, when
    given, converts on the device after the copy (e.g. float32 norm weights
    to the activation type)."""
    import torch

    issues = validate_tensor_file(file_path, expected_shape=expected_shape, expected_dtype=expected_dtype,
                                  expected_checksum=expected_checksum)
    if issues:
        raise ValueError("; ".join(issues))
    mm = _header(file_path)
    dev = torch.device(device)
    if dev.type != "cuda":
        out = torch.from_numpy(np.array(mm))
        return out.to(dtype) if dtype is not None else out
    flat = mm.reshape(-1).view(np.uint8) if mm.size else np.zeros(0, np.uint8)
    nbytes = int(flat.size)
    out = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    if nbytes:
        step = max(1, min(int(chunk_bytes), nbytes))
        staging = [torch.empty(step, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
        done = [None, None]
        stream = torch.cuda.Stream(device=dev)
        # `out` came from the current stream's pool: work still queued there
        # may use its block (e.g. the previous call's dtype conversion read
        # the tensor that block held), so the copies wait for that stream
        stream.wait_stream(torch.cuda.current_stream(dev))
        for i, lo in enumerate(range(0, nbytes, step)):
            hi = min(lo + step, nbytes)
            buf = staging[i % 2]
            if done[i % 2] is not None:
                done[i % 2].synchronize()  # the copy that last read this buffer has finished
            np.copyto(buf.numpy()[: hi - lo], flat[lo:hi])
            with torch.cuda.stream(stream):
                out[lo:hi].copy_(buf[: hi - lo], non_blocking=True)
                ev = torch.cuda.Event()
                ev.record(stream)
            done[i % 2] = ev
        stream.synchronize()
    tdt = torch.from_numpy(np.zeros(0, dtype=mm.dtype)).dtype
    res = out.view(tdt).reshape(tuple(int(d) for d in mm.shape))
    return res.to(dtype) if dtype is not None else res
