"""Saved backend choices per (op, shape, dtype, system) (ops/autotune_ops.py:1-185).

Same file format, key construction and lookup rules as the reference: a
JSON file ``{"version": 1, "entries": {key: entry}}`` where ``key`` is the
canonical JSON of ``{op, shape, dtype, system, extra}`` with sorted keys, and
an entry stores ``best_backend``, ``timings``, a UTC timestamp and
``status == "ok"``.  ``select_backend`` prefers a saved entry, then the
caller's default, then the built-in conservative default.

The system descriptor names this host (platform, machine, Python) plus the
HIP runtime torch was built against and the one GPU architecture the kernels
are compiled for, so results recorded on one machine type do not leak onto
another.  Building it touches no GPU.

``tune_backend`` is the measuring half that the reference keeps in its
benchmark driver (benchmarks/autotune.py): it times each candidate with HIP
events on the current stream, rejects candidates whose output disagrees
with the reference backend, and records the fastest.
"""

from __future__ import annotations

import json
import os
import platform
import sys
from datetime import datetime, timezone
from pathlib import Path

DEFAULT_AUTOTUNE_PATH = "~/.cache/mlx-metal-kernels/autotune_results.json"

# ops/autotune_ops.py:14-23, restricted to the ops of this package
_DEFAULT_BACKENDS = {
    "paged_decode_attention": "metal",
    "paged_gqa_decode_attention": "metal",
    "q4_matvec_decode": "metal_parallel",
    "q8_matvec_decode": "metal_parallel",
    "quantized_mlp_block": "tiled",
}

GPU_ARCH = "gfx950"


def _system_info() -> dict:
    try:
        import torch

        hip = getattr(torch.version, "hip", None)
    except Exception:  # noqa: BLE001
        hip = None
    return {
        "platform": platform.platform(),
        "machine": platform.machine(),
        "processor": platform.processor() or None,
        "python_version": sys.version.replace("\n", " "),
        "hip_version": hip,
        "gpu_arch": GPU_ARCH,
    }


def _normalize_shape(shape: dict | None) -> dict:
    return {} if shape is None else {str(k): shape[k] for k in sorted(shape)}


def _normalize_extra(extra: dict | None) -> dict:
    return {} if extra is None else {str(k): extra[k] for k in sorted(extra)}


def _normalize_dtype(dtype) -> str:
    if isinstance(dtype, str):
        return dtype
    name = getattr(dtype, "__name__", None)
    if name:
        return name
    text = str(dtype)
    return text.split(".")[-1] if "." in text else text


def _normalize_path(path=None) -> Path:
    return Path(os.path.expanduser(str(DEFAULT_AUTOTUNE_PATH if path is None else path)))


def load_autotune_results(path=None) -> dict:
    """ops/autotune_ops.py:74-83: a missing file is an empty result set; a
    bare ``{key: entry}`` mapping is wrapped as ``entries``."""
    p = _normalize_path(path)
    if not p.exists():
        return {"version": 1, "entries": {}}
    payload = json.loads(p.read_text(encoding="utf-8"))
    if "entries" not in payload:
        payload = {"version": 1, "entries": payload}
    payload.setdefault("version", 1)
    payload.setdefault("entries", {})
    return payload


def save_autotune_results(results, path=None) -> Path:
    p = _normalize_path(path)
    p.parent.mkdir(parents=True, exist_ok=True)
    p.write_text(json.dumps(results, indent=2, sort_keys=True), encoding="utf-8")
    return p


def make_tuning_key(op_name, shape, dtype, extra=None) -> str:
    payload = {
        "op": op_name,
        "shape": _normalize_shape(shape),
        "dtype": _normalize_dtype(dtype),
        "system": _system_info(),
        "extra": _normalize_extra(extra),
    }
    return json.dumps(payload, sort_keys=True, separators=(",", ":"))


def lookup_best_backend(op_name, shape, dtype, path=None, extra=None):
    entry = load_autotune_results(path).get("entries", {}).get(make_tuning_key(op_name, shape, dtype, extra=extra))
    if not entry or entry.get("status") != "ok":
        raise KeyError(
            f"No saved autotune result for op={op_name!r}, shape={_normalize_shape(shape)}, "
            f"dtype={_normalize_dtype(dtype)}"
        )
    return entry["best_backend"]


def record_best_backend(op_name, shape, dtype, backend, timing, path=None, extra=None):
    """ops/autotune_ops.py:106-124: ``timing`` is either the per-backend
    timing dict (must contain ``backend``) or the winner's own figure."""
    results = load_autotune_results(path)
    key = make_tuning_key(op_name, shape, dtype, extra=extra)
    timings = timing if isinstance(timing, dict) and backend in timing else {backend: timing}
    entry = {
        "op": op_name,
        "shape": _normalize_shape(shape),
        "dtype": _normalize_dtype(dtype),
        "system": _system_info(),
        "best_backend": backend,
        "timings": timings,
        "timestamp_utc": datetime.now(timezone.utc).isoformat(),
        "status": "ok",
        "extra": _normalize_extra(extra),
    }
    results.setdefault("entries", {})[key] = entry
    save_autotune_results(results, path=path)
    return entry


def _default_backend(op_name: str) -> str:
    if op_name not in _DEFAULT_BACKENDS:
        raise KeyError(f"No conservative default backend registered for op={op_name!r}")
    return _DEFAULT_BACKENDS[op_name]


def select_backend(op_name, shape, dtype, *, default_backend=None, path=None, extra=None, require_tuned=False):
    """ops/autotune_ops.py:134-156."""
    try:
        return lookup_best_backend(op_name, shape, dtype, path=path, extra=extra)
    except KeyError:
        if require_tuned:
            raise KeyError(
                f"No saved autotune backend for op={op_name!r}, shape={_normalize_shape(shape)}, "
                f"dtype={_normalize_dtype(dtype)}."
            ) from None
        return default_backend if default_backend is not None else _default_backend(op_name)


def explain_backend_choice(op_name, shape, dtype, *, default_backend=None, path=None, extra=None,
                           require_tuned=False):
    """ops/autotune_ops.py:159-185."""
    try:
        backend = lookup_best_backend(op_name, shape, dtype, path=path, extra=extra)
        return (f"Using autotuned backend {backend!r} for op={op_name!r}, "
                f"shape={_normalize_shape(shape)}, dtype={_normalize_dtype(dtype)}.")
    except KeyError:
        if require_tuned:
            raise
        chosen = default_backend if default_backend is not None else _default_backend(op_name)
        return (f"No saved autotune result for op={op_name!r}, shape={_normalize_shape(shape)}, "
                f"dtype={_normalize_dtype(dtype)}; using conservative default {chosen!r}.")


def tune_backend(op_name, shape, dtype, run, reference, *, backends=None, include_experimental=True,
                 warmup=5, iters=20, rtol=3e-2, atol=3e-2, path=None, extra=None, record=True):
    """Time ``run(backend)`` for each candidate backend of ``op_name`` on the
    current device stream and record the fastest whose output matches
    ``reference()`` (benchmarks/autotune.py: same tolerance, 3e-2).

    ``run`` and ``reference`` are zero-state callables returning a tensor.
    Returns ``(best_backend, timings)`` where ``timings[backend]`` is
    ``{"mean_ms": ...}`` or ``{"status": "mismatch"|"error", ...}``.
    Raises RuntimeError if no candidate passes.
    """
    import torch

    from . import backend_registry as reg

    names = reg.get_candidate_backends(op_name) if backends is None else list(backends)
    names = reg.filter_backends_for_shape(op_name, shape, dtype, names)
    if not include_experimental:
        names = [b for b in names if not reg.is_experimental_backend(b)]
    expect = reference().float()
    timings: dict = {}
    for b in names:
        try:
            out = run(b)
            if not torch.allclose(out.float(), expect, rtol=rtol, atol=atol):
                timings[b] = {"status": "mismatch"}
                continue
            for _ in range(warmup):
                run(b)
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record()
            for _ in range(iters):
                run(b)
            end.record()
            torch.cuda.synchronize()
            timings[b] = {"mean_ms": start.elapsed_time(end) / iters}
        except (RuntimeError, ValueError, TypeError) as exc:
            timings[b] = {"status": "error", "error": f"{type(exc).__name__}: {exc}"}
    ok = {b: t["mean_ms"] for b, t in timings.items() if "mean_ms" in t}
    if not ok:
        raise RuntimeError(f"no backend of {op_name!r} passed for shape={_normalize_shape(shape)}: {timings}")
    best = min(ok, key=ok.get)
    if record:
        record_best_backend(op_name, shape, dtype, best, timings, path=path, extra=extra)
    return best, timings
