"""Backend registry for the hot-path ops (benchmarks/backend_registry.py:1-320).

Same functions, argument meaning and error behaviour as the reference's
registry, restricted to the ops this package implements.  Backend names keep
the reference's spelling ("metal", "metal_parallel", "metal_tiled", ...) so
callers that pass them need no change; every name other than "reference"
selects a gfx950 HIP kernel of ``libmk_hip.so``.

``paged_gqa_decode_attention`` has no entry in the reference (it has no
kernel for that op); it is registered here with the single HIP backend
"metal" so that tuning and selection treat it like the other ops.
"""

from __future__ import annotations

from copy import deepcopy

BACKEND_REGISTRY = {
    "decode_attention": {
        "function": "mk.decode_ops.decode_attention",
        "reference_backend": "reference",
        "candidate_backends": ["metal", "metal_threadgroup", "metal_d64", "metal_d128"],
    },
    "quantized_kv_decode_attention": {
        "function": "mk.quantized_kv_cache_ops.quantized_kv_gqa_decode_attention",
        "reference_backend": "reference",
        "candidate_backends": ["metal_q8", "metal_q4"],
    },
    "llama_layer_decode": {
        "function": "mk.llama_layer_ops.llama_layer_decode_loop",
        "reference_backend": "reference",
        "candidate_backends": ["metal", "tiled", "fused_experimental"],
    },
    "llama_stack_decode": {
        "function": "mk.llama_stack_ops.llama_stack_decode_loop",
        "reference_backend": "reference",
        "candidate_backends": ["metal", "tiled", "fused_experimental"],
    },
    "paged_decode_attention": {
        "function": "mk.paged_kv_ops.paged_decode_attention",
        "reference_backend": "reference",
        "candidate_backends": ["metal", "metal_threadgroup", "metal_d64", "metal_d128"],
    },
    "paged_gqa_decode_attention": {
        "function": "mk.gqa_ops.paged_gqa_decode_attention",
        "reference_backend": "reference",
        "candidate_backends": ["metal"],
    },
    "q4_matvec_decode": {
        "function": "mk.quant_ops.q4_matvec_decode",
        "reference_backend": "reference",
        "candidate_backends": ["metal", "metal_parallel", "metal_tiled"],
    },
    "q8_matvec_decode": {
        "function": "mk.quant_ops.q8_matvec_decode",
        "reference_backend": "reference",
        "candidate_backends": ["metal", "metal_parallel", "metal_tiled"],
    },
    "quantized_mlp_block": {
        "function": "mk.mlp_block_ops.quantized_mlp_block",
        "reference_backend": "reference",
        "candidate_backends": ["tiled", "fused_experimental"],
    },
    "paged_quantized_kv_decode_attention": {
        "function": "mk.paged_quantized_kv_ops.paged_quantized_kv_gqa_decode_attention",
        "reference_backend": "reference",
        "candidate_backends": ["metal_q8", "metal_q4"],
    },
}

# benchmarks/backend_registry.py:163-176, restricted to the names used above
_EXPERIMENTAL_BACKENDS = {
    "metal_threadgroup",
    "metal_tiled",
    "fused_experimental",
    "metal_q8",
    "metal_q4",
}


def list_ops() -> list[str]:
    return sorted(BACKEND_REGISTRY)


def _entry(op_name: str) -> dict:
    if op_name not in BACKEND_REGISTRY:
        raise KeyError(f"Unknown op: {op_name}")
    return BACKEND_REGISTRY[op_name]


def get_candidate_backends(op_name: str) -> list[str]:
    return list(_entry(op_name)["candidate_backends"])


def get_reference_backend(op_name: str) -> str:
    return str(_entry(op_name)["reference_backend"])


def get_registry_entry(op_name: str) -> dict:
    return deepcopy(_entry(op_name))


def validate_backend(op_name: str, backend: str) -> str:
    """benchmarks/backend_registry.py:201-209."""
    allowed = set(get_candidate_backends(op_name)) | {get_reference_backend(op_name)}
    if backend not in allowed:
        raise ValueError(
            f"Unsupported backend={backend!r} for op={op_name!r}. Expected one of {sorted(allowed)}."
        )
    return backend


def is_experimental_backend(backend: str) -> bool:
    return backend in _EXPERIMENTAL_BACKENDS


def _dtype_name(dtype) -> str:
    if isinstance(dtype, str):
        return dtype
    name = getattr(dtype, "__name__", None)
    if name:
        return name
    text = str(dtype)
    return text.split(".")[-1] if "." in text else text


def _gqa_heads_ok(shape: dict) -> bool:
    hq, hkv = shape.get("Hq"), shape.get("Hkv")
    return hq is not None and hkv is not None and hq >= hkv and hq % hkv == 0


def _keep(op_name: str, backend: str, shape: dict, dtype_name: str) -> bool:
    """One backend's shape/dtype rule (benchmarks/backend_registry.py:225-320)."""
    dim = shape.get("D")
    if "d64" in backend and dim != 64:
        return False
    if "d128" in backend and dim != 128:
        return False
    if op_name == "quantized_mlp_block" and backend == "fused_experimental":
        return shape.get("bits") in (4, 8) and dtype_name == "float16"
    if op_name in ("llama_layer_decode", "llama_stack_decode"):
        # the reference also drops every backend of a paged stack (it has
        # none); the paged stack runs here, so that rule is not kept
        if shape.get("bits") not in (4, 8):
            return False
        return backend != "fused_experimental" or dtype_name == "float16"
    if op_name == "paged_gqa_decode_attention" and backend != "reference":
        return _gqa_heads_ok(shape)
    if op_name in ("paged_quantized_kv_decode_attention", "quantized_kv_decode_attention") and backend != "reference":
        bits = shape.get("bits")
        if not _gqa_heads_ok(shape):
            return False
        if backend == "metal_q8" and bits not in (None, 8):
            return False
        if backend == "metal_q4" and bits not in (None, 4):
            return False
        return dim is None or dim <= 128
    return True


def filter_backends_for_shape(op_name: str, shape: dict, dtype, backends) -> list[str]:
    """Backends of ``backends`` that support ``shape``/``dtype``; raises
    ValueError for a name the op does not know (as the reference does)."""
    _entry(op_name)
    dtype_name = _dtype_name(dtype).lower()
    out = []
    for backend in backends:
        validate_backend(op_name, backend)
        if _keep(op_name, backend, shape, dtype_name):
            out.append(backend)
    return out
