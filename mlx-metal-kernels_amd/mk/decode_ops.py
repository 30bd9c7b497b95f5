"""Decode attention over a contiguous fp16/bf16 KV cache -- drop-in for
``ops/decode_ops.py`` over ``torch.Tensor``.

q [B,1,H,D] attends to K/V_cache [B,MAX_S,H,D] at positions j < lengths[b]
(MHA, D <= 128).  The HIP backends ("metal", "metal_threadgroup",
"metal_d64", "metal_d128", "auto") run the paged decode attention kernel over
an identity-paged view of the cache (no copy): a contiguous cache is the
paged layout with block table bt[b, j] = b * MAX_S / P + j.
``decode_step`` writes the new token first (in place, as
``kv_cache_ops.kv_cache_update``) and attends over lengths = position + 1.
"""

from __future__ import annotations

import math

import torch

from . import _contig, _lib
from .kv_cache_ops import kv_cache_update, normalize_positions, reference_kv_cache_update
from .paged_kv_ops import _masked_attention, _resolve_backend

_BACKENDS_MSG = "backend must be one of 'reference', 'metal', 'metal_threadgroup', 'metal_d64', 'metal_d128', 'auto'"


def _validate_inputs(q, K_cache, V_cache, lengths):
    """ops/decode_ops.py:60-90."""
    if q.ndim != 4 or K_cache.ndim != 4 or V_cache.ndim != 4:
        raise ValueError(f"q, K_cache, and V_cache must be 4-D, got {tuple(q.shape)}, {tuple(K_cache.shape)}, "
                         f"{tuple(V_cache.shape)}")
    if q.shape[1] != 1:
        raise ValueError(f"decode_attention expects q.shape[1] == 1, got {tuple(q.shape)}")
    if K_cache.shape != V_cache.shape:
        raise ValueError(f"K_cache and V_cache must match, got {tuple(K_cache.shape)}, {tuple(V_cache.shape)}")
    if q.shape[0] != K_cache.shape[0] or q.shape[2] != K_cache.shape[2] or q.shape[3] != K_cache.shape[3]:
        raise ValueError(
            "q and cache tensors must agree on batch, heads, and head_dim. "
            f"Got q={tuple(q.shape)}, K_cache={tuple(K_cache.shape)}, V_cache={tuple(V_cache.shape)}. "
            "For GQA/MQA decode with Hq != Hkv, use mk.gqa_ops.reference_gqa_decode_attention.")
    B, _, H, D = q.shape
    MAX_S = K_cache.shape[1]
    if D > 128:
        raise ValueError(f"decode_attention currently supports D <= 128, got {D}")
    act = (torch.float16, torch.bfloat16)
    if q.dtype not in act:
        raise TypeError(f"q dtype must be float16 or bfloat16, got {q.dtype}")
    if K_cache.dtype not in act or V_cache.dtype not in act:
        raise TypeError(f"K_cache/V_cache dtype must be float16 or bfloat16, got {K_cache.dtype}, {V_cache.dtype}")
    lengths_arr = normalize_positions(lengths if lengths is not None else MAX_S, B, MAX_S + 1, device=q.device)
    lengths_arr = torch.clamp(lengths_arr, max=MAX_S)
    return lengths_arr, B, MAX_S, H, D


def reference_decode_attention(q, K_cache, V_cache, lengths=None, scale=None, *, causal: bool = False):
    """ops/decode_ops.py:93-123: fp32 masked softmax attention (``causal`` is
    accepted and ignored: the lengths already define the prefix)."""
    lengths_arr, B, MAX_S, H, D = _validate_inputs(q, K_cache, V_cache, lengths)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    valid = torch.ones((B, MAX_S), dtype=torch.bool, device=q.device)
    return _masked_attention(q[:, 0], K_cache, V_cache, lengths_arr, valid, scale).unsqueeze(1).to(q.dtype)


def hip_contiguous_attention(q3, K_cache, V_cache, lengths_arr, scale: float):
    """q3 [B,Hq,D] over a contiguous [B,MAX_S,Hkv,D] cache on the paged HIP
    kernel (identity-paged view) -> [B,Hq,D] in the cache dtype."""
    B, MAX_S, Hkv, D = K_cache.shape
    dev = _lib.require_device(q3, K_cache, V_cache)
    if K_cache.dtype != V_cache.dtype:
        raise TypeError(f"K_cache and V_cache must share a dtype, got {K_cache.dtype}, {V_cache.dtype}")
    P = _contig.page_size_for(MAX_S)
    Kp, Vp = _contig.as_pages(K_cache, P), _contig.as_pages(V_cache, P)
    bt = _contig.identity_table(B, MAX_S, P, dev)
    dtype = K_cache.dtype
    q3 = q3.to(dtype).contiguous()
    ln = lengths_arr.to(device=dev, dtype=torch.int32).contiguous()
    out = torch.empty((B, q3.shape[1], D), dtype=dtype, device=dev)
    ws, ws_bytes = _lib.attention_workspace(dev, B, q3.shape[1], Hkv, D, MAX_S // P, P)
    _lib.launch("mk_paged_decode_attention", dev, _lib.ptr(q3), _lib.ptr(Kp), _lib.ptr(Vp), _lib.ptr(bt),
                _lib.ptr(ln), _lib.ptr(out), B, q3.shape[1], Hkv, D, P, MAX_S // P, Kp.shape[0], float(scale),
                _lib.dtype_code(dtype), _lib.ptr(ws), ws_bytes)
    return out


def decode_attention(q, K_cache, V_cache, lengths=None, scale=None, *, causal: bool = False, backend: str = "auto"):
    """ops/decode_ops.py:126-176."""
    lengths_arr, B, MAX_S, H, D = _validate_inputs(q, K_cache, V_cache, lengths)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    backend_name = _resolve_backend(backend.lower(), D)
    if backend_name == "reference":
        return reference_decode_attention(q, K_cache, V_cache, lengths=lengths_arr, scale=scale, causal=causal)
    if backend_name not in ("metal", "metal_threadgroup", "metal_d64", "metal_d128"):
        raise ValueError(_BACKENDS_MSG)
    out = hip_contiguous_attention(q[:, 0], K_cache, V_cache, lengths_arr, scale)
    return out.unsqueeze(1).to(q.dtype)


def _step_lengths(position, K_cache):
    if isinstance(position, int):
        return position + 1
    return normalize_positions(position, K_cache.shape[0], K_cache.shape[1], device=K_cache.device) + 1


def reference_decode_step(q, k_new, v_new, K_cache, V_cache, position, scale=None):
    """ops/decode_ops.py:179-195."""
    K_updated, V_updated = reference_kv_cache_update(K_cache, V_cache, k_new, v_new, position)
    out = reference_decode_attention(q, K_updated, V_updated, lengths=_step_lengths(position, K_cache), scale=scale)
    return out, K_updated, V_updated


def decode_step(q, k_new, v_new, K_cache, V_cache, position, scale=None, *, backend: str = "auto"):
    """ops/decode_ops.py:198-220: update (in place on the HIP backends), then
    decode attention over lengths = position + 1."""
    backend_name = backend.lower()
    if backend_name == "reference":
        return reference_decode_step(q, k_new, v_new, K_cache, V_cache, position, scale=scale)
    upd_backend = "metal" if backend_name in ("metal_threadgroup", "metal_d64", "metal_d128") else backend_name
    K_updated, V_updated = kv_cache_update(K_cache, V_cache, k_new, v_new, position, backend=upd_backend)
    out = decode_attention(q, K_updated, V_updated, lengths=_step_lengths(position, K_cache), scale=scale,
                           causal=False, backend=backend_name)
    return out, K_updated, V_updated
