"""GQA/MQA decode over paged fp16/bf16 KV -- the decode part of
``ops/gqa_ops.py`` (prefill attention is outside this package).

The reference has no kernel for GQA decode: its
``paged_gqa_decode_block_from_qkv`` (ops/gqa_ops.py:493-547) and
``gqa_decode_block_from_qkv`` (ops/gqa_ops.py:391-444, contiguous cache) run
split + RoPE with array ops, the cache update, and then the pure-array
``reference_*gqa_decode_attention``.  Here each block is two HIP launches:
``mk_qkv_rope_paged_update`` (split + interleaved RoPE + in-place paged write)
and ``mk_paged_decode_attention`` (split-K GQA decode, one K/V read per GQA
group); the contiguous cache [B, MAX_S, Hkv, D] goes through both as an
identity-paged view of the same memory.  ``paged_gqa_decode_attention``
exposes the attention kernel on its own.
"""

from __future__ import annotations

import math

import torch

from . import _contig, _lib
from ._common import ACT_DTYPES
from .kv_cache_ops import normalize_positions, reference_kv_cache_update
from .paged_kv_ops import (
    _gather_pages,
    _hip_paged_attention,
    _i32,
    _masked_attention,
    paged_kv_cache_update,
    reference_paged_kv_cache_update,
)
from .rope_ops import reference_apply_rope


def validate_gqa_heads(num_attention_heads: int, num_key_value_heads: int) -> None:
    """ops/gqa_ops.py:42-54."""
    if num_key_value_heads < 1:
        raise ValueError(f"num_key_value_heads must be >= 1, got {num_key_value_heads}")
    if num_attention_heads < num_key_value_heads:
        raise ValueError(
            "num_attention_heads must be >= num_key_value_heads, "
            f"got {num_attention_heads}, {num_key_value_heads}")
    if num_attention_heads % num_key_value_heads != 0:
        raise ValueError(
            "num_attention_heads must be divisible by num_key_value_heads, "
            f"got {num_attention_heads}, {num_key_value_heads}")


def gqa_group_size(num_attention_heads: int, num_key_value_heads: int) -> int:
    """ops/gqa_ops.py:57-59."""
    validate_gqa_heads(num_attention_heads, num_key_value_heads)
    return num_attention_heads // num_key_value_heads


def q_head_to_kv_head(q_head: int, num_attention_heads: int, num_key_value_heads: int) -> int:
    """ops/gqa_ops.py:62-66."""
    group = gqa_group_size(num_attention_heads, num_key_value_heads)
    if q_head < 0 or q_head >= num_attention_heads:
        raise ValueError(f"q_head must be in [0, {num_attention_heads}), got {q_head}")
    return q_head // group


def reference_gqa_qkv_split(qkv, num_attention_heads, num_key_value_heads, head_dim):
    """ops/gqa_ops.py:118-145: packed [Q | K | V] (or [B,S,Hq+2Hkv,D])."""
    validate_gqa_heads(num_attention_heads, num_key_value_heads)
    q_dim = num_attention_heads * head_dim
    kv_dim = num_key_value_heads * head_dim
    if qkv.ndim == 3:
        expected = q_dim + 2 * kv_dim
        if qkv.shape[-1] != expected:
            raise ValueError(f"packed gqa qkv last dimension must be {expected}, got {qkv.shape[-1]}")
        B, S = qkv.shape[0], qkv.shape[1]
        q = qkv[:, :, :q_dim].reshape(B, S, num_attention_heads, head_dim)
        k = qkv[:, :, q_dim:q_dim + kv_dim].reshape(B, S, num_key_value_heads, head_dim)
        v = qkv[:, :, q_dim + kv_dim:].reshape(B, S, num_key_value_heads, head_dim)
        return q, k, v
    if qkv.ndim == 4:
        if qkv.shape[2] != num_attention_heads + 2 * num_key_value_heads or qkv.shape[3] != head_dim:
            raise ValueError(
                "explicit gqa qkv layout must have shape "
                f"[B,S,{num_attention_heads + 2 * num_key_value_heads},{head_dim}], got {tuple(qkv.shape)}")
        q = qkv[:, :, :num_attention_heads, :]
        k = qkv[:, :, num_attention_heads:num_attention_heads + num_key_value_heads, :]
        v = qkv[:, :, num_attention_heads + num_key_value_heads:, :]
        return q, k, v
    raise ValueError(f"qkv must have shape [B,S,Q+K+V] or [B,S,Hq+Hkv+Hkv,D], got {tuple(qkv.shape)}")


def reference_gqa_qkv_split_rope(qkv, cos, sin, num_attention_heads, num_key_value_heads, head_dim,
                                 position_offset=0):
    """ops/gqa_ops.py:148-160."""
    q, k, v = reference_gqa_qkv_split(qkv, num_attention_heads, num_key_value_heads, head_dim)
    return (reference_apply_rope(q, cos, sin, position_offset=position_offset),
            reference_apply_rope(k, cos, sin, position_offset=position_offset), v)


def _validate_gqa_decode_inputs(q, K_cache, V_cache, lengths):
    """ops/gqa_ops.py:254-275 (lengths clipped to max_s)."""
    if q.ndim != 4 or K_cache.ndim != 4 or V_cache.ndim != 4:
        raise ValueError(
            f"q, K_cache, and V_cache must be 4-D, got {tuple(q.shape)}, {tuple(K_cache.shape)}, {tuple(V_cache.shape)}")
    if q.shape[1] != 1:
        raise ValueError(f"q must have shape [B,1,Hq,D], got {tuple(q.shape)}")
    if K_cache.shape != V_cache.shape:
        raise ValueError(f"K_cache and V_cache must match, got {tuple(K_cache.shape)}, {tuple(V_cache.shape)}")
    B, _, Hq, D = q.shape
    cache_B, max_s, Hkv, cache_D = K_cache.shape
    if B != cache_B or D != cache_D:
        raise ValueError(
            f"q and caches must agree on batch/head_dim, got q={tuple(q.shape)}, K_cache={tuple(K_cache.shape)}, "
            f"V_cache={tuple(V_cache.shape)}")
    validate_gqa_heads(Hq, Hkv)
    lengths_arr = normalize_positions(lengths if lengths is not None else max_s, B, max_s + 1, device=q.device)
    lengths_arr = torch.clamp(lengths_arr, max=max_s)
    return lengths_arr, B, max_s, Hq, Hkv, D


def reference_gqa_decode_attention(q, K_cache, V_cache, lengths=None, scale=None):
    """ops/gqa_ops.py:278-304 over a contiguous cache [B, max_s, Hkv, D]."""
    lengths_arr, B, max_s, Hq, Hkv, D = _validate_gqa_decode_inputs(q, K_cache, V_cache, lengths)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    valid = torch.ones((B, max_s), dtype=torch.bool, device=q.device)
    return _masked_attention(q[:, 0], K_cache, V_cache, lengths_arr, valid, scale).unsqueeze(1).to(q.dtype)


def _validate_paged_gqa(q, K_pages, V_pages, block_table):
    if K_pages.ndim != 4 or V_pages.ndim != 4 or K_pages.shape != V_pages.shape:
        raise ValueError(
            f"K_pages and V_pages must match [NUM_PAGES,PAGE_SIZE,Hkv,D], got {tuple(K_pages.shape)}, {tuple(V_pages.shape)}")
    if block_table.ndim != 2:
        raise ValueError(f"block_table must be [B,MAX_BLOCKS], got {tuple(block_table.shape)}")
    if q.ndim != 4 or q.shape[1] != 1:
        raise ValueError(f"q must have shape [B,1,Hq,D], got {tuple(q.shape)}")
    B = block_table.shape[0]
    if q.shape[0] != B or q.shape[3] != K_pages.shape[3]:
        raise ValueError(f"q and caches must agree on batch/head_dim, got q={tuple(q.shape)}, "
                         f"K_pages={tuple(K_pages.shape)}, block_table={tuple(block_table.shape)}")
    validate_gqa_heads(q.shape[2], K_pages.shape[2])
    return B, block_table.shape[1] * K_pages.shape[1]


def reference_paged_gqa_decode_attention(q, K_pages, V_pages, block_table, lengths=None, scale=None):
    """ops/gqa_ops.py:307-342: gather positions through the block table, then
    per-sequence masked fp32 attention with head h on kv head h // (Hq/Hkv)."""
    B, max_s = _validate_paged_gqa(q, K_pages, V_pages, block_table)
    lengths_arr = normalize_positions(lengths if lengths is not None else max_s, B, max_s + 1,
                                      device=block_table.device)
    lengths_arr = torch.clamp(lengths_arr, max=max_s)
    D = q.shape[3]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    Kc, valid = _gather_pages(K_pages, block_table, max_s)
    Vc, _ = _gather_pages(V_pages, block_table, max_s)
    return _masked_attention(q[:, 0], Kc, Vc, lengths_arr, valid, scale).unsqueeze(1).to(q.dtype)


def paged_gqa_decode_attention(q, K_pages, V_pages, block_table, lengths=None, scale=None, *, backend: str = "auto"):
    """HIP paged GQA decode (no reference kernel exists; semantics of
    reference_paged_gqa_decode_attention, ops/gqa_ops.py:307-342).
    backend: 'auto' / 'metal' / 'metal_gqa' run the kernel, 'reference' the
    tensor-op path."""
    B, max_s = _validate_paged_gqa(q, K_pages, V_pages, block_table)
    backend_name = backend.lower()
    if backend_name == "reference":
        return reference_paged_gqa_decode_attention(q, K_pages, V_pages, block_table, lengths, scale)
    if backend_name not in ("auto", "metal", "metal_gqa", "metal_gqa_threadgroup"):
        raise ValueError("backend must be one of 'reference', 'metal', 'metal_gqa', 'metal_gqa_threadgroup', 'auto'")
    if K_pages.dtype not in ACT_DTYPES:
        raise TypeError(f"K_pages dtype must be float16 or bfloat16, got {K_pages.dtype}")
    lengths_arr = normalize_positions(lengths if lengths is not None else max_s, B, max_s + 1,
                                      device=block_table.device)
    D = q.shape[3]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    out = _hip_paged_attention(q[:, 0], K_pages, V_pages, block_table, lengths_arr, scale)
    return out.unsqueeze(1).to(q.dtype)


def _per_sequence_rope(qkv, cos, sin, Hq, Hkv, D, position):
    """The reference's split + RoPE at per-sequence offsets (ops/gqa_ops.py:513-539)."""
    if isinstance(position, int):
        return reference_gqa_qkv_split_rope(qkv, cos, sin, Hq, Hkv, D, position_offset=position)
    pos_arr = normalize_positions(position, qkv.shape[0], cos.shape[0])
    q_rows, k_rows, v_rows = [], [], []
    for b in range(qkv.shape[0]):
        q_b, k_b, v_b = reference_gqa_qkv_split_rope(qkv[b:b + 1], cos, sin, Hq, Hkv, D,
                                                     position_offset=int(pos_arr[b]))
        q_rows.append(q_b)
        k_rows.append(k_b)
        v_rows.append(v_b)
    return torch.cat(q_rows, 0), torch.cat(k_rows, 0), torch.cat(v_rows, 0)


def reference_paged_gqa_decode_block_from_qkv(qkv, K_pages, V_pages, block_table, cos, sin, position, *,
                                              num_attention_heads, num_key_value_heads, head_dim, scale=None):
    """ops/gqa_ops.py:446-490."""
    q_rope, k_rope, v = _per_sequence_rope(qkv, cos, sin, num_attention_heads, num_key_value_heads, head_dim,
                                           position)
    updated_K, updated_V = reference_paged_kv_cache_update(K_pages, V_pages, k_rope, v, block_table, position)
    max_s = block_table.shape[1] * K_pages.shape[1]
    lengths = position + 1 if isinstance(position, int) else normalize_positions(
        position, qkv.shape[0], max_s, device=block_table.device) + 1
    out = reference_paged_gqa_decode_attention(q_rope, updated_K, updated_V, block_table, lengths=lengths, scale=scale)
    return out, updated_K, updated_V


def _qkv_rope_update_prep(qkv, block_table, cos, sin, position, Hq, Hkv, D, page_size, dtype, dev):
    """Shape checks and device buffers for the fused qkv split + RoPE + paged
    write launches.  Returns (x [B,(Hq+2Hkv)*D], cos, sin, positions int32,
    q_out [B,1,Hq,D], B)."""
    if qkv.ndim == 4:
        B = qkv.shape[0]
        if qkv.shape[1] != 1 or qkv.shape[2] != Hq + 2 * Hkv or qkv.shape[3] != D:
            raise ValueError(f"decode qkv must have shape [B,1,{Hq + 2 * Hkv},{D}], got {tuple(qkv.shape)}")
    elif qkv.ndim == 3:
        B = qkv.shape[0]
        if qkv.shape[1] != 1 or qkv.shape[2] != (Hq + 2 * Hkv) * D:
            raise ValueError(f"decode qkv must have shape [B,1,{(Hq + 2 * Hkv) * D}], got {tuple(qkv.shape)}")
    else:
        raise ValueError(f"qkv must have shape [B,S,Q+K+V] or [B,S,Hq+Hkv+Hkv,D], got {tuple(qkv.shape)}")
    if D % 2 != 0:
        raise ValueError(f"RoPE requires even D, got D={D}")
    if block_table.shape[0] != B:
        raise ValueError(f"block_table batch {block_table.shape[0]} != qkv batch {B}")
    pos = normalize_positions(position, B, cos.shape[0], device=dev)
    pos = normalize_positions(pos, B, block_table.shape[1] * page_size, device=dev)
    x = qkv.reshape(B, -1).to(device=dev, dtype=dtype).contiguous()
    c = cos.to(device=dev, dtype=torch.float32).contiguous()
    s = sin.to(device=dev, dtype=torch.float32).contiguous()
    q_out = torch.empty((B, 1, Hq, D), dtype=dtype, device=dev)
    return x, c, s, pos, q_out, B


def paged_gqa_decode_block_from_qkv(qkv, K_pages, V_pages, block_table, cos, sin, position, *, num_attention_heads,
                                    num_key_value_heads, head_dim, scale=None, backend="auto", lengths=None):
    """ops/gqa_ops.py:493-547 as two HIP launches (fused split + RoPE +
    in-place paged update, then split-K GQA decode attention).  Returns
    (out [B,1,Hq,D], K_pages, V_pages) like the reference.  ``lengths``
    (extension): int32 [B] device tensor equal to position + 1, which a
    caller running many layers at the same positions computes once."""
    backend_name = backend.lower()
    if backend_name not in ("auto", "reference", "metal", "metal_gqa", "metal_gqa_threadgroup"):
        raise ValueError("backend must be one of 'reference', 'metal', 'metal_gqa', 'metal_gqa_threadgroup', 'auto'")
    if backend_name == "reference":
        return reference_paged_gqa_decode_block_from_qkv(
            qkv, K_pages, V_pages, block_table, cos, sin, position, num_attention_heads=num_attention_heads,
            num_key_value_heads=num_key_value_heads, head_dim=head_dim, scale=scale)
    Hq, Hkv, D = num_attention_heads, num_key_value_heads, head_dim
    validate_gqa_heads(Hq, Hkv)
    if K_pages.shape != V_pages.shape or K_pages.ndim != 4 or K_pages.shape[2] != Hkv or K_pages.shape[3] != D:
        raise ValueError(f"K_pages/V_pages must be [NUM_PAGES,PAGE_SIZE,{Hkv},{D}], got {tuple(K_pages.shape)}")
    if K_pages.dtype not in ACT_DTYPES or V_pages.dtype != K_pages.dtype:
        raise TypeError(f"K_pages/V_pages must share a float16/bfloat16 dtype, got {K_pages.dtype}, {V_pages.dtype}")
    if not (K_pages.is_contiguous() and V_pages.is_contiguous()):
        raise ValueError("K_pages and V_pages must be contiguous for the in-place update")
    dev = _lib.require_device(qkv, K_pages, V_pages, block_table)
    NUM_PAGES, P = K_pages.shape[0], K_pages.shape[1]
    MAX_BLOCKS = block_table.shape[1]
    x, c, s, pos, q_out, B = _qkv_rope_update_prep(qkv, block_table, cos, sin, position, Hq, Hkv, D, P,
                                                   K_pages.dtype, dev)
    bt = _i32(block_table, dev)
    _lib.launch("mk_qkv_rope_paged_update", dev, _lib.ptr(x), _lib.ptr(c), _lib.ptr(s), _lib.ptr(pos), _lib.ptr(bt),
                _lib.ptr(K_pages), _lib.ptr(V_pages), _lib.ptr(q_out), B, Hq, Hkv, D, P, MAX_BLOCKS, NUM_PAGES,
                c.shape[0], _lib.dtype_code(K_pages.dtype))
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    out = _hip_paged_attention(q_out[:, 0], K_pages, V_pages, bt, pos + 1 if lengths is None else lengths, scale)
    return out.unsqueeze(1).to(qkv.dtype), K_pages, V_pages


def reference_gqa_decode_block_from_qkv(qkv, K_cache, V_cache, cos, sin, position, *, num_attention_heads,
                                        num_key_value_heads, head_dim, scale=None):
    """ops/gqa_ops.py:345-388: split + RoPE at each sequence's position, the
    functional contiguous update, and fp32 GQA decode attention over
    lengths = position + 1."""
    q_rope, k_rope, v = _per_sequence_rope(qkv, cos, sin, num_attention_heads, num_key_value_heads, head_dim,
                                           position)
    updated_K, updated_V = reference_kv_cache_update(K_cache, V_cache, k_rope, v, position)
    lengths = position + 1 if isinstance(position, int) else normalize_positions(
        position, qkv.shape[0], K_cache.shape[1], device=K_cache.device) + 1
    out = reference_gqa_decode_attention(q_rope, updated_K, updated_V, lengths=lengths, scale=scale)
    return out, updated_K, updated_V


def gqa_decode_block_from_qkv(qkv, K_cache, V_cache, cos, sin, position, *, num_attention_heads,
                              num_key_value_heads, head_dim, scale=None, backend="auto"):
    """ops/gqa_ops.py:391-444 over a contiguous cache [B, MAX_S, Hkv, D]:
    the paged block's two launches on an identity-paged view of the cache
    (no copy).  The new token is written in place and the same tensors are
    returned as (out [B,1,Hq,D], K_cache, V_cache); the reference returns
    updated copies that its callers rebind, which reads the same."""
    backend_name = backend.lower()
    if backend_name not in ("auto", "reference", "metal", "metal_gqa", "metal_gqa_threadgroup"):
        raise ValueError("backend must be one of 'reference', 'metal', 'metal_gqa', 'metal_gqa_threadgroup', 'auto'")
    if backend_name == "reference":
        return reference_gqa_decode_block_from_qkv(
            qkv, K_cache, V_cache, cos, sin, position, num_attention_heads=num_attention_heads,
            num_key_value_heads=num_key_value_heads, head_dim=head_dim, scale=scale)
    Hq, Hkv, D = num_attention_heads, num_key_value_heads, head_dim
    validate_gqa_heads(Hq, Hkv)
    if K_cache.ndim != 4 or V_cache.ndim != 4 or K_cache.shape != V_cache.shape:
        raise ValueError(f"K_cache and V_cache must be matching [B,MAX_S,H,D], got {tuple(K_cache.shape)}, "
                         f"{tuple(V_cache.shape)}")
    B, MAX_S = K_cache.shape[0], K_cache.shape[1]
    if qkv.shape[0] != B or K_cache.shape[2] != Hkv or K_cache.shape[3] != D:
        raise ValueError(
            "k_new and v_new must match cache batch/head/head_dim after normalization. "
            f"Got qkv={tuple(qkv.shape)} for Hkv={Hkv}, D={D}, cache={tuple(K_cache.shape)}.")
    dev = _lib.require_device(qkv, K_cache, V_cache)
    P = _contig.page_size_for(MAX_S)
    Kp, Vp = _contig.as_pages(K_cache, P), _contig.as_pages(V_cache, P)
    bt = _contig.identity_table(B, MAX_S, P, dev)
    out, _, _ = paged_gqa_decode_block_from_qkv(qkv, Kp, Vp, bt, cos, sin, position, num_attention_heads=Hq,
                                                num_key_value_heads=Hkv, head_dim=D, scale=scale, backend="metal")
    return out, K_cache, V_cache
