"""Paged fp16/bf16 KV cache: block tables, lookup, update, decode attention --
drop-in for ``ops/paged_kv_ops.py`` over ``torch.Tensor``.

Backends: ``"reference"`` runs tensor ops; ``"metal"``, ``"metal_threadgroup"``,
``"metal_d64"``, ``"metal_d128"`` and ``"auto"`` run the gfx950 HIP kernels
(with the reference's name-specific validation kept: ``metal_d64`` needs
D == 64, ``metal_d128`` D == 128).

Ownership: the reference's MLX arrays are immutable and every update returns
new page arrays that callers rebind.  Here ``paged_kv_cache_update`` writes the
B*H*D new elements in place (O(token) instead of O(cache)) and returns the same
tensor objects, which is observationally identical for rebinding callers;
``copy=True`` restores the functional behaviour.
"""

from __future__ import annotations

import math
import os

import torch

from . import _lib
from ._common import ACT_DTYPES, ci_safe_mode_enabled
from .kv_cache_ops import _normalize_token_shape, normalize_positions

_ATTN_BACKENDS_MSG = "backend must be one of 'reference', 'metal', 'metal_threadgroup', 'metal_d64', 'metal_d128', 'auto'"


def _resolve_backend(backend_name: str, D: int) -> str:
    """ops/paged_kv_ops.py:80-96."""
    if backend_name == "auto":
        if ci_safe_mode_enabled():
            return "reference"
        if os.environ.get("MLX_METAL_USE_THREADGROUP_ATTENTION", "0") == "1":
            return "metal_threadgroup"
        if os.environ.get("MLX_METAL_USE_SPECIALIZED", "0") == "1":
            if D == 64:
                return "metal_d64"
            if D == 128:
                return "metal_d128"
        return "metal"
    if backend_name == "metal_d64" and D != 64:
        raise ValueError(f"backend='metal_d64' requires D == 64, got D={D}")
    if backend_name == "metal_d128" and D != 128:
        raise ValueError(f"backend='metal_d128' requires D == 128, got D={D}")
    return backend_name


def make_identity_block_table(B: int, MAX_S: int, PAGE_SIZE: int, *, device=None) -> torch.Tensor:
    """ops/paged_kv_ops.py:99-105: bt[b, j] = b * ceil(MAX_S/P) + j."""
    if B <= 0 or MAX_S <= 0 or PAGE_SIZE <= 0:
        raise ValueError(f"B, MAX_S, and PAGE_SIZE must be positive, got {B}, {MAX_S}, {PAGE_SIZE}")
    max_blocks = math.ceil(MAX_S / PAGE_SIZE)
    base = torch.arange(B, dtype=torch.int32, device=device).reshape(B, 1) * max_blocks
    return base + torch.arange(max_blocks, dtype=torch.int32, device=device).reshape(1, max_blocks)


def allocate_paged_kv_cache(B: int, MAX_S: int, H: int, D: int, PAGE_SIZE: int, dtype, *, device=None):
    """ops/paged_kv_ops.py:108-115."""
    if dtype not in ACT_DTYPES:
        raise TypeError(f"dtype must be float16 or bfloat16, got {dtype}")
    block_table = make_identity_block_table(B, MAX_S, PAGE_SIZE, device=device)
    num_pages = B * math.ceil(MAX_S / PAGE_SIZE)
    K_pages = torch.zeros((num_pages, PAGE_SIZE, H, D), dtype=dtype, device=device)
    V_pages = torch.zeros((num_pages, PAGE_SIZE, H, D), dtype=dtype, device=device)
    return K_pages, V_pages, block_table


def _validate_page_tensors(K_pages, V_pages, block_table):
    """ops/paged_kv_ops.py:118-131."""
    if K_pages.ndim != 4 or V_pages.ndim != 4:
        raise ValueError(
            f"K_pages and V_pages must be 4-D [NUM_PAGES,PAGE_SIZE,H,D], got {tuple(K_pages.shape)}, {tuple(V_pages.shape)}")
    if K_pages.shape != V_pages.shape:
        raise ValueError(f"K_pages and V_pages must match, got {tuple(K_pages.shape)}, {tuple(V_pages.shape)}")
    if block_table.ndim != 2:
        raise ValueError(f"block_table must be 2-D [B,MAX_BLOCKS], got {tuple(block_table.shape)}")
    NUM_PAGES, PAGE_SIZE, H, D = K_pages.shape
    B, MAX_BLOCKS = block_table.shape
    if K_pages.dtype not in ACT_DTYPES:
        raise TypeError(f"K_pages dtype must be float16 or bfloat16, got {K_pages.dtype}")
    if V_pages.dtype not in ACT_DTYPES:
        raise TypeError(f"V_pages dtype must be float16 or bfloat16, got {V_pages.dtype}")
    return NUM_PAGES, PAGE_SIZE, H, D, B, MAX_BLOCKS


def _i32(t: torch.Tensor, device) -> torch.Tensor:
    return t.to(device=device, dtype=torch.int32).contiguous()


# ----------------------------------------------------------------- lookup


def reference_block_table_lookup(block_table, positions, PAGE_SIZE: int):
    """ops/paged_kv_ops.py:138-152."""
    if PAGE_SIZE <= 0:
        raise ValueError("PAGE_SIZE must be positive")
    if block_table.ndim != 2:
        raise ValueError(f"block_table must be 2-D [B,MAX_BLOCKS], got {tuple(block_table.shape)}")
    B, MAX_BLOCKS = block_table.shape
    pos = normalize_positions(positions, B, MAX_BLOCKS * PAGE_SIZE, device=block_table.device).long()
    block_ids = pos // PAGE_SIZE
    offsets = pos % PAGE_SIZE
    page_ids = block_table[torch.arange(B, device=block_table.device), block_ids]
    return page_ids.to(torch.int32), offsets.to(torch.int32)


def block_table_lookup(block_table, positions, PAGE_SIZE: int, *, backend: str = "auto"):
    """ops/paged_kv_ops.py:155-182."""
    if PAGE_SIZE <= 0:
        raise ValueError("PAGE_SIZE must be positive")
    if block_table.ndim != 2:
        raise ValueError(f"block_table must be 2-D [B,MAX_BLOCKS], got {tuple(block_table.shape)}")
    B, MAX_BLOCKS = block_table.shape
    pos = normalize_positions(positions, B, MAX_BLOCKS * PAGE_SIZE, device=block_table.device)
    backend_name = backend.lower()
    if backend_name == "auto":
        backend_name = "metal"
    if ci_safe_mode_enabled() or backend_name == "reference":
        return reference_block_table_lookup(block_table, pos, PAGE_SIZE)
    if backend_name != "metal":
        raise ValueError("backend must be one of 'reference', 'metal', 'auto'")
    dev = _lib.require_device(block_table)
    bt = _i32(block_table, dev)
    pos = _i32(pos, dev)
    page_ids = torch.empty((B,), dtype=torch.int32, device=dev)
    offsets = torch.empty((B,), dtype=torch.int32, device=dev)
    _lib.launch("mk_block_table_lookup", dev, _lib.ptr(bt), _lib.ptr(pos), _lib.ptr(page_ids), _lib.ptr(offsets),
                B, MAX_BLOCKS, PAGE_SIZE)
    return page_ids, offsets


# ----------------------------------------------------------------- update


def reference_paged_kv_cache_update(K_pages, V_pages, k_new, v_new, block_table, positions):
    """ops/paged_kv_ops.py:185-213 (functional; a later b wins a collision)."""
    k_new = _normalize_token_shape(k_new, "k_new")
    v_new = _normalize_token_shape(v_new, "v_new")
    NUM_PAGES, PAGE_SIZE, H, D, B, MAX_BLOCKS = _validate_page_tensors(K_pages, V_pages, block_table)
    if tuple(k_new.shape) != (B, 1, H, D) or tuple(v_new.shape) != (B, 1, H, D):
        raise ValueError(
            f"k_new/v_new must normalize to [B,1,H,D]={(B, 1, H, D)}, got {tuple(k_new.shape)}, {tuple(v_new.shape)}")
    pos = normalize_positions(positions, B, MAX_BLOCKS * PAGE_SIZE, device=block_table.device)
    page_ids, offsets = reference_block_table_lookup(block_table, pos, PAGE_SIZE)
    K_updated = K_pages.clone()
    V_updated = V_pages.clone()
    for b in range(B):
        p, o = int(page_ids[b]), int(offsets[b])
        K_updated[p, o] = k_new[b, 0].to(K_pages.dtype)
        V_updated[p, o] = v_new[b, 0].to(V_pages.dtype)
    return K_updated, V_updated


def paged_kv_cache_update(K_pages, V_pages, k_new, v_new, block_table, positions, *, backend: str = "auto",
                          copy: bool = False):
    """ops/paged_kv_ops.py:216-255, in place on the HIP backend (see module
    docstring); ``copy=True`` updates fresh copies instead."""
    k_new = _normalize_token_shape(k_new, "k_new")
    v_new = _normalize_token_shape(v_new, "v_new")
    NUM_PAGES, PAGE_SIZE, H, D, B, MAX_BLOCKS = _validate_page_tensors(K_pages, V_pages, block_table)
    if tuple(k_new.shape) != (B, 1, H, D) or tuple(v_new.shape) != (B, 1, H, D):
        raise ValueError(
            f"k_new/v_new must normalize to [B,1,H,D]={(B, 1, H, D)}, got {tuple(k_new.shape)}, {tuple(v_new.shape)}")
    pos = normalize_positions(positions, B, MAX_BLOCKS * PAGE_SIZE, device=block_table.device)
    backend_name = backend.lower()
    if backend_name == "auto":
        backend_name = "metal"
    if ci_safe_mode_enabled() or backend_name == "reference":
        return reference_paged_kv_cache_update(K_pages, V_pages, k_new, v_new, block_table, pos)
    if backend_name != "metal":
        raise ValueError("backend must be one of 'reference', 'metal', 'auto'")
    if K_pages.dtype != V_pages.dtype:
        raise TypeError(f"K_pages and V_pages must share a dtype, got {K_pages.dtype}, {V_pages.dtype}")
    dev = _lib.require_device(K_pages, V_pages, block_table)
    if copy:
        K_pages, V_pages = K_pages.clone(), V_pages.clone()
    if not (K_pages.is_contiguous() and V_pages.is_contiguous()):
        raise ValueError("K_pages and V_pages must be contiguous for the in-place update")
    k = k_new.to(device=dev, dtype=K_pages.dtype).contiguous()
    v = v_new.to(device=dev, dtype=K_pages.dtype).contiguous()
    _lib.launch("mk_paged_kv_update", dev, _lib.ptr(K_pages), _lib.ptr(V_pages), _lib.ptr(k), _lib.ptr(v),
                _lib.ptr(_i32(block_table, dev)), _lib.ptr(_i32(pos, dev)), B, H, D, PAGE_SIZE, MAX_BLOCKS,
                NUM_PAGES, _lib.dtype_code(K_pages.dtype))
    return K_pages, V_pages


# ----------------------------------------------------------------- attention


def _gather_pages(pages, block_table, max_s: int):
    """[NP,P,H,D] pages -> [B, max_s, H, D] through the block table; entries
    outside [0, NP) gather page 0 (callers mask them)."""
    P = pages.shape[1]
    j = torch.arange(max_s, device=block_table.device)
    page = block_table.long()[:, j // P]
    valid = (page >= 0) & (page < pages.shape[0])
    page = torch.where(valid, page, torch.zeros_like(page))
    return pages[page, (j % P).unsqueeze(0).expand_as(page)], valid


def _masked_attention(q, K, V, lengths, valid, scale: float):
    """fp32 softmax attention of q [B,Hq,D] over K/V [B,S,Hkv,D] at positions
    j < lengths[b] with valid pages; GQA maps head h to kv head h // (Hq/Hkv).
    A row with no position gives zeros."""
    B, Hq, D = q.shape
    Hkv = K.shape[2]
    group = Hq // Hkv
    S = K.shape[1]
    kf = K.to(torch.float32).repeat_interleave(group, dim=2).permute(0, 2, 1, 3)  # [B,Hq,S,D]
    vf = V.to(torch.float32).repeat_interleave(group, dim=2).permute(0, 2, 1, 3)
    scores = torch.matmul(q.to(torch.float32).unsqueeze(2), kf.transpose(-1, -2)).squeeze(2) * float(scale)
    pos = torch.arange(S, device=q.device).reshape(1, S)
    mask = (pos < lengths.to(q.device).long().reshape(B, 1)) & valid
    scores = scores.masked_fill(~mask.unsqueeze(1), float("-inf"))
    probs = torch.softmax(scores, dim=-1)
    probs = torch.nan_to_num(probs, nan=0.0)
    return torch.matmul(probs.unsqueeze(2), vf).squeeze(2)


def reference_paged_decode_attention(q, K_pages, V_pages, block_table, lengths, *, scale=None):
    """ops/paged_kv_ops.py:258-304 (MHA: q [B,1,H,D] with H = page heads)."""
    NUM_PAGES, PAGE_SIZE, H, D, B, MAX_BLOCKS = _validate_page_tensors(K_pages, V_pages, block_table)
    if q.ndim != 4 or tuple(q.shape) != (B, 1, H, D):
        raise ValueError(
            f"q must have shape [B,1,H,D]={(B, 1, H, D)}, got {tuple(q.shape)}. "
            "For GQA/MQA paged decode with Hq != Hkv, use mk.gqa_ops.reference_paged_gqa_decode_attention.")
    max_s = MAX_BLOCKS * PAGE_SIZE
    lengths_arr = normalize_positions(lengths if lengths is not None else max_s, B, max_s + 1,
                                      device=block_table.device)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    Kc, valid = _gather_pages(K_pages, block_table, max_s)
    Vc, _ = _gather_pages(V_pages, block_table, max_s)
    out = _masked_attention(q[:, 0], Kc, Vc, lengths_arr, valid, scale)
    return out.unsqueeze(1).to(q.dtype)


def _hip_paged_attention(q3, K_pages, V_pages, block_table, lengths, scale: float):
    """q3 [B,Hq,D] -> [B,Hq,D] on the HIP kernel."""
    NUM_PAGES, PAGE_SIZE, Hkv, D = K_pages.shape
    B, MAX_BLOCKS = block_table.shape
    Hq = q3.shape[1]
    dev = _lib.require_device(q3, K_pages, V_pages, block_table)
    dtype = K_pages.dtype
    if V_pages.dtype != dtype:
        raise TypeError(f"K_pages and V_pages must share a dtype, got {dtype}, {V_pages.dtype}")
    q3 = q3.to(dtype).contiguous()
    Kp, Vp = K_pages.contiguous(), V_pages.contiguous()
    bt = _i32(block_table, dev)
    ln = _i32(lengths, dev)
    out = torch.empty((B, Hq, D), dtype=dtype, device=dev)
    ws, ws_bytes = _lib.attention_workspace(dev, B, Hq, Hkv, D, MAX_BLOCKS, PAGE_SIZE)
    _lib.launch("mk_paged_decode_attention", dev, _lib.ptr(q3), _lib.ptr(Kp), _lib.ptr(Vp), _lib.ptr(bt),
                _lib.ptr(ln), _lib.ptr(out), B, Hq, Hkv, D, PAGE_SIZE, MAX_BLOCKS, NUM_PAGES, float(scale),
                _lib.dtype_code(dtype), _lib.ptr(ws), ws_bytes)
    return out


def paged_decode_attention(q, K_pages, V_pages, block_table, lengths, *, scale=None, backend: str = "auto"):
    """ops/paged_kv_ops.py:307-360."""
    NUM_PAGES, PAGE_SIZE, H, D, B, MAX_BLOCKS = _validate_page_tensors(K_pages, V_pages, block_table)
    if q.ndim != 4 or tuple(q.shape) != (B, 1, H, D):
        raise ValueError(
            f"q must have shape [B,1,H,D]={(B, 1, H, D)}, got {tuple(q.shape)}. "
            "For GQA/MQA paged decode with Hq != Hkv, use mk.gqa_ops.reference_paged_gqa_decode_attention.")
    if D > 128:
        raise ValueError(f"paged_decode_attention currently supports D <= 128, got {D}")
    max_s = MAX_BLOCKS * PAGE_SIZE
    lengths_arr = normalize_positions(lengths if lengths is not None else max_s, B, max_s + 1,
                                      device=block_table.device)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    backend_name = _resolve_backend(backend.lower(), D)
    if backend_name == "reference":
        return reference_paged_decode_attention(q, K_pages, V_pages, block_table, lengths_arr, scale=scale)
    if backend_name not in ("metal", "metal_threadgroup", "metal_d64", "metal_d128"):
        raise ValueError(_ATTN_BACKENDS_MSG)
    out = _hip_paged_attention(q[:, 0], K_pages, V_pages, block_table, lengths_arr, scale)
    return out.unsqueeze(1).to(q.dtype)


def reference_paged_decode_step(q, k_new, v_new, K_pages, V_pages, block_table, position, *, scale=None):
    """ops/paged_kv_ops.py:363-380."""
    updated_K, updated_V = reference_paged_kv_cache_update(K_pages, V_pages, k_new, v_new, block_table, position)
    if isinstance(position, int):
        lengths = position + 1
    else:
        lengths = normalize_positions(position, block_table.shape[0], block_table.shape[1] * K_pages.shape[1],
                                      device=block_table.device) + 1
    out = reference_paged_decode_attention(q, updated_K, updated_V, block_table, lengths, scale=scale)
    return out, updated_K, updated_V


def paged_decode_step(q, k_new, v_new, K_pages, V_pages, block_table, position, *, scale=None, backend: str = "auto"):
    """ops/paged_kv_ops.py:383-404."""
    backend_name = backend.lower()
    if backend_name == "reference":
        return reference_paged_decode_step(q, k_new, v_new, K_pages, V_pages, block_table, position, scale=scale)
    upd_backend = "metal" if backend_name in ("metal_threadgroup", "metal_d64", "metal_d128") else backend_name
    updated_K, updated_V = paged_kv_cache_update(K_pages, V_pages, k_new, v_new, block_table, position,
                                                 backend=upd_backend)
    if isinstance(position, int):
        lengths = position + 1
    else:
        lengths = normalize_positions(position, block_table.shape[0], block_table.shape[1] * K_pages.shape[1],
                                      device=block_table.device) + 1
    out = paged_decode_attention(q, updated_K, updated_V, block_table, lengths, scale=scale, backend=backend_name)
    return out, updated_K, updated_V
