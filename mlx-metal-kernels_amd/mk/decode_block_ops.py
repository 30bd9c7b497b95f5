"""The paged decode block from a packed qkv row -- ``paged_decode_block_from_qkv``
of ``ops/decode_block_ops.py`` (:174-257) over ``torch.Tensor``.

One decode token per sequence: split qkv into q/k/v, rotate q and k at the
sequence's position (interleaved RoPE), write k/v into the paged cache at
(block_table[b, pos // P], pos % P), and attend over lengths = position + 1.
With ``H`` given and different from the cache's head count the call is GQA
and goes to ``gqa_ops.paged_gqa_decode_block_from_qkv``, as in the
reference.  The MHA block is the same two HIP launches with Hq = Hkv = H:
``mk_qkv_rope_paged_update`` (split + RoPE + in-place paged write) and
``mk_paged_decode_attention``.  The MHA qkv layouts are [B,1,3*H*D] (needs H
and D) and [B,1,3,H,D]; both hold q, k, v head-major in that order, which is
the GQA packed row with Hq = Hkv.
"""

from __future__ import annotations

import torch

from .gqa_ops import (
    _per_sequence_rope,
    paged_gqa_decode_block_from_qkv,
    reference_paged_gqa_decode_block_from_qkv,
)
from .kv_cache_ops import normalize_positions
from .paged_kv_ops import _ATTN_BACKENDS_MSG, reference_paged_decode_attention, reference_paged_kv_cache_update


def _validate_paged_cache(K_pages, V_pages, block_table):
    """ops/decode_block_ops.py:36-45."""
    if K_pages.ndim != 4 or V_pages.ndim != 4 or K_pages.shape != V_pages.shape:
        raise ValueError(f"K_pages and V_pages must be matching [NUM_PAGES,PAGE_SIZE,H,D], got "
                         f"{tuple(K_pages.shape)}, {tuple(V_pages.shape)}")
    if block_table.ndim != 2:
        raise ValueError(f"block_table must be [B,MAX_BLOCKS], got {tuple(block_table.shape)}")
    num_pages, page_size, heads, head_dim = K_pages.shape
    batch, max_blocks = block_table.shape
    return num_pages, page_size, heads, head_dim, batch, max_blocks


def _decode_lengths(position, B: int, max_positions: int, device=None):
    """ops/decode_block_ops.py:52-55."""
    if isinstance(position, int):
        return position + 1
    return normalize_positions(position, B, max_positions, device=device) + 1


def _mha_qkv_dims(qkv, H, D):
    """ops/layout_ops.py:42-60: (H, D) of an MHA qkv tensor."""
    if qkv.dtype not in (torch.float16, torch.bfloat16):
        raise TypeError(f"qkv dtype must be float16 or bfloat16, got {qkv.dtype}")
    if qkv.ndim == 5:
        if qkv.shape[2] != 3:
            raise ValueError(f"explicit qkv layout must have shape [B,S,3,H,D], got {tuple(qkv.shape)}")
        return qkv.shape[3], qkv.shape[4]
    if qkv.ndim == 3:
        if H is None or D is None:
            raise ValueError("H and D are required for packed qkv layout [B,S,3*H*D]")
        if qkv.shape[2] != 3 * H * D:
            raise ValueError(
                f"packed qkv last dimension must equal 3*H*D={3 * H * D}, got {qkv.shape[2]}. "
                "For GQA/MQA fused layouts [Q;K;V] with Hq != Hkv, use mk.gqa_ops.reference_gqa_qkv_split.")
        return H, D
    raise ValueError(f"qkv must have shape [B,S,3*H*D] or [B,S,3,H,D], got {tuple(qkv.shape)}")


def _packed_rows(qkv, H: int, D: int):
    """[B,S,3,H,D] or [B,S,3*H*D] -> [B,S,3*H*D] (a view: the orders agree)."""
    return qkv.reshape(qkv.shape[0], qkv.shape[1], 3 * H * D)


def reference_paged_decode_block_from_qkv(qkv, K_pages, V_pages, block_table, cos, sin, position, *, H=None, D=None,
                                          scale=None):
    """ops/decode_block_ops.py:174-195 (MHA): per-sequence split + RoPE, the
    functional paged update, fp32 paged attention over position + 1."""
    _, page_size, _, _, batch, max_blocks = _validate_paged_cache(K_pages, V_pages, block_table)
    H_val, D_val = _mha_qkv_dims(qkv, H, D)
    q_rope, k_rope, v = _per_sequence_rope(_packed_rows(qkv, H_val, D_val), cos, sin, H_val, H_val, D_val, position)
    updated_K, updated_V = reference_paged_kv_cache_update(K_pages, V_pages, k_rope, v, block_table, position)
    lengths = _decode_lengths(position, batch, max_blocks * page_size, device=block_table.device)
    out = reference_paged_decode_attention(q_rope, updated_K, updated_V, block_table, lengths, scale=scale)
    return out, updated_K, updated_V


def paged_decode_block_from_qkv(qkv, K_pages, V_pages, block_table, cos, sin, position, *, H=None, D=None,
                                scale=None, backend: str = "auto"):
    """ops/decode_block_ops.py:198-257.  Returns (out [B,1,H,D], K_pages,
    V_pages); the HIP path writes the new token into the pages in place and
    returns the same tensors (the reference returns updated copies that its
    callers rebind).  Backends: 'auto' / 'metal' run the HIP block;
    'reference' the tensor-op composition; the GQA route also takes
    'metal_gqa' / 'metal_gqa_threadgroup'.  The names the reference rejects on
    the MHA route are rejected with its messages: its split step takes only
    'reference' / 'metal' / 'auto', and its attention step the attention
    backends."""
    _, page_size, heads, head_dim, batch, max_blocks = _validate_paged_cache(K_pages, V_pages, block_table)
    backend_name = backend.lower()
    if H is not None and heads != H:
        heads_kw = dict(num_attention_heads=H, num_key_value_heads=heads,
                        head_dim=D if D is not None else head_dim, scale=scale)
        if backend_name == "reference":
            return reference_paged_gqa_decode_block_from_qkv(qkv, K_pages, V_pages, block_table, cos, sin,
                                                             position, **heads_kw)
        return paged_gqa_decode_block_from_qkv(qkv, K_pages, V_pages, block_table, cos, sin, position,
                                               backend=backend_name, **heads_kw)
    if backend_name == "reference":
        return reference_paged_decode_block_from_qkv(qkv, K_pages, V_pages, block_table, cos, sin, position, H=H,
                                                     D=D, scale=scale)
    if backend_name in ("metal_gqa", "metal_gqa_threadgroup"):
        raise ValueError(_ATTN_BACKENDS_MSG)
    if backend_name not in ("auto", "metal"):
        raise ValueError("backend must be one of 'reference', 'metal', 'auto'")
    H_val, D_val = _mha_qkv_dims(qkv, H, D)
    if qkv.shape[1] != 1 or qkv.shape[0] != batch or heads != H_val or head_dim != D_val:
        raise ValueError(
            f"k_new/v_new must normalize to [B,1,H,D]={(batch, 1, heads, head_dim)}, got qkv {tuple(qkv.shape)} "
            f"with H={H_val}, D={D_val}")
    if D_val > 128:
        raise ValueError(f"paged_decode_attention currently supports D <= 128, got {D_val}")
    out, _, _ = paged_gqa_decode_block_from_qkv(_packed_rows(qkv, H_val, D_val), K_pages, V_pages, block_table, cos,
                                                sin, position, num_attention_heads=H_val,
                                                num_key_value_heads=H_val, head_dim=D_val, scale=scale,
                                                backend="metal")
    return out, K_pages, V_pages
