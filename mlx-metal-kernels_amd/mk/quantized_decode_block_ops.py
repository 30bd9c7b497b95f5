"""Quantized paged decode block -- drop-in for the paged path of
``ops/quantized_decode_block_ops.py``.

One decode step of a layer's attention half on a paged fp16/bf16 KV cache
(ops/quantized_decode_block_ops.py:446-552):
    qkv = x . Wqkv^T            (q4/q8 matvec, mk_q{4,8}_matvec)
    q, k, v = split(qkv); RoPE(q, k) at each sequence's position; the new k, v
        written to (block_table[b, pos // P], pos % P)     (mk_qkv_rope_paged_update)
    attn = paged GQA decode attention over positions 0..pos  (mk_paged_decode_attention)
    projected = attn . Wo^T     (q4/q8 matvec)
The cache is updated in place and returned, as the reference returns its
updated copies.
"""

from __future__ import annotations

import math

import torch

from . import _lib
from ._common import as_u8, scales_for_kernel
from .gqa_ops import paged_gqa_decode_block_from_qkv, reference_paged_gqa_decode_block_from_qkv
from .kv_cache_ops import normalize_positions
from .norm_ops import reference_rms_norm
from .paged_kv_ops import _hip_paged_attention, _i32
from .quant_ops import (
    q4_matvec_decode,
    q8_matvec_decode,
    q_matvec_residual,
    q_rmsnorm_matvec,
    reference_q4_matvec_decode,
    reference_q8_matvec_decode,
)


def validate_bits(bits: int) -> int:
    """ops/quantized_decode_block_ops.py:20-23."""
    if bits not in (4, 8):
        raise ValueError(f"bits must be 4 or 8, got {bits}")
    return bits


def normalize_hidden_input(x):
    """ops/quantized_decode_block_ops.py:26-37: [B,K], [B,1,K], [B,H,D] or
    [B,1,H,D] -> ([B,K], B, original shape)."""
    if x.ndim == 2:
        return x, x.shape[0], tuple(x.shape)
    if x.ndim == 3 and x.shape[1] == 1:
        return x[:, 0, :], x.shape[0], tuple(x.shape)
    if x.ndim == 3:
        B = x.shape[0]
        return x.reshape(B, x.shape[1] * x.shape[2]), B, tuple(x.shape)
    if x.ndim == 4 and x.shape[1] == 1:
        B = x.shape[0]
        return x.reshape(B, x.shape[2] * x.shape[3]), B, tuple(x.shape)
    raise ValueError(f"x must have shape [B,K], [B,1,K], [B,H,D], or [B,1,H,D], got {tuple(x.shape)}")


def infer_gqa_qkv_output_dim(num_attention_heads: int, num_key_value_heads: int, head_dim: int) -> int:
    """ops/quantized_decode_block_ops.py:65-66."""
    return (num_attention_heads + 2 * num_key_value_heads) * head_dim


def infer_qkv_dims(qkv_w, H, D, bits: int):
    """ops/quantized_decode_block_ops.py:40-62 (fused MHA qkv: 3*H*D rows)."""
    validate_bits(bits)
    if qkv_w.ndim != 2:
        raise ValueError(f"qkv_w must be 2-D, got {tuple(qkv_w.shape)}")
    rows = qkv_w.shape[0]
    if rows % 3 != 0:
        raise ValueError(f"qkv_w output rows must be divisible by 3, got {rows}")
    if H is not None and D is not None:
        if 3 * H * D != rows:
            raise ValueError(f"qkv_w output rows must equal 3*H*D={3 * H * D}, got {rows}")
        return H, D
    per = rows // 3
    if H is not None:
        if per % H != 0:
            raise ValueError(f"qkv_w output rows imply per-projection dim {per}, not divisible by H={H}")
        return H, per // H
    if D is not None:
        if per % D != 0:
            raise ValueError(f"qkv_w output rows imply per-projection dim {per}, not divisible by D={D}")
        return per // D, D
    raise ValueError("H and D must be provided when qkv dimensions cannot be inferred uniquely")


def validate_quantized_weight_shapes(x2d, w, scales, zeros, *, bits: int, group_size: int,
                                     expected_in_dim: int | None = None, expected_out_dim: int | None = None,
                                     name: str):
    """ops/quantized_decode_block_ops.py:69-110 -> (in_dim, out_dim)."""
    validate_bits(bits)
    if group_size <= 0:
        raise ValueError(f"group_size must be positive, got {group_size}")
    if x2d.ndim != 2:
        raise ValueError(f"{name} input must normalize to [B,K], got {tuple(x2d.shape)}")
    if w.ndim != 2:
        raise ValueError(f"{name} weights must be 2-D, got {tuple(w.shape)}")
    in_dim = x2d.shape[1]
    if expected_in_dim is not None and in_dim != expected_in_dim:
        raise ValueError(f"{name} input dim must be {expected_in_dim}, got {in_dim}")
    out_dim = w.shape[0]
    if expected_out_dim is not None and out_dim != expected_out_dim:
        raise ValueError(f"{name} output dim must be {expected_out_dim}, got {out_dim}")
    if bits == 4:
        packed = math.ceil(in_dim / 2)
        if w.shape[1] != packed:
            raise ValueError(f"{name} q4 weights must have shape [N,{packed}], got {tuple(w.shape)}")
    elif w.shape[1] != in_dim:
        raise ValueError(f"{name} q8 weights must have shape [N,{in_dim}], got {tuple(w.shape)}")
    groups = math.ceil(in_dim / group_size)
    if tuple(scales.shape) != (out_dim, groups):
        raise ValueError(f"{name} scales must have shape {(out_dim, groups)}, got {tuple(scales.shape)}")
    if zeros is not None and tuple(zeros.shape) != (out_dim, groups):
        raise ValueError(f"{name} zeros must have shape {(out_dim, groups)}, got {tuple(zeros.shape)}")
    return in_dim, out_dim


def _matvec_dispatch(x2d, w, scales, zeros, *, bits: int, group_size: int, backend: str, reference: bool):
    """ops/quantized_decode_block_ops.py:113-131."""
    validate_bits(bits)
    if reference:
        fn = reference_q4_matvec_decode if bits == 4 else reference_q8_matvec_decode
        return fn(x2d, w, scales, zeros, group_size=group_size)
    fn = q4_matvec_decode if bits == 4 else q8_matvec_decode
    return fn(x2d, w, scales, zeros, group_size=group_size, backend=backend)


def quantized_qkv_projection(x, qkv_w, qkv_scales, qkv_zeros=None, *, bits=4, group_size=32, backend="auto"):
    """ops/quantized_decode_block_ops.py:154-184 -> [B,1,N]."""
    x2d, B, _ = normalize_hidden_input(x)
    validate_quantized_weight_shapes(x2d, qkv_w, qkv_scales, qkv_zeros, bits=bits, group_size=group_size,
                                     name="qkv_projection")
    qkv = _matvec_dispatch(x2d, qkv_w, qkv_scales, qkv_zeros, bits=bits, group_size=group_size, backend=backend,
                           reference=backend.lower() == "reference")
    return qkv.reshape(B, 1, qkv.shape[1])


def reference_quantized_qkv_projection(x, qkv_w, qkv_scales, qkv_zeros=None, *, bits=4, group_size=32):
    """ops/quantized_decode_block_ops.py:134-151."""
    return quantized_qkv_projection(x, qkv_w, qkv_scales, qkv_zeros, bits=bits, group_size=group_size,
                                    backend="reference")


def quantized_output_projection(x, out_w, out_scales, out_zeros=None, *, bits=4, group_size=32, backend="auto"):
    """ops/quantized_decode_block_ops.py:207-237 -> [B,1,out]."""
    x2d, B, _ = normalize_hidden_input(x)
    _, out_dim = validate_quantized_weight_shapes(x2d, out_w, out_scales, out_zeros, bits=bits,
                                                  group_size=group_size, name="output_projection")
    y = _matvec_dispatch(x2d, out_w, out_scales, out_zeros, bits=bits, group_size=group_size, backend=backend,
                         reference=backend.lower() == "reference")
    return y.reshape(B, 1, out_dim)


def reference_quantized_output_projection(x, out_w, out_scales, out_zeros=None, *, bits=4, group_size=32):
    """ops/quantized_decode_block_ops.py:187-204."""
    return quantized_output_projection(x, out_w, out_scales, out_zeros, bits=bits, group_size=group_size,
                                       backend="reference")


def _block_dims(qkv_w, H, num_key_value_heads, head_dim, D, bits):
    """Head counts as ops/quantized_decode_block_ops.py:475-484 resolves them."""
    if head_dim is not None:
        D = head_dim
    kv_heads = num_key_value_heads if num_key_value_heads is not None else H
    if kv_heads is None:
        H, D = infer_qkv_dims(qkv_w, H, D, bits)
        kv_heads = H
    elif H is None or D is None:
        raise ValueError("H and head_dim/D are required for GQA paged quantized decode block")
    return H, kv_heads, D


def rmsnorm_qkv_rope_paged_update(x2d, norm_weight, qkv_w, qkv_scales, qkv_zeros, K_pages, V_pages, block_table,
                                  cos, sin, position, *, num_attention_heads, num_key_value_heads, head_dim, bits=4,
                                  group_size=32, eps=1e-5):
    """Input RMSNorm + qkv projection + GQA split + interleaved RoPE + paged
    write of the new token (ops/llama_layer_ops.py:256-260 feeding
    ops/gqa_ops.py:493-547 up to the attention call) -- one HIP launch for a
    q4 fp16 decode row (mk_q4_rmsnorm_qkv_rope_paged), the projection then
    mk_qkv_rope_paged_update otherwise, with identical rounding either way.
    x2d [B, hidden]; K_pages/V_pages [NUM_PAGES, P, Hkv, D] in x's dtype,
    updated in place.  Returns (q [B, 1, Hq, D], positions int32 [B])."""
    Hq, Hkv, D = num_attention_heads, num_key_value_heads, head_dim
    if bits not in (4, 8):
        raise ValueError(f"bits must be 4 or 8, got {bits}")
    if D % 2 != 0:
        raise ValueError(f"RoPE requires even D, got D={D}")
    if K_pages.shape != V_pages.shape or K_pages.ndim != 4 or K_pages.shape[2] != Hkv or K_pages.shape[3] != D:
        raise ValueError(f"K_pages/V_pages must be [NUM_PAGES,PAGE_SIZE,{Hkv},{D}], got {tuple(K_pages.shape)}")
    if K_pages.dtype != x2d.dtype or V_pages.dtype != x2d.dtype:
        raise TypeError(f"K_pages/V_pages must carry the activation dtype {x2d.dtype}")
    if not (K_pages.is_contiguous() and V_pages.is_contiguous()):
        raise ValueError("K_pages and V_pages must be contiguous for the in-place update")
    B, K = x2d.shape
    if tuple(norm_weight.shape) != (K,):
        raise ValueError(f"norm_weight must have shape {(K,)}, got {tuple(norm_weight.shape)}")
    if block_table.shape[0] != B:
        raise ValueError(f"block_table batch {block_table.shape[0]} != x batch {B}")
    N = (Hq + 2 * Hkv) * D
    w8 = as_u8(qkv_w)
    cols = math.ceil(K / 2) if bits == 4 else K
    if w8.ndim != 2 or tuple(w8.shape) != (N, cols):
        raise ValueError(f"qkv_w must have shape [{N},{cols}], got {tuple(w8.shape)}")
    x2d = x2d.contiguous()
    nw = norm_weight.contiguous()
    dev = _lib.require_device(x2d, nw, w8, qkv_scales, qkv_zeros, K_pages, V_pages, block_table)
    s, z = scales_for_kernel(qkv_scales, qkv_zeros)
    P, MAX_BLOCKS = K_pages.shape[1], block_table.shape[1]
    pos = normalize_positions(position, B, cos.shape[0], device=dev)
    pos = normalize_positions(pos, B, MAX_BLOCKS * P, device=dev)
    c = cos.to(device=dev, dtype=torch.float32).contiguous()
    sn = sin.to(device=dev, dtype=torch.float32).contiguous()
    bt = _i32(block_table, dev)
    q_out = torch.empty((B, 1, Hq, D), dtype=x2d.dtype, device=dev)
    scratch = torch.empty((B, N), dtype=x2d.dtype, device=dev)  # the two-launch path's projection
    normed = torch.empty_like(x2d)
    name = "mk_q4_rmsnorm_qkv_rope_paged" if bits == 4 else "mk_q8_rmsnorm_qkv_rope_paged"
    _lib.launch(name, dev, _lib.ptr(x2d), _lib.ptr(nw), float(eps), _lib.ptr(w8), _lib.ptr(s), _lib.ptr(z),
                _lib.ptr(scratch), _lib.ptr(normed), _lib.ptr(c), _lib.ptr(sn), _lib.ptr(pos), _lib.ptr(bt),
                _lib.ptr(K_pages), _lib.ptr(V_pages), _lib.ptr(q_out), B, Hq, Hkv, D, P, MAX_BLOCKS,
                K_pages.shape[0], c.shape[0], K, group_size, _lib.dtype_code(x2d.dtype), _lib.dtype_code(s.dtype),
                _lib.dtype_code(nw.dtype))
    return q_out, pos


def paged_quantized_decode_block(x, qkv_w, qkv_scales, out_w, out_scales, K_pages, V_pages, block_table, cos, sin,
                                 position, *, qkv_zeros=None, out_zeros=None, bits=4, group_size=32, H=None,
                                 num_key_value_heads=None, head_dim=None, D=None, scale=None,
                                 matvec_backend="metal_parallel", block_backend="auto", return_intermediates=False,
                                 residual=None, norm_weight=None, eps=1e-5, lengths=None, verify_width=1):
    """ops/quantized_decode_block_ops.py:446-552: returns (projected [B,1,H*D
    -> hidden], K_pages, V_pages) or with (qkv, attn_out) appended.

    Extensions, not in the reference, that let the layer fuse its
    neighbours: ``residual`` makes ``projected`` residual + round(attn .
    Wo^T) (the matvec's residual epilogue; the layer's residual_add,
    ops/llama_layer_ops.py:355-359); ``norm_weight`` takes x before the
    layer's input RMSNorm and runs the norm inside the qkv matvec
    (ops/llama_layer_ops.py:256-260); ``lengths`` = position + 1 as a device
    tensor, computed once for all layers.  ``verify_width`` W > 1: x holds W
    consecutive draft rows per sequence (row b * W + w at position
    position[b * W + w], the block table repeated W times); the attention
    then runs as mk_paged_verify_attention over the sequences' own table rows
    (one K/V read for the W rows), with ``lengths`` (required) per sequence,
    the last row's position + 1."""
    x2d, _, _ = normalize_hidden_input(x)
    H, kv_heads, D = _block_dims(qkv_w, H, num_key_value_heads, head_dim, D, bits)
    validate_quantized_weight_shapes(x2d, qkv_w, qkv_scales, qkv_zeros, bits=bits, group_size=group_size,
                                     expected_out_dim=infer_gqa_qkv_output_dim(H, kv_heads, D),
                                     name="qkv_projection")
    validate_quantized_weight_shapes(x2d.new_empty((x2d.shape[0], H * D)), out_w, out_scales, out_zeros, bits=bits,
                                     group_size=group_size, expected_in_dim=H * D, name="output_projection")
    reference = matvec_backend.lower() == "reference"
    fuse_front = (norm_weight is not None and not reference and not return_intermediates and
                  block_backend.lower() != "reference" and K_pages.dtype == x2d.dtype and
                  K_pages.dtype in (torch.float16, torch.bfloat16))
    if fuse_front:
        # norm + qkv + RoPE + cache write in one launch, then the attention
        q, pos = rmsnorm_qkv_rope_paged_update(
            x2d, norm_weight, qkv_w, qkv_scales, qkv_zeros, K_pages, V_pages, block_table, cos, sin, position,
            num_attention_heads=H, num_key_value_heads=kv_heads, head_dim=D, bits=bits, group_size=group_size,
            eps=eps)
        sc = 1.0 / math.sqrt(D) if scale is None else scale
        if verify_width > 1:
            from .speculative_verify_ops import _hip_verify_attention

            W = verify_width
            if lengths is None or q.shape[0] % W:
                raise ValueError("verify_width needs B * W rows and per-sequence lengths")
            bt_seq = block_table[::W].contiguous()
            attn_out = _hip_verify_attention(q.reshape(-1, W, H, D), K_pages, V_pages, bt_seq, lengths,
                                             sc).reshape(q.shape[0], 1, H, D)
        else:
            attn_out = _hip_paged_attention(q[:, 0], K_pages, V_pages, _i32(block_table, q.device),
                                            pos + 1 if lengths is None else lengths, sc).unsqueeze(1)
    elif norm_weight is not None and not reference:
        qkv = q_rmsnorm_matvec(x2d, norm_weight, qkv_w, qkv_scales, qkv_zeros, bits=bits, group_size=group_size,
                               eps=eps).reshape(x2d.shape[0], 1, -1)
    else:
        if norm_weight is not None:
            x2d = reference_rms_norm(x2d[:, None], norm_weight, eps=eps)[:, 0]
        qkv = quantized_qkv_projection(x2d, qkv_w, qkv_scales, qkv_zeros, bits=bits, group_size=group_size,
                                       backend=matvec_backend)
    block_fn = reference_paged_gqa_decode_block_from_qkv if block_backend.lower() == "reference" else None
    if fuse_front:
        pass
    elif block_fn is not None:
        attn_out, K_pages, V_pages = block_fn(qkv, K_pages, V_pages, block_table, cos, sin, position,
                                              num_attention_heads=H, num_key_value_heads=kv_heads, head_dim=D,
                                              scale=scale)
    else:
        attn_out, K_pages, V_pages = paged_gqa_decode_block_from_qkv(
            qkv, K_pages, V_pages, block_table, cos, sin, position, num_attention_heads=H,
            num_key_value_heads=kv_heads, head_dim=D, scale=scale, backend=block_backend,
            lengths=lengths if verify_width == 1 else None)  # verify rows here: one sequence each
    B = attn_out.shape[0]
    a2d = attn_out.reshape(B, H * D)
    if residual is not None and not reference:
        _, out = q_matvec_residual(a2d, out_w, out_scales, out_zeros, residual.reshape(B, -1), bits=bits,
                                   group_size=group_size)
        projected = out.reshape(B, 1, -1)
    else:
        projected = quantized_output_projection(a2d, out_w, out_scales, out_zeros, bits=bits, group_size=group_size,
                                                backend=matvec_backend)
        if residual is not None:
            projected = (residual.reshape(B, 1, -1).float() + projected.float()).to(projected.dtype)
    if return_intermediates:
        return projected, K_pages, V_pages, qkv, attn_out
    return projected, K_pages, V_pages


def reference_paged_quantized_decode_block(x, qkv_w, qkv_scales, out_w, out_scales, K_pages, V_pages, block_table,
                                           cos, sin, position, *, qkv_zeros=None, out_zeros=None, bits=4,
                                           group_size=32, H=None, num_key_value_heads=None, head_dim=None, D=None,
                                           scale=None, return_intermediates=False):
    """ops/quantized_decode_block_ops.py:395-443 (reference matvecs and
    reference paged block; K_pages / V_pages are updated functionally)."""
    return paged_quantized_decode_block(
        x, qkv_w, qkv_scales, out_w, out_scales, K_pages.clone(), V_pages.clone(), block_table, cos, sin, position,
        qkv_zeros=qkv_zeros, out_zeros=out_zeros, bits=bits, group_size=group_size, H=H,
        num_key_value_heads=num_key_value_heads, head_dim=head_dim, D=D, scale=scale, matvec_backend="reference",
        block_backend="reference", return_intermediates=return_intermediates)

