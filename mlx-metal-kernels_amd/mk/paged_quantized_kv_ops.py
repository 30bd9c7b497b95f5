"""Paged symmetric q8/q4 KV cache -- drop-in for ``ops/paged_quantized_kv_ops.py``.

Format (ops/paged_quantized_kv_ops.py:146-186): per (page, slot, kv head,
group of ``group_size`` along D) one fp16 scale s = max(max|v|, 1e-8) / 127
(q8) or / 7 (q4), computed in fp32 and rounded to fp16 after use; codes
clip(round_half_even(v / s), -127, 127) + 128 (uint8) or
clip(..., -7, 7) + 8 packed two per byte (low nibble = even d).

Decode attention backends: ``"reference"`` (tensor ops), ``"metal_q8"`` /
``"metal_q4"`` (gfx950 HIP split-K kernel; bits must match).  Unlike the
reference's array path, the reference here honours per-sequence lengths
(the reference gathers only valid rows and then masks against MAX_S, which
only works when every length equals MAX_S).

New (no reference counterpart, whose docs list it as missing):
``paged_quantized_kv_update_from_qkv`` -- the fused qkv split + RoPE +
quantize + paged write of one decode token.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Any

import torch

from . import _lib
from .gqa_ops import _per_sequence_rope, _qkv_rope_update_prep, validate_gqa_heads
from .kv_cache_ops import normalize_positions
from .paged_kv_ops import _i32
from .quant_ops import unpack_q4_reference

_MAX_HEAD_DIM = 128


@dataclass
class PagedQuantizedKVConfig:
    """ops/paged_quantized_kv_ops.py:38-61."""

    bits: int = 8
    page_size: int = 16
    group_size: int = 32
    symmetric: bool = True
    with_zeros: bool = False
    scale_dtype: str = "float16"
    layout: str = "paged"

    def validate(self) -> "PagedQuantizedKVConfig":
        if self.bits not in (4, 8):
            raise ValueError(f"bits must be 4 or 8, got {self.bits}")
        if self.page_size <= 0:
            raise ValueError(f"page_size must be > 0, got {self.page_size}")
        if self.group_size <= 0:
            raise ValueError(f"group_size must be > 0, got {self.group_size}")
        if not self.symmetric:
            raise NotImplementedError("asymmetric quantization is not implemented yet")
        if self.with_zeros:
            raise NotImplementedError("zero-point quantization is not implemented yet")
        if self.layout != "paged":
            raise ValueError(f"layout must be 'paged', got {self.layout!r}")
        return self


@dataclass
class PagedQuantizedKVCache:
    """ops/paged_quantized_kv_ops.py:69-138."""

    k_pages_q: Any
    v_pages_q: Any
    k_scales: Any
    v_scales: Any
    block_table: Any
    lengths: Any
    k_zeros: Any | None = None
    v_zeros: Any | None = None
    bits: int = 8
    page_size: int = 16
    group_size: int = 32
    original_page_shape: tuple[int, ...] | None = None
    metadata: dict[str, Any] = field(default_factory=dict)

    def shapes(self) -> dict[str, tuple[int, ...] | None]:
        return {
            "k_pages_q": tuple(self.k_pages_q.shape),
            "v_pages_q": tuple(self.v_pages_q.shape),
            "k_scales": tuple(self.k_scales.shape),
            "v_scales": tuple(self.v_scales.shape),
            "block_table": tuple(self.block_table.shape),
            "lengths": tuple(self.lengths.shape),
            "original_page_shape": None if self.original_page_shape is None else tuple(self.original_page_shape),
        }

    def validate(self) -> "PagedQuantizedKVCache":
        if self.bits not in (4, 8):
            raise ValueError(f"bits must be 4 or 8, got {self.bits}")
        if self.k_pages_q.shape != self.v_pages_q.shape:
            raise ValueError(f"k_pages_q and v_pages_q shapes must match, got {tuple(self.k_pages_q.shape)} != {tuple(self.v_pages_q.shape)}")
        if self.k_scales.shape != self.v_scales.shape:
            raise ValueError(f"k_scales and v_scales shapes must match, got {tuple(self.k_scales.shape)} != {tuple(self.v_scales.shape)}")
        if self.block_table.ndim != 2:
            raise ValueError(f"block_table must be 2-D [B,MAX_BLOCKS], got {tuple(self.block_table.shape)}")
        if self.lengths.ndim != 1:
            raise ValueError(f"lengths must be 1-D [B], got {tuple(self.lengths.shape)}")
        B = self.block_table.shape[0]
        if self.lengths.shape[0] != B:
            raise ValueError(f"lengths batch {self.lengths.shape[0]} != block_table batch {B}")
        if self.original_page_shape is not None and len(self.original_page_shape) != 4:
            raise ValueError(f"original_page_shape must be 4-D [NUM_PAGES,PAGE_SIZE,Hkv,D], got {self.original_page_shape}")
        return self

    def num_pages(self) -> int:
        return self.k_pages_q.shape[0]

    def memory_bytes(self) -> int:
        total = 0
        for arr in (self.k_pages_q, self.v_pages_q, self.k_scales, self.v_scales, self.block_table, self.lengths):
            total += arr.numel() * arr.element_size()
        for arr in (self.k_zeros, self.v_zeros):
            if arr is not None:
                total += arr.numel() * arr.element_size()
        return total

    def compression_ratio(self, fp_bytes_per_value: int = 2) -> float | None:
        if self.original_page_shape is None:
            return None
        NUM_PAGES, PAGE_SIZE, Hkv, D = self.original_page_shape
        fp_bytes = 2 * NUM_PAGES * PAGE_SIZE * Hkv * D * fp_bytes_per_value
        q_bytes = sum(a.numel() * a.element_size() for a in (self.k_pages_q, self.v_pages_q, self.k_scales, self.v_scales))
        return None if q_bytes == 0 else fp_bytes / q_bytes


# ----------------------------------------------------------------- quantizers


def _qparams(bits: int):
    return (127.0, 128) if bits == 8 else (7.0, 8)


def _quantize_last_dim(values: torch.Tensor, group_size: int, bits: int):
    """Symmetric per-group quantization along the last dim of an fp32 tensor.
    Returns (codes uint8 [..., D] unpacked, scales fp16 [..., G])."""
    qmax, off = _qparams(bits)
    D = values.shape[-1]
    G = (D + group_size - 1) // group_size
    pad = G * group_size - D
    v = values.to(torch.float32)
    vp = torch.nn.functional.pad(v, (0, pad)) if pad else v
    amax = vp.reshape(*v.shape[:-1], G, group_size).abs().amax(dim=-1)
    amax = torch.clamp(amax, min=1e-8)
    scale = amax / torch.tensor(qmax, dtype=torch.float32)
    scale_full = torch.repeat_interleave(scale, group_size, dim=-1)[..., :D]
    q = torch.clamp(torch.round(v / scale_full), -qmax, qmax) + off
    return q.to(torch.uint8), scale.to(torch.float16)


def _pack_last_dim(codes: torch.Tensor) -> torch.Tensor:
    D = codes.shape[-1]
    if D % 2:
        codes = torch.nn.functional.pad(codes, (0, 1))
    return (codes[..., 0::2] + (codes[..., 1::2] << 4)).to(torch.uint8)


def _quantize_group_symmetric_8(values, eps: float = 1e-8):
    """ops/paged_quantized_kv_ops.py:146-153 (one group along the last dim)."""
    max_abs = torch.clamp(values.to(torch.float32).abs().amax(dim=-1, keepdim=True), min=eps)
    scale = max_abs / 127.0
    q = torch.clamp(torch.round(values.to(torch.float32) / scale), -127, 127) + 128
    return q.to(torch.uint8), scale.squeeze(-1).to(torch.float16)


def _quantize_group_symmetric_4(values, eps: float = 1e-8):
    """ops/paged_quantized_kv_ops.py:168-175."""
    max_abs = torch.clamp(values.to(torch.float32).abs().amax(dim=-1, keepdim=True), min=eps)
    scale = max_abs / 7.0
    q = torch.clamp(torch.round(values.to(torch.float32) / scale), -7, 7) + 8
    return q.to(torch.uint8), scale.squeeze(-1).to(torch.float16)


def _dequant_last_dim(codes_unpacked: torch.Tensor, scales: torch.Tensor, group_size: int, bits: int, D: int):
    """ops/paged_quantized_kv_ops.py:156-186: (code - off) * |s| in fp32."""
    _, off = _qparams(bits)
    s = torch.repeat_interleave(scales.to(torch.float32).abs(), group_size, dim=-1)
    if s.shape[-1] >= D:
        s = s[..., :D]
    else:
        s = torch.nn.functional.pad(s, (0, D - s.shape[-1]))
    return (codes_unpacked.to(torch.float32) - float(off)) * s


def _dequant_group_symmetric_8(q_unsigned, scales, group_size: int, D: int):
    return _dequant_last_dim(q_unsigned, scales, group_size, 8, D)


def _dequant_group_symmetric_4(q_unsigned, scales, group_size: int, D: int):
    return _dequant_last_dim(q_unsigned, scales, group_size, 4, D)


def quantize_kv_pages(K_pages, V_pages, block_table, lengths, config: PagedQuantizedKVConfig) -> PagedQuantizedKVCache:
    """ops/paged_quantized_kv_ops.py:194-292 (every page, vectorised)."""
    config = config.validate()
    if K_pages.shape != V_pages.shape:
        raise ValueError(f"K_pages and V_pages must match, got {tuple(K_pages.shape)} != {tuple(V_pages.shape)}")
    if K_pages.ndim != 4:
        raise ValueError(f"K_pages must be 4-D [NUM_PAGES,PAGE_SIZE,Hkv,D], got {tuple(K_pages.shape)}")
    if K_pages.device.type == "cuda":
        kq, ks = _hip_quantize_rows(K_pages, config.group_size, config.bits)
        vq, vs = _hip_quantize_rows(V_pages, config.group_size, config.bits)
    else:
        kq, ks = _quantize_last_dim(K_pages.to(torch.float32), config.group_size, config.bits)
        vq, vs = _quantize_last_dim(V_pages.to(torch.float32), config.group_size, config.bits)
        if config.bits == 4:
            kq, vq = _pack_last_dim(kq), _pack_last_dim(vq)
    return PagedQuantizedKVCache(
        k_pages_q=kq, v_pages_q=vq, k_scales=ks, v_scales=vs, block_table=block_table, lengths=lengths,
        bits=config.bits, page_size=config.page_size, group_size=config.group_size,
        original_page_shape=tuple(K_pages.shape),
    )


def _hip_quantize_rows(pages: torch.Tensor, group_size: int, bits: int):
    """mk_quantize_kv over every (page, slot, head) row of a device tensor."""
    if pages.dtype not in (torch.float16, torch.bfloat16):
        pages = pages.to(torch.float16)
    src = pages.contiguous()
    dev = _lib.require_device(src)
    *lead, D = src.shape
    rows = src.numel() // D
    G = (D + group_size - 1) // group_size
    codes = torch.empty(tuple(lead) + ((D if bits == 8 else (D + 1) // 2),), dtype=torch.uint8, device=dev)
    scales = torch.empty(tuple(lead) + (G,), dtype=torch.float16, device=dev)
    _lib.launch("mk_quantize_kv", dev, _lib.ptr(src), _lib.ptr(codes), _lib.ptr(scales), rows, D, group_size, bits,
                _lib.dtype_code(src.dtype))
    return codes, scales


def _unpacked_codes(paged_qkv: PagedQuantizedKVCache, which: str, D: int) -> torch.Tensor:
    codes = paged_qkv.k_pages_q if which == "k" else paged_qkv.v_pages_q
    if paged_qkv.bits == 8:
        return codes
    flat = codes.reshape(-1, codes.shape[-1])
    return unpack_q4_reference(flat, K=D).reshape(*codes.shape[:-1], D)


def dequantize_kv_pages(paged_qkv: PagedQuantizedKVCache):
    """ops/paged_quantized_kv_ops.py:295-341 -> fp16 (K, V)."""
    paged_qkv = paged_qkv.validate()
    orig = paged_qkv.original_page_shape
    if orig is None:
        raise ValueError("original_page_shape is required for dequantization")
    D = orig[3]
    K = _dequant_last_dim(_unpacked_codes(paged_qkv, "k", D), paged_qkv.k_scales, paged_qkv.group_size,
                          paged_qkv.bits, D).to(torch.float16)
    V = _dequant_last_dim(_unpacked_codes(paged_qkv, "v", D), paged_qkv.v_scales, paged_qkv.group_size,
                          paged_qkv.bits, D).to(torch.float16)
    return K, V


def paged_quantized_kv_error(K_pages, V_pages, paged_qkv: PagedQuantizedKVCache) -> dict[str, float]:
    """ops/paged_quantized_kv_ops.py:344-367."""
    K_deq, V_deq = dequantize_kv_pages(paged_qkv)
    kd = K_pages.to(torch.float32) - K_deq.to(torch.float32)
    vd = V_pages.to(torch.float32) - V_deq.to(torch.float32)
    cr = paged_qkv.compression_ratio(fp_bytes_per_value=2)
    return {
        "k_max_abs_error": float(kd.abs().max()),
        "k_mean_abs_error": float(kd.abs().mean()),
        "k_rmse": float(torch.sqrt(torch.mean(kd ** 2))),
        "v_max_abs_error": float(vd.abs().max()),
        "v_mean_abs_error": float(vd.abs().mean()),
        "v_rmse": float(torch.sqrt(torch.mean(vd ** 2))),
        "compression_ratio": float(cr) if cr is not None else 0.0,
    }


def contiguous_kv_to_pages(K_cache, V_cache, lengths, *, page_size: int):
    """ops/paged_quantized_kv_ops.py:375-403: identity paging, page_id =
    b*max_blocks + blk, unused block-table entries -1."""
    if K_cache.ndim != 4 or V_cache.ndim != 4:
        raise ValueError(f"K_cache/V_cache must be 4-D [B,MAX_S,Hkv,D], got {tuple(K_cache.shape)}, {tuple(V_cache.shape)}")
    B, MAX_S, Hkv, D = K_cache.shape
    max_blocks = (MAX_S + page_size - 1) // page_size
    num_pages = B * max_blocks
    dev = K_cache.device
    K_pages = torch.zeros((num_pages, page_size, Hkv, D), dtype=K_cache.dtype, device=dev)
    V_pages = torch.zeros((num_pages, page_size, Hkv, D), dtype=V_cache.dtype, device=dev)
    block_table = torch.full((B, max_blocks), -1, dtype=torch.int32, device=dev)
    length_list = [int(v) for v in (lengths.tolist() if hasattr(lengths, "tolist") else lengths)]
    for b in range(B):
        valid = length_list[b]
        if valid <= 0:
            continue
        pos = torch.arange(valid, device=dev)
        pid = b * max_blocks + pos // page_size
        K_pages[pid, pos % page_size] = K_cache[b, :valid]
        V_pages[pid, pos % page_size] = V_cache[b, :valid]
        nblk = (valid + page_size - 1) // page_size
        block_table[b, :nblk] = torch.arange(nblk, dtype=torch.int32, device=dev) + b * max_blocks
    return K_pages, V_pages, block_table, torch.tensor(length_list, dtype=torch.int32, device=dev)


def pages_to_contiguous_kv(K_pages, V_pages, block_table, lengths, *, max_seq_len=None):
    """ops/paged_quantized_kv_ops.py:406-432."""
    B, MAX_BLOCKS = block_table.shape
    NUM_PAGES, PAGE_SIZE, Hkv, D = K_pages.shape
    if max_seq_len is None:
        max_seq_len = MAX_BLOCKS * PAGE_SIZE
    dev = K_pages.device
    K_cache = torch.zeros((B, max_seq_len, Hkv, D), dtype=K_pages.dtype, device=dev)
    V_cache = torch.zeros((B, max_seq_len, Hkv, D), dtype=V_pages.dtype, device=dev)
    for b in range(B):
        valid = int(lengths[b])
        if valid <= 0:
            continue
        pos = torch.arange(valid, device=dev)
        pid = block_table[b].long()[pos // PAGE_SIZE]
        keep = pid >= 0
        pos, pid = pos[keep], pid[keep]
        K_cache[b, pos] = K_pages[pid, pos % PAGE_SIZE]
        V_cache[b, pos] = V_pages[pid, pos % PAGE_SIZE]
    return K_cache, V_cache


# ----------------------------------------------------------------- decode attention


def _validate_paged_quantized_decode_inputs(q, paged_qkv: PagedQuantizedKVCache):
    """ops/paged_quantized_kv_ops.py:440-466."""
    if q.ndim != 4:
        raise ValueError(f"q must be 4-D [B,1,Hq,D], got {tuple(q.shape)}")
    if q.shape[1] != 1:
        raise ValueError(f"q must have shape [B,1,Hq,D], got {tuple(q.shape)}")
    B, _, Hq, D = q.shape
    orig = paged_qkv.original_page_shape
    if orig is None:
        raise ValueError("original_page_shape is required for decode attention")
    _, PAGE_SIZE, Hkv, D_cache = orig
    cache_B = paged_qkv.block_table.shape[0]
    if B != cache_B:
        raise ValueError(f"batch mismatch: q batch={B}, cache batch={cache_B}")
    if D != D_cache:
        raise ValueError(f"head_dim mismatch: q D={D}, cache D={D_cache}")
    validate_gqa_heads(Hq, Hkv)
    MAX_BLOCKS = paged_qkv.block_table.shape[1]
    MAX_S = MAX_BLOCKS * PAGE_SIZE
    lengths_arr = torch.clamp(paged_qkv.lengths.reshape(B).to(torch.int32), max=MAX_S)
    return lengths_arr, B, MAX_S, PAGE_SIZE, MAX_BLOCKS, Hq, Hkv, D


def reference_paged_quantized_kv_gqa_decode_attention(q, paged_qkv: PagedQuantizedKVCache, *, scale=None):
    """ops/paged_quantized_kv_ops.py:469-515 with per-sequence lengths:
    dequantize to fp16, gather positions j < lengths[b] through the block
    table (page ids < 0 skipped), fp32 softmax attention per query head."""
    from .paged_kv_ops import _gather_pages, _masked_attention

    lengths_arr, B, MAX_S, PAGE_SIZE, MAX_BLOCKS, Hq, Hkv, D = _validate_paged_quantized_decode_inputs(q, paged_qkv)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    K_deq, V_deq = dequantize_kv_pages(paged_qkv)
    bt = paged_qkv.block_table.to(K_deq.device)
    Kc, valid = _gather_pages(K_deq, bt, MAX_S)
    Vc, _ = _gather_pages(V_deq, bt, MAX_S)
    return _masked_attention(q[:, 0], Kc, Vc, lengths_arr, valid, scale).unsqueeze(1).to(q.dtype)


def _check_kernel_layout(paged_qkv: PagedQuantizedKVCache, Hkv: int, D: int) -> int:
    """The kernels index codes and scales from (num_pages, page_size, Hkv, D,
    bits, group_size) alone, so the tensors must have exactly that layout:
    codes [NP, P, Hkv, D] (q8) or [NP, P, Hkv, ceil(D/2)] (q4), scales
    [NP, P, Hkv, ceil(D/group_size)].  Returns NP, taken from the tensors."""
    P, g = int(paged_qkv.page_size), int(paged_qkv.group_size)
    if paged_qkv.bits not in (4, 8):
        raise ValueError(f"bits must be 4 or 8, got {paged_qkv.bits}")
    if P <= 0 or g <= 0:
        raise ValueError(f"page_size and group_size must be positive, got {P}, {g}")
    if paged_qkv.k_pages_q.ndim != 4:
        raise ValueError(f"k_pages_q must be 4-D [NUM_PAGES,PAGE_SIZE,Hkv,Dq], got {tuple(paged_qkv.k_pages_q.shape)}")
    NP = int(paged_qkv.k_pages_q.shape[0])
    Dq = D if paged_qkv.bits == 8 else (D + 1) // 2
    want_codes = (NP, P, Hkv, Dq)
    want_scales = (NP, P, Hkv, (D + g - 1) // g)
    for name, t, want in (("k_pages_q", paged_qkv.k_pages_q, want_codes), ("v_pages_q", paged_qkv.v_pages_q, want_codes),
                          ("k_scales", paged_qkv.k_scales, want_scales), ("v_scales", paged_qkv.v_scales, want_scales)):
        if tuple(t.shape) != want:
            raise ValueError(f"{name} must have shape {want} for bits={paged_qkv.bits}, page_size={P}, Hkv={Hkv}, "
                             f"D={D}, group_size={g}; got {tuple(t.shape)}")
    orig = paged_qkv.original_page_shape
    if orig is not None and tuple(orig[1:]) != (P, Hkv, D):
        raise ValueError(f"original_page_shape {tuple(orig)} disagrees with page_size={P}, Hkv={Hkv}, D={D}")
    return NP


def _hip_quantized_attention(q, paged_qkv: PagedQuantizedKVCache, lengths_arr, scale: float):
    B, _, Hq, D = q.shape
    _, _, Hkv, _ = paged_qkv.original_page_shape
    PAGE_SIZE = int(paged_qkv.page_size)
    NUM_PAGES = _check_kernel_layout(paged_qkv, Hkv, D)
    MAX_BLOCKS = paged_qkv.block_table.shape[1]
    kq = paged_qkv.k_pages_q.contiguous()
    vq = paged_qkv.v_pages_q.contiguous()
    ks = paged_qkv.k_scales.to(torch.float16).contiguous()
    vs = paged_qkv.v_scales.to(torch.float16).contiguous()
    dev = _lib.require_device(q, kq, vq, ks, vs)
    if kq.dtype != torch.uint8 or vq.dtype != torch.uint8:
        raise TypeError(f"quantized pages must be uint8, got {kq.dtype}, {vq.dtype}")
    q3 = q[:, 0].contiguous()
    bt = _i32(paged_qkv.block_table, dev)
    ln = _i32(lengths_arr, dev)
    out = torch.empty((B, Hq, D), dtype=q.dtype, device=dev)
    ws, ws_bytes = _lib.attention_workspace(dev, B, Hq, Hkv, D, MAX_BLOCKS, PAGE_SIZE)
    _lib.launch("mk_paged_quantized_decode_attention", dev, _lib.ptr(q3), _lib.ptr(kq), _lib.ptr(vq), _lib.ptr(ks),
                _lib.ptr(vs), _lib.ptr(bt), _lib.ptr(ln), _lib.ptr(out), B, Hq, Hkv, D, PAGE_SIZE, MAX_BLOCKS,
                NUM_PAGES, paged_qkv.group_size, paged_qkv.bits, float(scale), _lib.dtype_code(q.dtype),
                _lib.ptr(ws), ws_bytes)
    return out.unsqueeze(1)


def paged_quantized_kv_gqa_decode_attention(q, paged_qkv: PagedQuantizedKVCache, *, scale=None,
                                            backend: str = "reference"):
    """ops/paged_quantized_kv_ops.py:632-661."""
    lengths_arr, B, MAX_S, PAGE_SIZE, MAX_BLOCKS, Hq, Hkv, D = _validate_paged_quantized_decode_inputs(q, paged_qkv)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    backend_name = backend.lower()
    if backend_name == "reference":
        return reference_paged_quantized_kv_gqa_decode_attention(q, paged_qkv, scale=scale)
    if backend_name == "metal_q8":
        if paged_qkv.bits != 8:
            raise ValueError(f"metal_q8 backend requires bits=8, got bits={paged_qkv.bits}")
        if D > _MAX_HEAD_DIM:
            raise ValueError(f"metal_q8 backend supports D <= {_MAX_HEAD_DIM}, got D={D}")
        return _hip_quantized_attention(q, paged_qkv, lengths_arr, scale)
    if backend_name == "metal_q4":
        if paged_qkv.bits != 4:
            raise ValueError(f"metal_q4 backend requires bits=4, got bits={paged_qkv.bits}")
        if D > _MAX_HEAD_DIM:
            raise ValueError(f"metal_q4 backend supports D <= {_MAX_HEAD_DIM}, got D={D}")
        return _hip_quantized_attention(q, paged_qkv, lengths_arr, scale)
    raise ValueError(f"backend must be one of 'reference', 'metal_q8', 'metal_q4', got {backend_name!r}")


# ----------------------------------------------------------------- new-token write


def reference_paged_quantized_kv_update_from_qkv(qkv, paged_qkv: PagedQuantizedKVCache, cos, sin, position, *,
                                                 num_attention_heads, num_key_value_heads, head_dim):
    """Tensor-op statement of the fused write: split + RoPE
    (ops/gqa_ops.py:148-160), per-group symmetric quantization of the rounded
    k_rope / v (ops/paged_quantized_kv_ops.py:146-175), scatter into slot
    (block_table[b, pos//P], pos % P); a later sequence wins a collision.
    Returns (q_rope [B,1,Hq,D], updated copy of the cache)."""
    Hq, Hkv, D = num_attention_heads, num_key_value_heads, head_dim
    q_rope, k_rope, v = _per_sequence_rope(qkv.reshape(qkv.shape[0], 1, -1) if qkv.ndim == 2 else qkv, cos, sin,
                                           Hq, Hkv, D, position)
    B = q_rope.shape[0]
    P = paged_qkv.page_size
    bt = paged_qkv.block_table
    pos = normalize_positions(position, B, bt.shape[1] * P, device=bt.device)
    kq, ks = _quantize_last_dim(k_rope[:, 0].to(torch.float32), paged_qkv.group_size, paged_qkv.bits)
    vq, vs = _quantize_last_dim(v[:, 0].to(torch.float32), paged_qkv.group_size, paged_qkv.bits)
    if paged_qkv.bits == 4:
        kq, vq = _pack_last_dim(kq), _pack_last_dim(vq)
    new = PagedQuantizedKVCache(
        k_pages_q=paged_qkv.k_pages_q.clone(), v_pages_q=paged_qkv.v_pages_q.clone(),
        k_scales=paged_qkv.k_scales.clone(), v_scales=paged_qkv.v_scales.clone(), block_table=bt,
        lengths=paged_qkv.lengths, bits=paged_qkv.bits, page_size=P, group_size=paged_qkv.group_size,
        original_page_shape=paged_qkv.original_page_shape)
    for b in range(B):
        p = int(pos[b])
        page = int(bt[b, p // P])
        if page < 0 or page >= new.k_pages_q.shape[0]:
            continue
        new.k_pages_q[page, p % P] = kq[b].to(new.k_pages_q.device)
        new.v_pages_q[page, p % P] = vq[b].to(new.v_pages_q.device)
        new.k_scales[page, p % P] = ks[b].to(new.k_scales.device)
        new.v_scales[page, p % P] = vs[b].to(new.v_scales.device)
    return q_rope, new


def paged_quantized_kv_update_from_qkv(qkv, paged_qkv: PagedQuantizedKVCache, cos, sin, position, *,
                                       num_attention_heads, num_key_value_heads, head_dim, backend: str = "auto"):
    """Fused qkv split + interleaved RoPE + symmetric quantize + paged write of
    one decode token (one HIP launch, in place).  Returns (q_rope [B,1,Hq,D],
    paged_qkv).  ``backend='reference'`` runs the tensor-op statement instead
    (returning an updated copy)."""
    backend_name = backend.lower()
    if backend_name == "reference":
        return reference_paged_quantized_kv_update_from_qkv(
            qkv, paged_qkv, cos, sin, position, num_attention_heads=num_attention_heads,
            num_key_value_heads=num_key_value_heads, head_dim=head_dim)
    if backend_name not in ("auto", "metal", "metal_q8", "metal_q4"):
        raise ValueError(f"backend must be one of 'reference', 'metal', 'metal_q8', 'metal_q4', 'auto', got {backend_name!r}")
    Hq, Hkv, D = num_attention_heads, num_key_value_heads, head_dim
    validate_gqa_heads(Hq, Hkv)
    paged_qkv.validate()
    if paged_qkv.original_page_shape is None or tuple(paged_qkv.original_page_shape[2:]) != (Hkv, D):
        raise ValueError(f"cache original_page_shape must end with ({Hkv}, {D}), got {paged_qkv.original_page_shape}")
    for t in (paged_qkv.k_pages_q, paged_qkv.v_pages_q, paged_qkv.k_scales, paged_qkv.v_scales):
        if not t.is_contiguous():
            raise ValueError("quantized cache tensors must be contiguous for the in-place update")
    if paged_qkv.k_scales.dtype != torch.float16 or paged_qkv.v_scales.dtype != torch.float16:
        raise TypeError("in-place update needs float16 scales")
    if paged_qkv.k_pages_q.dtype != torch.uint8:
        raise TypeError("quantized pages must be uint8")
    if Hkv * D > 4096:
        raise ValueError(f"fused quantized update supports Hkv*D <= 4096, got {Hkv * D}")
    NUM_PAGES = _check_kernel_layout(paged_qkv, Hkv, D)
    P = int(paged_qkv.page_size)
    dtype = qkv.dtype if qkv.dtype in (torch.float16, torch.bfloat16) else torch.float16
    dev = _lib.require_device(qkv, paged_qkv.k_pages_q, paged_qkv.v_pages_q, paged_qkv.k_scales, paged_qkv.v_scales)
    MAX_BLOCKS = paged_qkv.block_table.shape[1]
    x, c, s, pos, q_out, B = _qkv_rope_update_prep(qkv, paged_qkv.block_table, cos, sin, position, Hq, Hkv, D, P,
                                                   dtype, dev)
    bt = _i32(paged_qkv.block_table, dev)
    _lib.launch("mk_qkv_rope_paged_update_quant", dev, _lib.ptr(x), _lib.ptr(c), _lib.ptr(s), _lib.ptr(pos),
                _lib.ptr(bt), _lib.ptr(paged_qkv.k_pages_q), _lib.ptr(paged_qkv.v_pages_q),
                _lib.ptr(paged_qkv.k_scales), _lib.ptr(paged_qkv.v_scales), _lib.ptr(q_out), B, Hq, Hkv, D, P,
                MAX_BLOCKS, NUM_PAGES, c.shape[0], paged_qkv.group_size, paged_qkv.bits, _lib.dtype_code(dtype))
    return q_out, paged_qkv
