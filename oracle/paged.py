"""Oracle: paged KV plumbing, RoPE, symmetric KV quantizers and paged decode
attention (fp16/bf16 and q8/q4 caches).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
"""

from __future__ import annotations

import math

import numpy as np

from .quant import pack_q4, unpack_q4


def identity_block_table(B: int, max_s: int, P: int) -> np.ndarray:
    """ops/paged_kv_ops.py:99-105."""
    mb = math.ceil(max_s / P)
    return (np.arange(B, dtype=np.int32)[:, None] * mb + np.arange(mb, dtype=np.int32)[None, :]).astype(np.int32)


def block_table_lookup(bt: np.ndarray, pos: np.ndarray, P: int):
    """ops/paged_kv_ops.py:138-152."""
    pos = np.asarray(pos, dtype=np.int64)
    return bt[np.arange(bt.shape[0]), pos // P].astype(np.int32), (pos % P).astype(np.int32)


def paged_kv_update(Kp, Vp, k_new, v_new, bt, pos):
    """ops/paged_kv_ops.py:185-213: functional copy with slot
    (bt[b, pos//P], pos%P) <- token b; a later b wins a collision."""
    Kp, Vp = Kp.copy(), Vp.copy()
    P = Kp.shape[1]
    page, off = block_table_lookup(bt, pos, P)
    for b in range(bt.shape[0]):
        Kp[page[b], off[b]] = k_new[b]
        Vp[page[b], off[b]] = v_new[b]
    return Kp, Vp


def gather(pages: np.ndarray, bt: np.ndarray, max_s: int):
    """Positions j < max_s of every sequence through the block table
    (ops/gqa_ops.py:325-340); invalid page ids gather page 0 and are
    reported in the mask."""
    P = pages.shape[1]
    j = np.arange(max_s)
    page = bt.astype(np.int64)[:, j // P]
    valid = (page >= 0) & (page < pages.shape[0])
    page = np.where(valid, page, 0)
    return pages[page, np.broadcast_to(j % P, page.shape)], valid


def attention(q, K, V, lengths, valid, scale):
    """Per-sequence softmax attention in float64, head h on kv head
    h // (Hq/Hkv) (ops/gqa_ops.py:278-304 with per-sequence lengths;
    the F4 fix of ops/paged_quantized_kv_ops.py:469-515).
    q [B,Hq,D]; K/V [B,S,Hkv,D]; returns float64 [B,Hq,D]; no position -> 0."""
    B, Hq, D = q.shape
    Hkv = K.shape[2]
    g = Hq // Hkv
    out = np.zeros((B, Hq, D), dtype=np.float64)
    for b in range(B):
        n = int(min(lengths[b], K.shape[1]))
        keep = np.nonzero(valid[b, :n])[0]
        if keep.size == 0:
            continue
        for kh in range(Hkv):  # the g query heads of kv head kh together
            k = K[b, keep, kh].astype(np.float64)
            v = V[b, keep, kh].astype(np.float64)
            s = (q[b, kh * g:(kh + 1) * g].astype(np.float64) @ k.T) * scale
            p = np.exp(s - s.max(axis=1, keepdims=True))
            out[b, kh * g:(kh + 1) * g] = (p / p.sum(axis=1, keepdims=True)) @ v
    return out


def paged_attention(q, Kp, Vp, bt, lengths, scale=None):
    """Paged GQA decode: ops/gqa_ops.py:307-342 (fp16/bf16 cache)."""
    D = q.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    max_s = bt.shape[1] * Kp.shape[1]
    lengths = np.minimum(np.asarray(lengths), max_s)
    K, valid = gather(Kp, bt, max_s)
    V, _ = gather(Vp, bt, max_s)
    return attention(q, K, V, lengths, valid, scale)


def verify_row_lengths(lengths, W: int) -> np.ndarray:
    """[B, W] positions visible to each query row of a W-row verify pass:
    draft token w sits at position lengths[b] - W + w and its staged decode
    step attends over the positions up to and including its own
    (ops/speculative_verify_ops.py:228-262: step i runs llama_stack_decode_step
    at staged position `position + i` after the steps before it wrote their
    K/V), so row w sees lengths[b] - (W - 1 - w) positions (none below 0)."""
    lengths = np.asarray(lengths, dtype=np.int64)
    return np.maximum(lengths[:, None] - (W - 1 - np.arange(W))[None, :], 0)


def paged_verify_attention(q, Kp, Vp, bt, lengths, scale=None):
    """The attention of the W staged decode steps of parallel_verify_tokens
    (ops/speculative_verify_ops.py:161-296) in one call: q [B, W, Hq, D] ->
    float64 [B, W, Hq, D], row w the single-token paged attention
    (ops/gqa_ops.py:307-342) over verify_row_lengths(lengths, W)[:, w]
    positions.  lengths[b] counts the context and all W new positions."""
    W = q.shape[1]
    rows = verify_row_lengths(lengths, W)
    out = np.empty(q.shape, dtype=np.float64)
    for w in range(W):
        out[:, w] = paged_attention(q[:, w], Kp, Vp, bt, rows[:, w], scale)
    return out


def quantized_paged_verify_attention(q, kq, vq, ks, vs, bt, lengths, group_size, bits, scale=None):
    """paged_verify_attention over q8/q4 pages (dequantized as
    quantized_paged_attention does)."""
    D = q.shape[-1]
    K, V = dequantize_pages(kq, vq, ks, vs, group_size, bits, D)
    return paged_verify_attention(q, K, V, bt, lengths, scale)


# ----------------------------------------------------------------- RoPE


def rope_tables(seq_len: int, D: int, theta: float):
    """models/llama_config.py:107-124 / ops/llama_stack_ops.py:97-103."""
    pos = np.arange(seq_len, dtype=np.float32)
    inv = (1.0 / (np.float32(theta) ** (np.arange(0, D, 2, dtype=np.float32) / np.float32(D)))).astype(np.float32)
    f = pos[:, None] * inv[None, :]
    return np.cos(f).astype(np.float32), np.sin(f).astype(np.float32)


def apply_rope(x: np.ndarray, c: np.ndarray, s: np.ndarray) -> np.ndarray:
    """ops/rope_ops.py:61-75: x [..., D] with c/s [..., D/2] broadcastable;
    ye = xe*c - xo*s, yo = xe*s + xo*c, each product rounded to fp32 before
    the add (numpy evaluates them separately), result in x's dtype."""
    xe = x[..., 0::2].astype(np.float32)
    xo = x[..., 1::2].astype(np.float32)
    ye = xe * c - xo * s
    yo = xe * s + xo * c
    return np.stack([ye, yo], axis=-1).reshape(x.shape).astype(x.dtype)


def qkv_split_rope(qkv: np.ndarray, cos, sin, pos, Hq: int, Hkv: int, D: int):
    """ops/gqa_ops.py:118-160 for one decode token per sequence at
    per-sequence positions.  qkv [B, (Hq+2Hkv)*D] -> q, k [B,H,D] roped, v."""
    B = qkv.shape[0]
    q = qkv[:, :Hq * D].reshape(B, Hq, D)
    k = qkv[:, Hq * D:(Hq + Hkv) * D].reshape(B, Hkv, D)
    v = qkv[:, (Hq + Hkv) * D:].reshape(B, Hkv, D)
    c = cos[np.asarray(pos)][:, None, :]
    s = sin[np.asarray(pos)][:, None, :]
    return apply_rope(q, c, s), apply_rope(k, c, s), v


# ----------------------------------------------------------------- quantized KV


def quantize_groups(v: np.ndarray, group_size: int, bits: int):
    """ops/paged_quantized_kv_ops.py:146-175 along the last dim:
    s = max(max|v|, 1e-8) / (127|7) in fp32, codes clip(rint(v / s)) + 128|8,
    the fp16 scale rounded after use.  Returns (codes [..., D], scales fp16)."""
    qmax, off = (127.0, 128) if bits == 8 else (7.0, 8)
    v = v.astype(np.float32)
    D = v.shape[-1]
    G = -(-D // group_size)
    codes = np.zeros(v.shape, dtype=np.uint8)
    scales = np.zeros(v.shape[:-1] + (G,), dtype=np.float16)
    for g in range(G):
        blk = v[..., g * group_size:min((g + 1) * group_size, D)]
        amax = np.maximum(np.abs(blk).max(axis=-1, keepdims=True), np.float32(1e-8))
        s = (amax / np.float32(qmax)).astype(np.float32)
        q = np.clip(np.rint(blk / s), -qmax, qmax) + off
        codes[..., g * group_size:g * group_size + blk.shape[-1]] = q.astype(np.uint8)
        scales[..., g] = s[..., 0].astype(np.float16)
    return codes, scales


def pack_last(codes: np.ndarray) -> np.ndarray:
    shp = codes.shape
    return pack_q4(codes.reshape(-1, shp[-1])).reshape(shp[:-1] + (-(-shp[-1] // 2),))


def unpack_last(packed: np.ndarray, D: int) -> np.ndarray:
    shp = packed.shape
    return unpack_q4(packed.reshape(-1, shp[-1]), D).reshape(shp[:-1] + (D,))


def dequantize(codes_unpacked: np.ndarray, scales: np.ndarray, group_size: int, bits: int) -> np.ndarray:
    """ops/paged_quantized_kv_ops.py:156-186 and :295-341: (code - 128|8) *
    |s| in fp32, rounded to fp16."""
    off = 128.0 if bits == 8 else 8.0
    D = codes_unpacked.shape[-1]
    s = np.repeat(np.abs(scales.astype(np.float32)), group_size, axis=-1)[..., :D]
    return ((codes_unpacked.astype(np.float32) - np.float32(off)) * s).astype(np.float16)


def quantize_pages(Kp, Vp, group_size: int, bits: int):
    """ops/paged_quantized_kv_ops.py:194-292 -> (kq, vq, ks, vs), q4 packed."""
    kq, ks = quantize_groups(Kp, group_size, bits)
    vq, vs = quantize_groups(Vp, group_size, bits)
    if bits == 4:
        kq, vq = pack_last(kq), pack_last(vq)
    return kq, vq, ks, vs


def dequantize_pages(kq, vq, ks, vs, group_size: int, bits: int, D: int):
    if bits == 4:
        kq, vq = unpack_last(kq, D), unpack_last(vq, D)
    return dequantize(kq, ks, group_size, bits), dequantize(vq, vs, group_size, bits)


def quantized_paged_attention(q, kq, vq, ks, vs, bt, lengths, group_size, bits, scale=None):
    """ops/paged_quantized_kv_ops.py:469-515 with per-sequence lengths:
    dequantize to fp16, gather valid positions (page id < 0 skipped,
    kernels/q8_paged_gqa_decode_attention.metal:52-57), softmax attention."""
    D = q.shape[-1]
    K, V = dequantize_pages(kq, vq, ks, vs, group_size, bits, D)
    return paged_attention(q, K, V, bt, lengths, scale)


def qkv_rope_paged_update(qkv, cos, sin, pos, bt, Kp, Vp, Hq, Hkv, D):
    """Composition run by ops/gqa_ops.py:493-547: split + RoPE, then the
    paged scatter of (k_rope, v).  Returns (q_rope [B,Hq,D], K', V')."""
    q, k, v = qkv_split_rope(qkv, cos, sin, pos, Hq, Hkv, D)
    K2, V2 = paged_kv_update(Kp, Vp, k, v, bt, pos)
    return q, K2, V2


def qkv_rope_paged_update_quant(qkv, cos, sin, pos, bt, kq, vq, ks, vs, Hq, Hkv, D, group_size, bits):
    """Quantized new-token write (no reference kernel exists):
    split + RoPE, a29 quantization of the rounded k_rope / v, scatter of
    codes and fp16 scales into (bt[b, pos//P], pos%P); later b wins."""
    q, k, v = qkv_split_rope(qkv, cos, sin, pos, Hq, Hkv, D)
    kc, ksn = quantize_groups(k, group_size, bits)
    vc, vsn = quantize_groups(v, group_size, bits)
    if bits == 4:
        kc, vc = pack_last(kc), pack_last(vc)
    kq, vq, ks, vs = kq.copy(), vq.copy(), ks.copy(), vs.copy()
    P = kq.shape[1]
    page, off = block_table_lookup(bt, pos, P)
    for b in range(qkv.shape[0]):
        kq[page[b], off[b]] = kc[b]
        vq[page[b], off[b]] = vc[b]
        ks[page[b], off[b]] = ksn[b]
        vs[page[b], off[b]] = vsn[b]
    return q, kq, vq, ks, vs


# ----------------------------------------------------------------- contiguous caches


def contiguous_update(K, V, k_new, v_new, pos):
    """ops/kv_cache_ops.py:93-107: functional copy of K/V [B, MAX_S, H, D]
    with row pos[b] of sequence b replaced by k_new[b] / v_new[b]."""
    K, V = K.copy(), V.copy()
    for b, p in enumerate(np.broadcast_to(np.asarray(pos), (K.shape[0],))):
        K[b, p] = k_new[b]
        V[b, p] = v_new[b]
    return K, V


def contiguous_attention(q, K, V, lengths, scale=None):
    """Decode attention over a contiguous cache K/V [B, MAX_S, Hkv, D] at
    positions j < min(lengths[b], MAX_S): ops/decode_ops.py:93-123 (MHA),
    ops/gqa_ops.py:278-304 (GQA) and ops/quantized_kv_cache_ops.py:377-406
    (after dequantization).  float64 [B, Hq, D]."""
    D = q.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    lengths = np.minimum(np.broadcast_to(np.asarray(lengths), (q.shape[0],)), K.shape[1])
    return attention(q, K, V, lengths, np.ones(K.shape[:2], bool), scale)


def quantize_contiguous(K, V, group_size: int, bits: int, lengths=None):
    """ops/quantized_kv_cache_ops.py:173-277: the quantizer of :131-170 on
    positions j < lengths[b] (all when None); the other positions keep zero
    codes and zero scales.  Returns (kq, vq, ks, vs), q4 codes packed."""
    kq, ks = quantize_groups(K, group_size, bits)
    vq, vs = quantize_groups(V, group_size, bits)
    if lengths is not None:
        keep = np.arange(K.shape[1])[None, :] < np.asarray(lengths).reshape(-1, 1)
        kq[~keep], vq[~keep] = 0, 0
        ks[~keep], vs[~keep] = 0, 0
    if bits == 4:
        kq, vq = pack_last(kq), pack_last(vq)
    return kq, vq, ks, vs
