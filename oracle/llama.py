"""Oracle: one quantized Llama-like decode layer and stack step on paged
fp16 KV caches, composed from the pinned pieces of oracle.quant and
oracle.paged.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
"""

from __future__ import annotations

import math

import numpy as np

from . import paged as op
from . import quant as oq


def layer_decode_step(x, w, K, V, bt, cos, sin, pos, Hq, Hkv, D, bits=4, group_size=32, eps=1e-5):
    """ops/llama_layer_ops.py:234-428 with the paged decode block of
    ops/quantized_decode_block_ops.py:446-552.  x [B, hidden] fp16; w a dict
    of (codes, scales, zeros) triples 'qkv', 'o', 'gate', 'up', 'down' and
    norm weights 'ln1', 'ln2'; K, V [NP, P, Hkv, D] fp16; pos [B] ints.
    Returns (out [B, hidden] fp16, K', V')."""
    mv = oq.q4_matvec if bits == 4 else oq.q8_matvec
    B = x.shape[0]
    xn = oq.rms_norm(x, w["ln1"], eps)
    qkv = mv(xn, *w["qkv"], group_size=group_size)
    q, K2, V2 = op.qkv_rope_paged_update(qkv, cos, sin, pos, bt, K, V, Hq, Hkv, D)
    attn = op.paged_attention(q, K2, V2, bt, np.asarray(pos) + 1, 1.0 / math.sqrt(D)).astype(np.float16)
    proj = mv(attn.reshape(B, Hq * D), *w["o"], group_size=group_size)
    h = oq.residual_add(x, proj)
    out = oq.mlp_block(h, np.zeros_like(h), w["ln2"], w["gate"], w["up"], w["down"], bits=bits,
                       group_size=group_size, eps=eps)
    return out, K2, V2


def stack_decode_step(tokens, weights, caches, bt, cos, sin, pos, Hq, Hkv, D, bits=4, group_size=32, eps=1e-5):
    """ops/llama_stack_ops.py:352-411 + models/sampling.py:120-124 on paged
    caches: embedding gather, every layer, final RMSNorm, q4/q8 head, argmax.
    Returns (next tokens [B], logits fp32 [B, vocab], caches')."""
    mv = oq.q4_matvec if bits == 4 else oq.q8_matvec
    x = weights["embedding"][np.asarray(tokens)]
    new = []
    for lw, (K, V) in zip(weights["layers"], caches):
        x, K, V = layer_decode_step(x, lw, K, V, bt, cos, sin, pos, Hq, Hkv, D, bits, group_size, eps)
        new.append((K, V))
    fh = oq.rms_norm(x, weights["final_norm"], eps)
    logits = mv(fh, *weights["lm_head"], group_size=group_size).astype(np.float32)
    return np.argmax(logits, axis=-1), logits, new
