"""Writes the golden fixtures of this directory from the numpy oracle.

The reference ships no stored expected values (its tests draw MLX random
inputs and compare against its own reference path), so these fixtures are
the oracle's outputs on explicitly seeded small inputs.  They pin the oracle
against regressions (tests/test_golden.py re-derives every output on the
CPU) and give the GPU tests fixed inputs/outputs that travel as data.

Run from the repository root:  python tests/golden/make_golden.py
Every case is fully determined by its seed; rerunning rewrites identical
inputs (the float outputs can differ in the last bit only if numpy's BLAS
changes its summation order, which the CPU test tolerates for matmuls).
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import paged as op  # noqa: E402
from oracle import quant as oq  # noqa: E402


def _save(name: str, **arrays):
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **arrays)


def quant_cases():
    rng = np.random.default_rng(1001)
    # a1/a2: pack/unpack incl. odd K
    codes = rng.integers(0, 16, size=(8, 33), dtype=np.uint8)
    _save("q4_pack", codes=codes, packed=oq.pack_q4(codes))

    # a4/a5: dequant with affine zeros (K not a multiple of the group)
    c4 = rng.integers(0, 16, size=(16, 96), dtype=np.uint8)
    p4 = oq.pack_q4(c4)
    s = (rng.random((16, 3)) * 0.1 + 0.001).astype(np.float32)
    z = rng.integers(0, 16, size=(16, 3)).astype(np.float32)
    c8 = rng.integers(0, 256, size=(16, 80), dtype=np.uint8)
    s8 = (rng.random((16, 3)) * 0.01).astype(np.float32)
    z8 = rng.integers(100, 156, size=(16, 3)).astype(np.float32)
    _save("dequant", q4_packed=p4, q4_scales=s, q4_zeros=z, q4_out=oq.dequant_q4(p4, s, z, 32),
          q8_codes=c8, q8_scales=s8, q8_zeros=z8, q8_out=oq.dequant_q8(c8, s8, z8, 32))

    # a7/a9: Llama-slice matvec (K = 4096, g = 64, quantized by a35), M = 1 and 4
    for bits in (4, 8):
        W = (rng.standard_normal((32, 4096)) * 0.02).astype(np.float32)
        w, sc = oq.quantize_weight_groupwise(W, bits, 64)
        sc16 = sc.astype(np.float16)
        zp = np.full(sc.shape, 8.0 if bits == 4 else 128.0, np.float16)
        x = rng.standard_normal((4, 4096)).astype(np.float16)
        mv = oq.q4_matvec if bits == 4 else oq.q8_matvec
        y = mv(x, w, sc16.astype(np.float32), zp.astype(np.float32), 64)
        # the quantizer is per row: its first 8 rows pin a35 without storing all of W
        _save(f"q{bits}_matvec_llama_slice", weight=w, scales=sc16, zeros=zp, x=x, y=y, W_fp32_rows=W[:8],
              scales_fp32_rows=sc[:8])

    # a16: MLP block (hidden 256, intermediate 512, g 64, q4)
    D, I, g = 256, 512, 64
    mats = {}
    for nm, (n, k) in (("gate", (I, D)), ("up", (I, D)), ("down", (D, I))):
        w, sc = oq.quantize_weight_groupwise((rng.standard_normal((n, k)) * 0.02).astype(np.float32), 4, g)
        mats[nm] = (w, sc.astype(np.float16), np.full(sc.shape, 8.0, np.float16))
    x = rng.standard_normal((2, D)).astype(np.float16)
    r = rng.standard_normal((2, D)).astype(np.float16)
    nw = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float16)
    trip = lambda m: (m[0], m[1].astype(np.float32), m[2].astype(np.float32))  # noqa: E731
    out, inter = oq.mlp_block(x, r, nw, trip(mats["gate"]), trip(mats["up"]), trip(mats["down"]), bits=4,
                              group_size=g, intermediates=True)
    arrays = {"x": x, "residual": r, "norm_w": nw, "out": out}
    for nm, (w, sc, zp) in mats.items():
        arrays.update({f"{nm}_w": w, f"{nm}_s": sc, f"{nm}_z": zp})
    arrays.update({f"i_{k}": v for k, v in inter.items()})
    _save("q4_mlp_block", **arrays)


def paged_cases():
    rng = np.random.default_rng(2002)
    B, Hq, Hkv, D, P, mb = 3, 8, 2, 64, 16, 4
    NP = B * mb
    Kp = rng.standard_normal((NP, P, Hkv, D)).astype(np.float16)
    Vp = rng.standard_normal((NP, P, Hkv, D)).astype(np.float16)
    bt = rng.permutation(NP).astype(np.int32).reshape(B, mb)
    bt_holes = bt.copy()
    bt_holes[1, 3] = -1  # an unmapped block beyond sequence 1's length
    lengths = np.array([1, 37, 64], np.int32)
    pos = np.array([0, 17, 63], np.int32)
    page, off = op.block_table_lookup(bt, pos, P)
    kn = rng.standard_normal((B, Hkv, D)).astype(np.float16)
    vn = rng.standard_normal((B, Hkv, D)).astype(np.float16)
    K2, V2 = op.paged_kv_update(Kp, Vp, kn, vn, bt, pos)
    q = rng.standard_normal((B, Hq, D)).astype(np.float16)
    attn = op.paged_attention(q, Kp, Vp, bt, lengths)
    attn_holes = op.paged_attention(q, Kp, Vp, bt_holes, np.array([1, 37, 20], np.int32))
    _save("paged_gqa", K_pages=Kp, V_pages=Vp, block_table=bt, block_table_holes=bt_holes, lengths=lengths,
          positions=pos, page=page, offset=off, k_new=kn, v_new=vn, K_updated=K2, V_updated=V2, q=q,
          attention=attn, attention_holes=attn_holes)

    # a25: qkv split + RoPE (theta 500000) + paged update
    cos, sin = op.rope_tables(64, D, 500000.0)
    qkv = rng.standard_normal((B, (Hq + 2 * Hkv) * D)).astype(np.float16)
    q_r, K3, V3 = op.qkv_rope_paged_update(qkv, cos, sin, pos, bt, Kp, Vp, Hq, Hkv, D)
    _save("qkv_rope_update", qkv=qkv, cos=cos, sin=sin, q_rope=q_r, K_updated=K3, V_updated=V3)

    # a29/a30/a33/a34: quantized KV (q8 and q4, g = 32)
    for bits in (8, 4):
        g = 32
        kq, vq, ks, vs = op.quantize_pages(Kp, Vp, g, bits)
        att = op.quantized_paged_attention(q, kq, vq, ks, vs, bt, lengths, g, bits)
        qr, kq2, vq2, ks2, vs2 = op.qkv_rope_paged_update_quant(qkv, cos, sin, pos, bt, kq, vq, ks, vs, Hq, Hkv, D,
                                                                g, bits)
        _save(f"paged_q{bits}", k_q=kq, v_q=vq, k_s=ks, v_s=vs, attention=att, q_rope=qr, k_q_updated=kq2,
              v_q_updated=vq2, k_s_updated=ks2, v_s_updated=vs2)


if __name__ == "__main__":
    quant_cases()
    paged_cases()
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f"{f:32s} {os.path.getsize(os.path.join(HERE, f)):8d} B")
