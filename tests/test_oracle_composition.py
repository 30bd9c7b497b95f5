"""Pins the oracle's composition functions -- qkv split + RoPE, the MLP block,
the new-token writes, the decode layer and the stack step -- with closed forms
and invariants that a wiring mistake (swapped operands, a wrong slice offset,
the wrong tensor fed to a stage, an off-by-one length) fails.  No GPU, no torch.
"""

import math

import numpy as np
import pytest

from oracle import llama as ol
from oracle import paged as op
from oracle import quant as oq


# ------------------------------------------------------------ qkv split + RoPE

def test_qkv_split_rope_slices_and_rotation():
    # ops/gqa_ops.py:118-145 packs one token as [Q (Hq*D); K (Hkv*D); V (Hkv*D)].
    # With qkv[b, i] = 1000 b + i every element names its own source index.
    B, Hq, Hkv, D = 2, 4, 2, 8
    W = (Hq + 2 * Hkv) * D
    qkv = (1000.0 * np.arange(B)[:, None] + np.arange(W)[None, :]).astype(np.float32)
    cos = np.ones((4, D // 2), np.float32)
    sin = np.zeros((4, D // 2), np.float32)
    cos[1], sin[1] = 0.0, 1.0  # row 1: 90 degrees on every pair
    q, k, v = op.qkv_split_rope(qkv, cos, sin, [0, 1], Hq, Hkv, D)
    for b in range(B):
        base = 1000.0 * b
        for h in range(Hq):
            src = base + h * D + np.arange(D)
            if b == 0:  # angle 0: the Q slice itself
                assert np.array_equal(q[b, h], src)
            else:  # 90 degrees on interleaved pairs: (e, o) -> (-o, e)
                assert np.array_equal(q[b, h, 0::2], -src[1::2]) and np.array_equal(q[b, h, 1::2], src[0::2])
        for h in range(Hkv):
            ks = base + (Hq + h) * D + np.arange(D)
            vs = base + (Hq + Hkv + h) * D + np.arange(D)
            if b == 0:
                assert np.array_equal(k[b, h], ks)
            else:
                assert np.array_equal(k[b, h, 0::2], -ks[1::2]) and np.array_equal(k[b, h, 1::2], ks[0::2])
            assert np.array_equal(v[b, h], vs)  # v is never rotated


def test_qkv_rope_paged_update_composition():
    # ops/gqa_ops.py:493-547: roped k and raw v land in slot (bt[b, pos//P], pos%P)
    rng = np.random.default_rng(3)
    B, Hq, Hkv, D, P, mb = 3, 4, 2, 8, 4, 3
    qkv = rng.standard_normal((B, (Hq + 2 * Hkv) * D)).astype(np.float16)
    cos, sin = op.rope_tables(16, D, 10000.0)
    NP = B * mb
    K = rng.standard_normal((NP, P, Hkv, D)).astype(np.float16)
    V = rng.standard_normal((NP, P, Hkv, D)).astype(np.float16)
    bt = rng.permutation(NP).astype(np.int32).reshape(B, mb)
    pos = np.array([0, 5, 11])
    q, K2, V2 = op.qkv_rope_paged_update(qkv, cos, sin, pos, bt, K, V, Hq, Hkv, D)
    for b in range(B):
        p = pos[b]
        page, off = bt[b, p // P], p % P
        kraw = qkv[b, Hq * D:(Hq + Hkv) * D].reshape(Hkv, D)
        assert np.array_equal(K2[page, off], op.apply_rope(kraw, cos[p], sin[p]))
        assert np.array_equal(V2[page, off], qkv[b, (Hq + Hkv) * D:].reshape(Hkv, D))
        assert np.array_equal(q[b], op.apply_rope(qkv[b, :Hq * D].reshape(Hq, D), cos[p], sin[p]))
    touched = np.zeros((NP, P), bool)
    touched[[bt[b, pos[b] // P] for b in range(B)], pos % P] = True
    assert np.array_equal(K2[~touched], K[~touched]) and np.array_equal(V2[~touched], V[~touched])


@pytest.mark.parametrize("bits", [8, 4])
def test_quantized_update_composition(bits):
    # angle 0: the written codes/scales are the quantizer's output on the raw
    # k / v slices; 90 degrees: codes of (-o, e) pairs, i.e. the angle-0 codes
    # of the odd element reflected about the zero point, same group scales.
    rng = np.random.default_rng(4 + bits)
    B, Hq, Hkv, D, P, mb, g = 2, 4, 2, 64, 4, 2, 32
    off = 128 if bits == 8 else 8
    qkv = rng.standard_normal((B, (Hq + 2 * Hkv) * D)).astype(np.float16)
    NP = B * mb
    Dq = D if bits == 8 else D // 2
    kq = rng.integers(0, 256, (NP, P, Hkv, Dq)).astype(np.uint8)
    vq = rng.integers(0, 256, (NP, P, Hkv, Dq)).astype(np.uint8)
    ks = rng.standard_normal((NP, P, Hkv, D // g)).astype(np.float16)
    vs = rng.standard_normal((NP, P, Hkv, D // g)).astype(np.float16)
    bt = np.arange(NP, dtype=np.int32).reshape(B, mb)[::-1].copy()
    cos = np.ones((8, D // 2), np.float32)
    sin = np.zeros((8, D // 2), np.float32)
    cos[6], sin[6] = 0.0, 1.0
    pos = np.array([1, 6])
    _, kq2, vq2, ks2, vs2 = op.qkv_rope_paged_update_quant(qkv, cos, sin, pos, bt, kq, vq, ks, vs, Hq, Hkv, D, g,
                                                           bits)
    unpack = (lambda a: a) if bits == 8 else (lambda a: op.unpack_last(a, D))
    kraw = qkv[:, Hq * D:(Hq + Hkv) * D].reshape(B, Hkv, D)
    vraw = qkv[:, (Hq + Hkv) * D:].reshape(B, Hkv, D)
    # sequence 0 at angle 0
    page, o = bt[0, pos[0] // P], pos[0] % P
    kc, kscale = op.quantize_groups(kraw[0], g, bits)
    vc, vscale = op.quantize_groups(vraw[0], g, bits)
    assert np.array_equal(unpack(kq2[page, o]), kc) and np.array_equal(ks2[page, o], kscale)
    assert np.array_equal(unpack(vq2[page, o]), vc) and np.array_equal(vs2[page, o], vscale)
    # sequence 1 at 90 degrees
    page, o = bt[1, pos[1] // P], pos[1] % P
    kc, kscale = op.quantize_groups(kraw[1], g, bits)
    got = unpack(kq2[page, o]).astype(int)
    assert np.array_equal(got[:, 0::2], 2 * off - kc[:, 1::2].astype(int))
    assert np.array_equal(got[:, 1::2], kc[:, 0::2])
    assert np.array_equal(ks2[page, o], kscale)
    vc, vscale = op.quantize_groups(vraw[1], g, bits)
    assert np.array_equal(unpack(vq2[page, o]), vc)
    # every other slot untouched
    keep = np.ones((NP, P), bool)
    keep[[bt[b, pos[b] // P] for b in range(B)], pos % P] = False
    for a, a2 in ((kq, kq2), (vq, vq2), (ks, ks2), (vs, vs2)):
        assert np.array_equal(a[keep].view(np.uint8), a2[keep].view(np.uint8))


# ------------------------------------------------------------ MLP block

def _const_rows(vals, k, g, scale, bits=4):
    """Weight triple whose row i dequantizes to vals[i] * scale everywhere
    (codes zero point + vals[i], zero point 8/128)."""
    zp = 8 if bits == 4 else 128
    codes = np.repeat((zp + np.asarray(vals, int))[:, None], k, axis=1).astype(np.uint8)
    n = len(vals)
    packed = oq.pack_q4(codes) if bits == 4 else codes
    return packed, np.full((n, k // g), scale, np.float32), np.full((n, k // g), float(zp), np.float32)


def _silu(v):
    return v / (1.0 + math.exp(-v))


@pytest.mark.parametrize("bits", [4, 8])
def test_mlp_block_closed_form(bits):
    # ops/mlp_block_ops.py:343-361: z = x + r; n = rmsnorm(z) w; g, u = gate(n),
    # up(n); m = silu(g) u; out = z + down(m).  x = 2, r = 1 (z = 3), w = 0.5:
    # n = 0.5 exactly in fp16.  Constant-code rows make every stage a closed
    # form: gate_i = K n a_i sg, up_i = K n b_i su, down_j = c_j sd sum_i m_i.
    D, I, g = 64, 32, 32
    a = np.tile([1, -2, 3, 0, 2, -1, 1, 2], 4)
    b = np.tile([2, 3, -1, 4, -2, 1, 0, 3], 4)
    c = np.arange(D) % 7 - 3
    sg, su, sd = 1.0 / 32, 1.0 / 16, 1.0 / 64
    x = np.full((1, D), 2.0, np.float16)
    r = np.full((1, D), 1.0, np.float16)
    w = np.full(D, 0.5, np.float16)
    gate, up, down = _const_rows(a, D, g, sg, bits), _const_rows(b, D, g, su, bits), _const_rows(c, I, g, sd, bits)
    out, mid = oq.mlp_block(x, r, w, gate, up, down, bits=bits, group_size=g, intermediates=True)

    def closed(feed, gi, ui, res, down_in="m"):
        gv = np.float16(D * feed) * gi * sg  # exact: small integers times powers of two
        uv = np.float16(D * feed) * ui * su
        m = np.array([np.float16(_silu(float(p)) * float(q)) for p, q in zip(gv, uv)], np.float64)
        src = {"m": m, "g": gv.astype(np.float64), "u": uv.astype(np.float64)}[down_in]
        d = (c * sd * src.sum()).astype(np.float16)
        return (res + d.astype(np.float32)).astype(np.float16), gv, uv, m, d

    want, gv, uv, m, d = closed(0.5, a, b, 3.0)
    assert np.array_equal(mid["z"], np.full((1, D), 3.0, np.float16))
    assert np.array_equal(mid["normed"], np.full((1, D), 0.5, np.float16))
    assert np.array_equal(mid["gate"][0], gv.astype(np.float16)) and np.array_equal(mid["up"][0], uv.astype(np.float16))
    assert np.allclose(mid["mlp"][0].astype(np.float64), m, rtol=1e-3, atol=1e-3)
    assert np.allclose(mid["down"][0].astype(np.float64), d.astype(np.float64), rtol=2e-3, atol=2e-3)
    assert np.allclose(out[0].astype(np.float64), want.astype(np.float64), rtol=2e-3, atol=2e-3)
    # each plausible wiring mistake moves the output far outside that tolerance
    for wrong in (closed(0.5, b * su / sg, a * sg / su, 3.0)[0],  # gate and up swapped
                  closed(3.0, a, b, 3.0)[0],  # z fed to gate/up instead of the normed row
                  closed(0.5, a, b, 2.0)[0],  # residual taken from x instead of z
                  closed(0.5, a, b, 3.0, "g")[0], closed(0.5, a, b, 3.0, "u")[0]):  # down fed gate / up
        assert not np.allclose(out[0].astype(np.float64), wrong.astype(np.float64), rtol=2e-3, atol=2e-3)


# ------------------------------------------------------------ decode layer

def _layer(seed, H=64, Hq=4, Hkv=2, D=16, I=128, g=32, scale=0.05):
    rng = np.random.default_rng(seed)

    def qw(n, k):
        w = (rng.standard_normal((n, k)) * scale).astype(np.float32)
        packed, s = oq.quantize_weight_groupwise(w, 4, g)
        return packed, s, np.full(s.shape, 8.0, np.float32)

    return {"qkv": qw((Hq + 2 * Hkv) * D, H), "o": qw(H, Hq * D), "gate": qw(I, H), "up": qw(I, H),
            "down": qw(H, I), "ln1": (1 + 0.1 * rng.standard_normal(H)).astype(np.float16),
            "ln2": (1 + 0.1 * rng.standard_normal(H)).astype(np.float16)}


def _layer_inputs(seed, B=2, H=64, Hkv=2, D=16, P=4, mb=4):
    rng = np.random.default_rng(seed)
    NP = B * mb
    K = rng.standard_normal((NP, P, Hkv, D)).astype(np.float16)
    V = rng.standard_normal((NP, P, Hkv, D)).astype(np.float16)
    bt = rng.permutation(NP).astype(np.int32).reshape(B, mb)
    x = rng.standard_normal((B, H)).astype(np.float16)
    return x, K, V, bt


def test_decode_layer_at_position_zero_closed_form():
    # ops/llama_layer_ops.py:234-428: at position 0 the new token is the only
    # key (lengths = pos + 1 = 1), so every query head h returns v of kv head
    # h // (Hq/Hkv) whatever q, k and the cache hold; then o-proj, residual,
    # MLP block on h = x + o(attn) with a zero residual.
    Hq, Hkv, D, H = 4, 2, 16, 64
    w = _layer(1)
    x, K, V, bt = _layer_inputs(2)
    cos, sin = op.rope_tables(32, D, 500000.0)
    pos = [0, 0]
    out, _, _ = ol.layer_decode_step(x, w, K, V, bt, cos, sin, pos, Hq, Hkv, D, group_size=32)
    qkv = oq.q4_matvec(oq.rms_norm(x, w["ln1"]), *w["qkv"], group_size=32)
    v = qkv[:, (Hq + Hkv) * D:].reshape(2, Hkv, D)
    attn = np.repeat(v, Hq // Hkv, axis=1).reshape(2, Hq * D)
    h = oq.residual_add(x, oq.q4_matvec(attn, *w["o"], group_size=32))
    want = oq.mlp_block(h, np.zeros_like(h), w["ln2"], w["gate"], w["up"], w["down"], bits=4, group_size=32)
    assert np.array_equal(out, want)
    # independent of the q/k rows of the projection and of the cache contents
    w2 = dict(w)
    p2, s2, z2 = (a.copy() for a in w["qkv"])
    p2[: (Hq + Hkv) * D] = np.random.default_rng(9).integers(0, 256, p2[: (Hq + Hkv) * D].shape).astype(np.uint8)
    w2["qkv"] = (p2, s2, z2)
    out2, _, _ = ol.layer_decode_step(x, w2, K * 0 + 7, V[::-1].copy(), bt, cos, sin, pos, Hq, Hkv, D, group_size=32)
    assert np.array_equal(out2, out)
    # a wrong GQA head map (h % Hkv instead of h // group) is caught
    wrong = np.tile(v, (1, Hq // Hkv, 1)).reshape(2, Hq * D)
    hw = oq.residual_add(x, oq.q4_matvec(wrong, *w["o"], group_size=32))
    assert not np.array_equal(oq.mlp_block(hw, np.zeros_like(hw), w["ln2"], w["gate"], w["up"], w["down"],
                                           bits=4, group_size=32), out)


def test_decode_layer_invariants():
    Hq, Hkv, D, P = 4, 2, 16, 4
    w = _layer(3)
    x, K, V, bt = _layer_inputs(4)
    cos, sin = op.rope_tables(32, D, 500000.0)
    pos = np.array([6, 9])
    out, K2, V2 = ol.layer_decode_step(x, w, K, V, bt, cos, sin, pos, Hq, Hkv, D, group_size=32)
    # garbage past each sequence's new position changes nothing (lengths = pos + 1)
    Kg, Vg = K.copy(), V.copy()
    rng = np.random.default_rng(5)
    for b in range(2):
        for j in range(pos[b] + 1, bt.shape[1] * P):
            Kg[bt[b, j // P], j % P] = rng.standard_normal((Hkv, D)) * 50
            Vg[bt[b, j // P], j % P] = rng.standard_normal((Hkv, D)) * 50
    outg, _, _ = ol.layer_decode_step(x, w, Kg, Vg, bt, cos, sin, pos, Hq, Hkv, D, group_size=32)
    assert np.array_equal(outg, out)
    # ...but the positions before it are read: changing one changes the output
    Kc = K.copy()
    Kc[bt[0, 0], 1] += 3.0
    outc, _, _ = ol.layer_decode_step(x, w, Kc, V, bt, cos, sin, pos, Hq, Hkv, D, group_size=32)
    assert not np.array_equal(outc[0], out[0]) and np.array_equal(outc[1], out[1])
    # permuting the physical pages (and the table with them) is bit-identical
    perm = np.random.default_rng(6).permutation(K.shape[0])
    inv = np.argsort(perm)
    outp, K2p, _ = ol.layer_decode_step(x, w, K[perm], V[perm], inv[bt].astype(np.int32), cos, sin, pos, Hq, Hkv, D,
                                        group_size=32)
    assert np.array_equal(outp, out) and np.array_equal(K2p[inv], K2)
    # with a non-trivial cache, position 1 differs from position 0
    o0, _, _ = ol.layer_decode_step(x, w, K, V, bt, cos, sin, [0, 0], Hq, Hkv, D, group_size=32)
    o1, _, _ = ol.layer_decode_step(x, w, K, V, bt, cos, sin, [1, 1], Hq, Hkv, D, group_size=32)
    assert not np.array_equal(o0, o1)


# ------------------------------------------------------------ stack step

def test_stack_step_zero_layer_is_norm_head_argmax():
    # ops/llama_stack_ops.py:352-411 + models/sampling.py:120-124: a layer whose
    # projections dequantize to 0 passes x through, so the logits are
    # head(rmsnorm(embedding[token])) and the next tokens their argmax.
    rng = np.random.default_rng(11)
    H, Hq, Hkv, D, I, g, P, mb, vocab, B = 64, 4, 2, 16, 128, 32, 4, 4, 50, 3
    zero_pt = lambda n, k: (oq.pack_q4(np.full((n, k), 8, np.uint8)), np.ones((n, k // g), np.float32),
                            np.full((n, k // g), 8.0, np.float32))
    layer = {"qkv": zero_pt((Hq + 2 * Hkv) * D, H), "o": zero_pt(H, Hq * D), "gate": zero_pt(I, H),
             "up": zero_pt(I, H), "down": zero_pt(H, I), "ln1": np.ones(H, np.float16), "ln2": np.ones(H, np.float16)}
    emb = rng.standard_normal((vocab, H)).astype(np.float16)
    hw = (rng.standard_normal((vocab, H)) * 0.1).astype(np.float32)
    packed, s = oq.quantize_weight_groupwise(hw, 4, g)
    head = (packed, s, np.full(s.shape, 8.0, np.float32))
    fnorm = (1 + 0.1 * rng.standard_normal(H)).astype(np.float16)
    weights = {"embedding": emb, "layers": [layer, layer], "final_norm": fnorm, "lm_head": head}
    NP = B * mb
    caches = [(rng.standard_normal((NP, P, Hkv, D)).astype(np.float16),
               rng.standard_normal((NP, P, Hkv, D)).astype(np.float16)) for _ in range(2)]
    bt = np.arange(NP, dtype=np.int32).reshape(B, mb)
    cos, sin = op.rope_tables(16, D, 500000.0)
    tokens = np.array([7, 0, 48])
    nxt, logits, _ = ol.stack_decode_step(tokens, weights, caches, bt, cos, sin, [2, 3, 4], Hq, Hkv, D, group_size=g)
    # float64 closed form over the dequantized head (fp16-rounded weights)
    fh = oq.rms_norm(emb[tokens], fnorm).astype(np.float64)
    Wd = oq.dequant_q4(packed, s, np.full(s.shape, 8.0), g).astype(np.float64)
    ref = fh @ Wd.T
    assert np.allclose(logits, ref, rtol=2e-3, atol=2e-3)
    assert np.array_equal(nxt, np.argmax(logits, axis=-1))
    assert np.array_equal(nxt, np.argmax(ref, axis=-1))
    # the embedding row is the token's: shifting tokens changes the logits
    _, l2, _ = ol.stack_decode_step(tokens + 1, weights, caches, bt, cos, sin, [2, 3, 4], Hq, Hkv, D, group_size=g)
    assert not np.allclose(l2, logits)
