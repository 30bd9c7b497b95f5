"""Quantized paged decode layer and stack (HIP) against the oracle's
composition of the same reference ops."""

import numpy as np
import pytest
import torch

from mk import llama_layer_ops as ll
from mk import llama_stack_ops as ls
from oracle import llama as ol
from oracle import paged as op
from oracle import quant as oq
from tests._data import assert_close

pytestmark = pytest.mark.gpu


def _cfg(layers=2, vocab=512):
    return ll.LlamaLikeConfig(hidden_size=256, intermediate_size=512, num_attention_heads=4, num_key_value_heads=2,
                              head_dim=64, num_hidden_layers=layers, max_position_embeddings=512,
                              rope_theta=500000.0, vocab_size=vocab).validate()


def _linear(rng, out_dim, in_dim, bits, g):
    w = (rng.standard_normal((out_dim, in_dim)) * 0.02).astype(np.float32)
    codes, s = oq.quantize_weight_groupwise(w, bits, g)
    s = s.astype(np.float16).astype(np.float32)  # the fp16 scales the kernels read
    z = np.full(s.shape, 8.0 if bits == 4 else 128.0, np.float32)
    return codes, s, z


def _np_layer(rng, cfg, bits, g):
    H, I = cfg.hidden_size, cfg.intermediate_size
    return {"qkv": _linear(rng, cfg.qkv_output_dim(), H, bits, g), "o": _linear(rng, H, H, bits, g),
            "gate": _linear(rng, I, H, bits, g), "up": _linear(rng, I, H, bits, g),
            "down": _linear(rng, H, I, bits, g),
            "ln1": (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float16),
            "ln2": (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float16)}


def _t_layer(lw, dev, bits, g):
    def t3(name):
        c, s, z = lw[name]
        return (torch.from_numpy(c).to(dev), torch.from_numpy(s).to(torch.float16).to(dev),
                torch.from_numpy(z).to(torch.float16).to(dev))

    (qw, qs, qz), (ow, os_, oz), (gw, gs, gz), (uw, us, uz), (dw, ds, dz) = (t3(n) for n in
                                                                             ("qkv", "o", "gate", "up", "down"))
    return ll.LlamaLayerKernelWeights(
        input_layernorm_weight=torch.from_numpy(lw["ln1"]).to(dev),
        post_attention_layernorm_weight=torch.from_numpy(lw["ln2"]).to(dev), qkv_w=qw, qkv_scales=qs,
        qkv_zeros=qz, o_w=ow, o_scales=os_, o_zeros=oz, gate_w=gw, gate_scales=gs, gate_zeros=gz, up_w=uw,
        up_scales=us, up_zeros=uz, down_w=dw, down_scales=ds, down_zeros=dz, bits=bits, group_size=g)


def _caches(rng, B, mb, P, Hkv, D, fill):
    NP = B * mb + 2
    bt = rng.permutation(NP)[:B * mb].astype(np.int32).reshape(B, mb)
    K = (rng.standard_normal((NP, P, Hkv, D)) * fill).astype(np.float16)
    V = (rng.standard_normal((NP, P, Hkv, D)) * fill).astype(np.float16)
    return K, V, bt


@pytest.mark.parametrize("bits", [4, 8])
def test_paged_decode_layer_vs_oracle(dev, bits):
    """One layer: RMSNorm -> qkv matvec -> split + RoPE + paged write ->
    paged GQA attention -> o-proj + residual -> MLP block."""
    rng = np.random.default_rng(50 + bits)
    cfg, g, B, P, mb = _cfg(1), 32, 3, 16, 8
    lw = _np_layer(rng, cfg, bits, g)
    K, V, bt = _caches(rng, B, mb, P, cfg.num_key_value_heads, cfg.head_dim, 1.0)
    pos = np.array([5, 37, 100], np.int32)
    x = rng.standard_normal((B, cfg.hidden_size)).astype(np.float16)
    cos, sin = op.rope_tables(cfg.max_position_embeddings, cfg.head_dim, cfg.rope_theta)
    ref, Kr, Vr = ol.layer_decode_step(x, lw, K, V, bt, cos, sin, pos, cfg.num_attention_heads,
                                       cfg.num_key_value_heads, cfg.head_dim, bits, g)
    # the device-built tables differ from numpy's by float32 pow/cos ulps, which
    # grow with the position: the layer runs on the oracle's own tables
    tc, ts = ll.build_rope_tables(cfg, device=dev)
    assert np.allclose(tc.cpu().numpy(), cos, atol=2e-4) and np.allclose(ts.cpu().numpy(), sin, atol=2e-4)
    tc, ts = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)
    Kt, Vt, btt = (torch.from_numpy(a).to(dev) for a in (K, V, bt))
    out, (K2, V2, _), inter = ll.llama_layer_decode_step(
        torch.from_numpy(x).to(dev)[:, None], _t_layer(lw, dev, bits, g), (Kt, Vt, btt), tc, ts,
        torch.from_numpy(pos).to(dev), cfg, cache_layout="paged", return_intermediates=True)
    assert_close(out[:, 0], ref, what=f"layer out q{bits}")
    # the new token's k/v, written in place at (bt[b, pos // P], pos % P)
    page, off = op.block_table_lookup(bt, pos, P)
    for b in range(B):
        assert_close(K2[page[b], off[b]], Kr[page[b], off[b]], what=f"k written b{b}")
        assert_close(V2[page[b], off[b]], Vr[page[b], off[b]], what=f"v written b{b}")
    untouched = np.ones(K.shape[:2], bool)
    untouched[page, off] = False
    assert np.array_equal(K2.cpu().numpy()[untouched], K[untouched]), "cache rows other than the new token"
    # the HIP intermediates against the oracle's stages on the kernel's own inputs
    mv = oq.q4_matvec if bits == 4 else oq.q8_matvec
    xn = inter["x_norm"][:, 0].cpu().numpy()
    assert_close(inter["qkv"][:, 0], mv(xn, *lw["qkv"], group_size=g), what="qkv")
    h = inter["h"][:, 0].cpu().numpy()
    a = inter["attn_out"].reshape(B, -1).cpu().numpy()
    assert_close(h, oq.residual_add(x, mv(a, *lw["o"], group_size=g)), what="h = x + o-proj")


def test_paged_decode_layer_matches_reference_backend(dev):
    """The HIP layer against the package's own torch reference path (the
    reference backends of every stage)."""
    rng = np.random.default_rng(61)
    cfg, g, B, P, mb = _cfg(1), 32, 2, 16, 6
    lw = _np_layer(rng, cfg, 4, g)
    K, V, bt = _caches(rng, B, mb, P, cfg.num_key_value_heads, cfg.head_dim, 1.0)
    pos = torch.tensor([3, 90], dtype=torch.int32, device=dev)
    x = torch.from_numpy(rng.standard_normal((B, 1, cfg.hidden_size)).astype(np.float16)).to(dev)
    tc, ts = ll.build_rope_tables(cfg, device=dev)
    w = _t_layer(lw, dev, 4, g)
    cache = tuple(torch.from_numpy(a).to(dev) for a in (K, V, bt))
    ref, (Kr, _, _) = ll.reference_llama_layer_decode_step(x, w, cache, tc, ts, pos, cfg, cache_layout="paged")
    assert torch.equal(cache[0].cpu(), torch.from_numpy(K)), "the reference path leaves its input cache alone"
    out, (K2, _, _) = ll.llama_layer_decode_step(x, w, tuple(t.clone() for t in cache), tc, ts, pos, cfg,
                                                 cache_layout="paged")
    assert_close(out, ref.float().cpu().numpy(), what="HIP vs reference backend")
    assert_close(K2, Kr.float().cpu().numpy(), what="cache after the step")


def test_decode_stack_greedy_tokens_vs_oracle(dev):
    """A 2-layer stack, q4 head, greedy decode for 4 steps through the
    captured decode graph: each step's tokens against the oracle's, with the
    oracle fed the HIP tokens (a near-tie may flip an argmax; then both
    candidates' oracle logits must agree to within the tolerance)."""
    rng = np.random.default_rng(71)
    cfg, g, B, P, bits = _cfg(2, vocab=512), 32, 2, 16, 4
    ctx = [40, 75]
    mb = 8
    layers = [_np_layer(rng, cfg, bits, g) for _ in range(cfg.num_hidden_layers)]
    emb = rng.standard_normal((cfg.vocab_size, cfg.hidden_size)).astype(np.float16)
    head = _linear(rng, cfg.vocab_size, cfg.hidden_size, bits, g)
    fnorm = np.ones(cfg.hidden_size, np.float16)
    caches_np = []
    bt = rng.permutation(B * mb).astype(np.int32).reshape(B, mb)
    for _ in range(cfg.num_hidden_layers):
        K = (rng.standard_normal((B * mb, P, cfg.num_key_value_heads, cfg.head_dim))).astype(np.float16)
        V = (rng.standard_normal((B * mb, P, cfg.num_key_value_heads, cfg.head_dim))).astype(np.float16)
        caches_np.append((K, V))
    cos, sin = op.rope_tables(cfg.max_position_embeddings, cfg.head_dim, cfg.rope_theta)
    tc, ts = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)

    hc, hs, hz = head
    wts = ls.LlamaStackWeights(
        layers=[_t_layer(lw, dev, bits, g) for lw in layers], final_norm_weight=torch.from_numpy(fnorm).to(dev),
        lm_head=ls.QuantizedHead(torch.from_numpy(hc).to(dev), torch.from_numpy(hs).to(torch.float16).to(dev),
                                 torch.from_numpy(hz).to(torch.float16).to(dev), bits, g),
        embedding=torch.from_numpy(emb).to(dev)).validate(cfg)
    btt = torch.from_numpy(bt).to(dev)
    cache = ls.LlamaStackCache([(torch.from_numpy(K.copy()).to(dev), torch.from_numpy(V.copy()).to(dev), btt)
                                for K, V in caches_np], "paged", mb * P, P)
    tokens = np.array([7, 300])
    pos = np.array(ctx, np.int32)
    graph = ls.DecodeGraph(wts, cache, tc, ts, cfg, torch.from_numpy(tokens).to(dev),
                           torch.from_numpy(pos).to(dev))
    first = graph.first_tokens.cpu().numpy()  # the construction's eager step
    assert np.array_equal(first, graph.tokens.cpu().numpy())
    hip_steps = [first] + [graph.step().cpu().numpy() for _ in range(3)]
    oc = caches_np
    cur = tokens
    for s, got in enumerate(hip_steps):
        want, logits, oc = ol.stack_decode_step(cur, {"layers": layers, "embedding": emb, "final_norm": fnorm,
                                                      "lm_head": head}, oc, bt, cos, sin, pos + s,
                                                cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim,
                                                bits, g)
        for b in range(B):
            if got[b] != want[b]:
                lg = logits[b]
                assert abs(lg[got[b]] - lg[want[b]]) <= 2e-2 * max(1.0, abs(lg[want[b]])), (s, b, got[b], want[b])
        cur = got
    # the caches hold every written token, and the positions advanced by one per step
    assert np.array_equal(graph.positions.cpu().numpy(), pos + len(hip_steps))


@pytest.mark.parametrize("bits,B", [(4, 1), (4, 2), (4, 3), (4, 8), (4, 20), (4, 33), (8, 1), (8, 4), (8, 20)])
def test_fused_norm_qkv_rope_paged_matches_two_step(dev, bits, B):
    """RMSNorm + qkv projection + split + RoPE + paged write -- one launch for
    one q4 row, else the norm kernel then a projection (v_dot2 rows, MFMA,
    two-column tiles, in passes past 32 rows) whose epilogue rotates and
    writes -- against the separate norm + projection + update ops on the same
    inputs: q and every cache byte equal.  From B = 3 on, rows 1 and 2 target
    one slot (the later row wins)."""
    rng = np.random.default_rng(90 + bits + B)
    cfg, g, P, mb = _cfg(1), 32, 16, 4
    fused_vs_two_step(dev, rng, cfg, _t_layer(_np_layer(rng, cfg, bits, g), dev, bits, g), bits, B, g, P, mb)


def fused_vs_two_step(dev, rng, cfg, w, bits, B, g, P, mb):
    from mk import _lib
    from mk import gqa_ops
    from mk import quantized_decode_block_ops as qd
    from mk.quant_ops import q_rmsnorm_matvec

    Hq, Hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    K0, V0, bt = _caches(rng, B, mb, P, Hkv, D, 1.0)
    pos = rng.integers(0, mb * P, size=B).astype(np.int32)
    if B >= 3:
        bt[2] = bt[1]  # rows 1 and 2 share the page holding one position
        pos[2] = pos[1]
    x = torch.from_numpy(rng.standard_normal((B, cfg.hidden_size)).astype(np.float16)).to(dev)
    cos, sin = op.rope_tables(cfg.max_position_embeddings, D, cfg.rope_theta)
    tc, ts = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)
    btt, post = torch.from_numpy(bt).to(dev), torch.from_numpy(pos).to(dev)
    Kf, Vf = torch.from_numpy(K0.copy()).to(dev), torch.from_numpy(V0.copy()).to(dev)
    q, _ = qd.rmsnorm_qkv_rope_paged_update(x, w.input_layernorm_weight, w.qkv_w, w.qkv_scales, w.qkv_zeros, Kf, Vf,
                                            btt, tc, ts, post, num_attention_heads=Hq, num_key_value_heads=Hkv,
                                            head_dim=D, bits=bits, group_size=g)
    Kr, Vr = torch.from_numpy(K0.copy()).to(dev), torch.from_numpy(V0.copy()).to(dev)
    qkv = q_rmsnorm_matvec(x, w.input_layernorm_weight, w.qkv_w, w.qkv_scales, w.qkv_zeros, bits=bits,
                           group_size=g)
    x_, c_, s_, p_, q_ref, _ = gqa_ops._qkv_rope_update_prep(qkv[:, None], btt, tc, ts, post, Hq, Hkv, D, P,
                                                             torch.float16, dev)
    _lib.launch("mk_qkv_rope_paged_update", dev, _lib.ptr(x_), _lib.ptr(c_), _lib.ptr(s_), _lib.ptr(p_),
                _lib.ptr(btt), _lib.ptr(Kr), _lib.ptr(Vr), _lib.ptr(q_ref), B, Hq, Hkv, D, P, mb, Kr.shape[0],
                c_.shape[0], _lib.DT_F16)
    assert torch.equal(q, q_ref), "q"
    assert torch.equal(Kf, Kr) and torch.equal(Vf, Vr), "caches"
    # and the cache rows that changed are exactly the written slots
    changed = (Kf.cpu().numpy() != K0).any(axis=(2, 3))
    page, off = op.block_table_lookup(bt, pos, P)
    expect = np.zeros_like(changed)
    expect[page, off] = True
    assert np.array_equal(changed, expect)
