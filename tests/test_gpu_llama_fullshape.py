"""Config 5 at its real shape: Llama-3-8B layer geometry (hidden 4096, 32/8
heads, head_dim 128, intermediate 14336, q4 group 64, paged fp16 KV, P 16,
RoPE theta 500000) against the oracle, at batch 1 and 32, plus one stack step
through the 128256-entry q4 head and the HIP row argmax, and the benched
32-layer stack: one step held layer by layer against the oracle, and the
graph-replayed decode loop against eager steps.

Weights are random codes (uniform 0..15, zero point 8) with fp16 scales in
[0.002, 0.004] -- the statistics of N(0, 0.02) weights quantized at group 64 --
drawn directly, so the oracle does not have to run the weight quantizer over
218M parameters."""

import numpy as np
import pytest
import torch

from mk import llama_layer_ops as ll
from mk import llama_stack_ops as ls
from oracle import llama as ol
from oracle import paged as op
from oracle import quant as oq
from tests._data import assert_close
from tests.test_gpu_llama import _caches, _t_layer, fused_vs_two_step

pytestmark = pytest.mark.gpu

H, I, HQ, HKV, D, G, P, VOCAB = 4096, 14336, 32, 8, 128, 64, 16, 128256
CTX = 2048


def _cfg(layers=1, vocab=None):
    return ll.LlamaLikeConfig(hidden_size=H, intermediate_size=I, num_attention_heads=HQ, num_key_value_heads=HKV,
                              head_dim=D, num_hidden_layers=layers, max_position_embeddings=CTX + 256,
                              rope_theta=500000.0, vocab_size=vocab).validate()


def _q4(rng, n, k):
    codes = rng.integers(0, 16, size=(n, k // 2), dtype=np.uint8)
    packed = (codes & 0x0F) | (rng.integers(0, 16, size=(n, k // 2), dtype=np.uint8) << 4)
    s = rng.uniform(0.002, 0.004, size=(n, k // G)).astype(np.float16).astype(np.float32)
    return packed.astype(np.uint8), s, np.full(s.shape, 8.0, np.float32)


def _np_layer(rng):
    return {"qkv": _q4(rng, (HQ + 2 * HKV) * D, H), "o": _q4(rng, H, H), "gate": _q4(rng, I, H),
            "up": _q4(rng, I, H), "down": _q4(rng, H, I),
            "ln1": (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float16),
            "ln2": (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float16)}


@pytest.mark.parametrize("B", [1, 8, 32])
def test_fused_front_full_shape_bit_exact(dev, B):
    """RMSNorm (K = 4096) + 6144-row qkv projection + D = 128 RoPE pairs +
    paged write, fused, against norm + projection + mk_qkv_rope_paged_update:
    q and every cache byte equal (batch 1: one launch; batch 8 / 32: norm
    kernel + the activation-stationary projection with the RoPE epilogue, one
    and two 16-column tiles)."""
    rng = np.random.default_rng(500 + B)
    print(f"fused front full shape B={B}", flush=True)
    cfg = _cfg()
    w = _t_layer(_np_layer(rng), dev, 4, G)
    fused_vs_two_step(dev, rng, cfg, w, 4, B, G, P, CTX // P + 1)


@pytest.mark.parametrize("B", [1, 32])
def test_full_shape_layer_vs_oracle(dev, B):
    """One Llama-3-8B-shape q4 layer over a ~2048-position permuted paged
    cache: output, the written K/V slot and every untouched cache row."""
    rng = np.random.default_rng(600 + B)
    print(f"full-shape layer B={B}", flush=True)
    cfg = _cfg()
    lw = _np_layer(rng)
    mb = CTX // P + 1
    K, V, bt = _caches(rng, B, mb, P, HKV, D, 1.0)
    pos = rng.integers(CTX - 64, CTX + 8, size=B).astype(np.int32)
    x = rng.standard_normal((B, H)).astype(np.float16)
    cos, sin = op.rope_tables(cfg.max_position_embeddings, D, cfg.rope_theta)
    tc, ts = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)
    Kt, Vt, btt = (torch.from_numpy(a).to(dev) for a in (K, V, bt))
    out, (K2, V2, _), inter = ll.llama_layer_decode_step(
        torch.from_numpy(x).to(dev)[:, None], _t_layer(lw, dev, 4, G), (Kt, Vt, btt), tc, ts,
        torch.from_numpy(pos).to(dev), cfg, cache_layout="paged", return_intermediates=True)
    torch.cuda.synchronize(dev)
    ref, Kr, Vr = ol.layer_decode_step(x, lw, K, V, bt, cos, sin, pos, HQ, HKV, D, 4, G)
    # out = h + down, both rounded to fp16: where they cancel, one ulp of
    # either (at the size of the residual stream h) shows in the output
    assert_close(out[:, 0], ref, extra=2 * _ulp16(inter["h"][:, 0]), what=f"full-shape layer B={B}")
    page, off = op.block_table_lookup(bt, pos, P)
    K2n, V2n = K2.cpu().numpy(), V2.cpu().numpy()
    for b in range(B):
        assert_close(K2n[page[b], off[b]], Kr[page[b], off[b]], what=f"k written b{b}")
        assert_close(V2n[page[b], off[b]], Vr[page[b], off[b]], what=f"v written b{b}")
    untouched = np.ones(K.shape[:2], bool)
    untouched[page, off] = False
    assert np.array_equal(K2n[untouched], K[untouched]) and np.array_equal(V2n[untouched], V[untouched])


def _ulp16(t):
    a = np.abs(t.float().cpu().numpy() if isinstance(t, torch.Tensor) else np.asarray(t, np.float32))
    return 2.0 ** (np.floor(np.log2(np.maximum(a, 2.0 ** -14))) - 10)


@pytest.mark.parametrize("B", [1, 4])
def test_full_shape_stack_step_with_llama3_head(dev, B):
    """One decode step of a 1-layer Llama-3-8B-shape stack: embedding gather,
    the layer, final RMSNorm fused into the 128256 x 4096 q4 head, and the
    HIP row argmax, against oracle.stack_decode_step.  Each stage is checked
    at the kernel tolerance on its own HIP input (layer against the oracle
    layer, final norm and head against the oracle on the HIP layer output);
    the end-to-end logits carry the layer's fp16 differences through a
    4096-term dot product, so they are checked relative to the logits' rms.
    A near-tie may flip an argmax; then the two candidates' oracle logits
    must agree within that end-to-end tolerance."""
    rng = np.random.default_rng(700 + B)
    print(f"full-shape stack step B={B}", flush=True)
    cfg = _cfg(1, VOCAB)
    lw = _np_layer(rng)
    emb = rng.standard_normal((VOCAB, H)).astype(np.float16)
    head = _q4(rng, VOCAB, H)
    fnorm = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float16)
    mb = CTX // P + 1
    K, V, bt = _caches(rng, B, mb, P, HKV, D, 1.0)
    pos = rng.integers(CTX - 64, CTX, size=B).astype(np.int32)
    tokens = rng.integers(0, VOCAB, size=B)
    cos, sin = op.rope_tables(cfg.max_position_embeddings, D, cfg.rope_theta)
    tc, ts = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)
    hc, hs, hz = head
    wts = ls.LlamaStackWeights(
        layers=[_t_layer(lw, dev, 4, G)], final_norm_weight=torch.from_numpy(fnorm).to(dev),
        lm_head=ls.QuantizedHead(torch.from_numpy(hc).to(dev), torch.from_numpy(hs).to(torch.float16).to(dev),
                                 torch.from_numpy(hz).to(torch.float16).to(dev), 4, G),
        embedding=torch.from_numpy(emb).to(dev)).validate(cfg)
    btt = torch.from_numpy(bt).to(dev)
    cache = ls.LlamaStackCache([(torch.from_numpy(K.copy()).to(dev), torch.from_numpy(V.copy()).to(dev), btt)],
                               "paged", mb * P, P)
    x = ls.embed_token_ids(torch.from_numpy(tokens).to(dev), wts.embedding)
    assert np.array_equal(x[:, 0].cpu().numpy(), emb[tokens])
    logits, final_hidden, _, inter = ls.llama_stack_decode_step(
        x, wts, cache, tc, ts, torch.from_numpy(pos).to(dev), cfg, float_logits=False, return_intermediates=True)
    got = ls.greedy_sample(logits).cpu().numpy()
    got_logits = logits.float().cpu().numpy().reshape(B, VOCAB)
    want, ref_logits, _ = ol.stack_decode_step(tokens, {"layers": [lw], "embedding": emb, "final_norm": fnorm,
                                                        "lm_head": head}, [(K, V)], bt, cos, sin, pos, HQ, HKV, D,
                                               4, G)
    # the layer
    layer_out = inter["layers"][0][:, 0]
    ref_layer, _, _ = ol.layer_decode_step(emb[tokens], lw, K, V, bt, cos, sin, pos, HQ, HKV, D, 4, G)
    # out = h + down with h = x + o-proj: where they cancel, ulps of the
    # residual stream (the size of the layer's input row) show
    assert_close(layer_out, ref_layer, extra=2 * _ulp16(emb[tokens]) + 2 * _ulp16(layer_out), what=f"layer B={B}")
    # final norm (summed in another order: an element may land one step away)
    hl = layer_out.cpu().numpy()
    fh_ref = oq.rms_norm(hl, fnorm)
    fh = final_hidden[:, 0].float().cpu().numpy()
    assert np.all(np.abs(fh - fh_ref.astype(np.float32)) <= _ulp16(fh_ref) + 1e-7)
    # the head on the HIP normalised row: the kernel tolerance
    assert_close(got_logits, oq.q4_matvec(final_hidden[:, 0].cpu().numpy(), *head, group_size=G),
                 what=f"head logits B={B}")
    # end to end, relative to the logits' size: the layer output may differ
    # from the oracle's by up to 4 fp16 ulps of the residual stream (checked
    # above), i.e. a relative 4 * 2^-11 ~ 2e-3 per element, which the head's
    # 4096-term dot product carries into each logit at the logits' rms scale
    rms = float(np.sqrt(np.mean(ref_logits.astype(np.float64) ** 2)))
    e2e_atol = 2 * 4 * 2.0 ** -11  # twice that bound, for the tail over 128256 logits
    assert_close(got_logits / rms, ref_logits / rms, atol=e2e_atol, what=f"end-to-end logits B={B}")
    # the HIP argmax is np.argmax of the HIP logits exactly
    assert np.array_equal(got, np.argmax(got_logits, axis=-1))
    for b in range(B):
        if got[b] != want[b]:
            lg = ref_logits[b]
            assert abs(lg[got[b]] - lg[want[b]]) <= 1e-2 * abs(lg[want[b]]) + e2e_atol * rms, (b, got[b], want[b])


@pytest.mark.parametrize("B", [32, 17])
def test_head_full_shape_batched(dev, B):
    """The stack's final RMSNorm + 128256 x 4096 q4 head at decode batch 32
    (config 5's benched batch: the norm kernel, then the activation-stationary
    batched matvec over all 8016 row tiles) and at an odd batch: the whole
    head runs on the device; the oracle checks the normalised rows and a
    sample of 2,240 head rows -- the first and last 512 and every 97th between
    them -- on the HIP normalised rows, at the kernel tolerance."""
    rng = np.random.default_rng(800 + B)
    print(f"full-shape head B={B}", flush=True)
    hidden = rng.standard_normal((B, H)).astype(np.float16)
    fnorm = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float16)
    hc, hs, hz = _q4(rng, VOCAB, H)
    from mk.quant_ops import q_rmsnorm_matvec
    y, normed = q_rmsnorm_matvec(torch.from_numpy(hidden).to(dev), torch.from_numpy(fnorm).to(dev),
                                 torch.from_numpy(hc).to(dev), torch.from_numpy(hs).to(torch.float16).to(dev),
                                 torch.from_numpy(hz).to(torch.float16).to(dev), bits=4, group_size=G, eps=1e-5,
                                 return_normed=True)
    assert tuple(y.shape) == (B, VOCAB)
    nrm = normed.cpu().numpy()
    ref_n = oq.rms_norm(hidden, fnorm)
    assert np.all(np.abs(nrm.astype(np.float32) - ref_n.astype(np.float32)) <= _ulp16(ref_n) + 1e-7)
    rows = np.unique(np.concatenate([np.arange(512), np.arange(VOCAB - 512, VOCAB), np.arange(512, VOCAB - 512, 97)]))
    got = y.float().cpu().numpy()[:, rows]
    ref = oq.q4_matvec(nrm, hc[rows], hs[rows], hz[rows], group_size=G)
    assert_close(got, ref, what=f"head rows B={B}")


# ------------------------------------------------------------ full depth

LAYERS = 32


def _deep_stack(dev, seed, B):
    """32 Llama-3-8B-shape layers sharing one random q4 weight set (so the
    oracle dequantizes it once), the 128256-entry q4 head, and the embedding
    table and per-layer paged caches of ~2048 positions drawn on the device.
    Returns the embedding rows of the tokens (host) for the oracle.

    The o-proj and down scales are a tenth of the others: with one weight set
    in every layer the layers' residual updates line up, and at full size the
    stream would grow outliers whose fp16 ulps exceed the tolerance; at a
    tenth each layer adds ~0.1 and the stream keeps its N(0, 1) scale over 32
    layers, as in the one-layer tests."""
    rng = np.random.default_rng(seed)
    cfg = _cfg(LAYERS, VOCAB)
    lw = _np_layer(rng)
    for name in ("o", "down"):
        c, sc, z = lw[name]
        lw[name] = (c, (sc * 0.1).astype(np.float16).astype(np.float32), z)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    emb_t = torch.randn((VOCAB, H), device=dev, generator=gen).to(torch.float16)
    head = _q4(rng, VOCAB, H)
    fnorm = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float16)
    tw = _t_layer(lw, dev, 4, G)
    hc, hs, hz = head
    wts = ls.LlamaStackWeights(
        layers=[tw] * LAYERS, final_norm_weight=torch.from_numpy(fnorm).to(dev),
        lm_head=ls.QuantizedHead(torch.from_numpy(hc).to(dev), torch.from_numpy(hs).to(torch.float16).to(dev),
                                 torch.from_numpy(hz).to(torch.float16).to(dev), 4, G),
        embedding=emb_t).validate(cfg)
    mb = CTX // P + 4
    NP = B * mb + 2
    bt = rng.permutation(NP)[:B * mb].astype(np.int32).reshape(B, mb)
    caches = [(torch.randn((NP, P, HKV, D), device=dev, generator=gen).to(torch.float16),
               torch.randn((NP, P, HKV, D), device=dev, generator=gen).to(torch.float16)) for _ in range(LAYERS)]
    pos = rng.integers(CTX - 64, CTX, size=B).astype(np.int32)
    tokens = rng.integers(0, VOCAB, size=B)
    emb_rows = emb_t[torch.from_numpy(tokens).to(dev)].cpu().numpy()
    return cfg, lw, emb_rows, head, fnorm, wts, bt, caches, pos, tokens, mb


@pytest.mark.parametrize("B,checked", [(1, tuple(range(LAYERS))), (32, (0, 1, 16, LAYERS - 1))])
def test_full_depth_stack_step_vs_oracle(dev, B, checked):
    """One decode step of the benched config-5 stack -- 32 Llama-3-8B-shape
    q4 layers, the 128256 x 4096 q4 head, ~2048-position paged caches -- at
    batch 1 and 32.  Each checked layer is held against the oracle layer run
    on that layer's HIP input (so the differences of earlier layers do not
    compound): its output at the tolerance of the one-layer test, its written
    K/V slot, every other cache row untouched.  The final norm and the head
    are checked on the HIP final hidden state."""
    print(f"full-depth stack B={B}", flush=True)
    cfg, lw, emb, head, fnorm, wts, bt, caches, pos, tokens, mb = _deep_stack(dev, 1000 + B, B)
    cos, sin = op.rope_tables(cfg.max_position_embeddings, D, cfg.rope_theta)
    tc, ts = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)
    btt = torch.from_numpy(bt).to(dev)
    before = {li: (caches[li][0].cpu().numpy(), caches[li][1].cpu().numpy()) for li in checked}
    cache = ls.LlamaStackCache([(K, V, btt) for K, V in caches], "paged", mb * P, P)
    x = ls.embed_token_ids(torch.from_numpy(tokens).to(dev), wts.embedding)
    logits, final_hidden, cache, inter = ls.llama_stack_decode_step(
        x, wts, cache, tc, ts, torch.from_numpy(pos).to(dev), cfg, float_logits=False, return_intermediates=True)
    torch.cuda.synchronize(dev)
    outs = [t[:, 0].cpu().numpy() for t in inter["layers"]]
    page, off = op.block_table_lookup(bt, pos, P)
    with oq.memoized_dequant():
        for li in checked:
            xin = emb[:] if li == 0 else outs[li - 1]
            K0, V0 = before[li]
            ref, Kr, Vr = ol.layer_decode_step(xin, lw, K0, V0, bt, cos, sin, pos, HQ, HKV, D, 4, G)
            assert_close(outs[li], ref, extra=2 * _ulp16(xin) + 2 * _ulp16(outs[li]), what=f"layer {li} B={B}")
            K2, V2 = (t.cpu().numpy() for t in cache.layer_caches[li][:2])
            for b in range(B):
                # k and v are 4096-term projections of the normalised input,
                # which the HIP norm and the oracle may round one ulp apart
                # in any element: with every element off by an ulp of random
                # sign the error's std is 2^-11 rms(k) (rms(k) = |W|_rms
                # |n|_2), plus half that for the M = 1 kernel's fp32 W; at
                # the residual stream of deep layers such flips are common,
                # so allow 6 x 2^-11 rms -- about 5 sigma over B x 1024 values
                for nm, got_kv, ref_kv in (("k", K2, Kr), ("v", V2, Vr)):
                    r = ref_kv[page[b], off[b]].astype(np.float64)
                    assert_close(got_kv[page[b], off[b]], r, extra=6 * 2.0 ** -11 * np.sqrt(np.mean(r * r)),
                                 what=f"layer {li} {nm} written b{b}")
            untouched = np.ones(K0.shape[:2], bool)
            untouched[page, off] = False
            assert np.array_equal(K2[untouched], K0[untouched]) and np.array_equal(V2[untouched], V0[untouched])
            del K2, V2, K0, V0, Kr, Vr
            before.pop(li)
        hl = outs[-1]
        fh = final_hidden[:, 0].float().cpu().numpy()
        assert np.all(np.abs(fh - oq.rms_norm(hl, fnorm).astype(np.float32)) <= _ulp16(oq.rms_norm(hl, fnorm)) + 1e-7)
        got = logits.float().cpu().numpy().reshape(B, VOCAB)
        assert_close(got, oq.q4_matvec(final_hidden[:, 0].cpu().numpy(), *head, group_size=G), what=f"head B={B}")
    assert np.array_equal(ls.greedy_sample(logits).cpu().numpy(), np.argmax(got, axis=-1))


@pytest.mark.parametrize("B", [1, 32])
def test_full_depth_decode_graph_matches_eager(dev, B):
    """The benched config-5 loop: DecodeGraph (one eager step, then HIP graph
    replays) against eager llama_stack_decode_step calls fed back their own
    greedy tokens, on copies of the same 32-layer caches: tokens of every
    step and every cache byte after three steps identical."""
    print(f"full-depth decode graph B={B}", flush=True)
    cfg, _, _, _, _, wts, bt, caches, pos, tokens, mb = _deep_stack(dev, 1100 + B, B)
    cos, sin = op.rope_tables(cfg.max_position_embeddings, D, cfg.rope_theta)
    tc, ts = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)
    btt = torch.from_numpy(bt).to(dev)
    c1 = ls.LlamaStackCache([(K.clone(), V.clone(), btt) for K, V in caches], "paged", mb * P, P)
    c2 = ls.LlamaStackCache([(K, V, btt) for K, V in caches], "paged", mb * P, P)
    tok = torch.from_numpy(tokens).to(dev)
    p = torch.from_numpy(pos).to(dev)
    graph = ls.DecodeGraph(wts, c1, tc, ts, cfg, tok, p)
    got = [graph.first_tokens.clone(), graph.step().clone(), graph.step().clone()]
    torch.cuda.synchronize(dev)
    want = []
    t, pp = tok.clone(), p.clone().to(torch.int32)
    for _ in range(3):
        lg, _, c2 = ls.llama_stack_decode_step(ls.embed_token_ids(t, wts.embedding), wts, c2, tc, ts, pp, cfg,
                                               float_logits=False)
        t = ls.greedy_sample(lg)
        want.append(t.clone())
        pp = pp + 1
    for s, (a, b) in enumerate(zip(got, want)):
        assert torch.equal(a, b), f"step {s} tokens"
    for li, ((K1, V1, _), (K2, V2, _)) in enumerate(zip(c1.layer_caches, c2.layer_caches)):
        assert torch.equal(K1, K2) and torch.equal(V1, V2), f"layer {li} caches"
