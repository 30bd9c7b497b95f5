"""Multi-row (speculative-verify) paged attention and the one-pass verify of
a draft: the HIP path (mk_paged_verify_attention: the W * Hq/Hkv rows of a kv
head as the columns of one MFMA contraction over one K/V read, row w masked
at its own causal limit) against oracle.paged_verify_attention (the staged
decode loop of ops/speculative_verify_ops.py:228-262 restated), the
stack-level pass against W staged HIP decode steps and the oracle, and the
accept / replacement / commit rules."""

import numpy as np
import pytest
import torch

import mk.llama_stack_ops as ls
import mk.paged_quantized_kv_ops as pq
import mk.speculative_verify_ops as sv
from oracle import llama as ol
from oracle import paged as op
from tests._data import assert_close
from tests.test_gpu_llama import _cfg, _linear, _np_layer, _t_layer

pytestmark = pytest.mark.gpu


def _pages(rng, B, mb, P, Hkv, D, extra=3):
    NP = B * mb + extra
    K = rng.standard_normal((NP, P, Hkv, D)).astype(np.float32)
    V = rng.standard_normal((NP, P, Hkv, D)).astype(np.float32)
    bt = rng.permutation(NP)[:B * mb].astype(np.int32).reshape(B, mb)
    return K, V, bt


def _t(a, dev, dt):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dt).to(dev)


def _np16(a, dt):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dt).float().numpy()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("B,W,Hq,Hkv,D,P,mb", [
    (1, 2, 32, 8, 128, 16, 8), (3, 4, 32, 8, 128, 16, 40), (5, 8, 32, 8, 128, 16, 24),
    (2, 4, 32, 8, 64, 16, 16), (4, 3, 8, 8, 64, 16, 12), (2, 8, 8, 1, 128, 16, 10),
    (3, 5, 32, 4, 128, 8, 20), (2, 4, 16, 2, 96, 16, 6),
    (1, 16, 8, 2, 64, 16, 12), (2, 33, 4, 1, 64, 16, 8), (1, 64, 4, 4, 128, 16, 10)])
def test_verify_attention_vs_oracle(dev, dtype, B, W, Hq, Hkv, D, P, mb):
    """GQA 32/8, MHA, MQA, a non-16 page size (LDS page list), D = 96
    (generic kernel) and widths up to the limit of 64 (W·G rows of a kv head
    over several 16-column blocks, the division-free row mapping at its
    widest); lengths include rows that see nothing (length < W) and contexts
    split over several pairs."""
    print(f"verify attention {dtype} B={B} W={W} Hq={Hq} Hkv={Hkv} D={D} P={P} mb={mb}", flush=True)
    rng = np.random.default_rng(7 * B + W + D)
    K, V, bt = _pages(rng, B, mb, P, Hkv, D)
    q = rng.standard_normal((B, W, Hq, D)).astype(np.float32)
    lengths = rng.integers(W, mb * P + 1, size=B)
    lengths[0] = mb * P
    if B > 2:
        lengths[1] = max(1, W - 2)  # rows 0 .. 1 see nothing
    got = sv.paged_verify_attention(_t(q, dev, dtype), _t(K, dev, dtype), _t(V, dev, dtype), _t(bt, dev, torch.int32),
                                    _t(lengths, dev, torch.int32))
    ref = op.paged_verify_attention(_np16(q, dtype), _np16(K, dtype), _np16(V, dtype), bt, lengths)
    tol = dict(rtol=3e-2, atol=3e-2) if dtype == torch.bfloat16 else {}
    assert_close(got, ref, what=f"verify B={B} W={W}", **tol)
    if B > 2:
        assert torch.count_nonzero(got[1, :W - lengths[1]]) == 0


@pytest.mark.parametrize("W", [2, 4, 8])
def test_verify_attention_config3_lengths(dev, W):
    """Config-3 geometry (B = 16, Hq 32 / Hkv 8, D = 128, P = 16, lengths
    U[512, 8192]) with W draft rows per sequence."""
    print(f"verify attention config 3 W={W}", flush=True)
    rng = np.random.default_rng(300 + W)
    B, Hq, Hkv, D, P = 16, 32, 8, 128, 16
    lengths = rng.integers(512, 8193, size=B)
    mb = 8192 // P
    K, V, bt = _pages(rng, B, mb, P, Hkv, D, extra=0)
    K16, V16 = K.astype(np.float16), V.astype(np.float16)
    q = rng.standard_normal((B, W, Hq, D)).astype(np.float16)
    got = sv.paged_verify_attention(_t(q, dev, torch.float16), _t(K16, dev, torch.float16),
                                    _t(V16, dev, torch.float16), _t(bt, dev, torch.int32),
                                    _t(lengths, dev, torch.int32))
    ref = op.paged_verify_attention(q, K16, V16, bt, lengths)
    assert_close(got, ref, what=f"config-3 verify W={W}")


@pytest.mark.parametrize("B,W,Hq,Hkv,mb", [(2, 4, 32, 8, 8), (2, 3, 24, 3, 6), (16, 4, 32, 8, 512), (16, 5, 40, 5, 512)])
def test_verify_causal_limits_straddle_blocks(dev, B, W, Hq, Hkv, mb):
    """Lengths 32k + 1 .. 32k + W - 2, so the W rows' limits fall on both
    sides of a 32-position block boundary (and, for the long tables, of
    split boundaries of the stream plan); W * G columns that are not a
    multiple of 16 (G = 8, W = 3 / 5) put a row boundary inside a 16-column
    tile.  Short tables run the short-context plan, 8192-wide tables the
    stream plan."""
    print(f"verify limits B={B} W={W} Hq={Hq} Hkv={Hkv} mb={mb}", flush=True)
    rng = np.random.default_rng(B * 100 + W * 10 + Hq)
    D, P = 128, 16
    K, V, bt = _pages(rng, B, mb, P, Hkv, D)
    K16, V16 = K.astype(np.float16), V.astype(np.float16)
    q = rng.standard_normal((B, W, Hq, D)).astype(np.float16)
    k = rng.integers(1, (mb * P) // 32, size=B)
    lengths = 32 * k + 1 + (np.arange(B) % max(1, W - 2))
    got = sv.paged_verify_attention(_t(q, dev, torch.float16), _t(K16, dev, torch.float16),
                                    _t(V16, dev, torch.float16), _t(bt, dev, torch.int32),
                                    _t(lengths, dev, torch.int32))
    ref = op.paged_verify_attention(q, K16, V16, bt, lengths)
    assert_close(got, ref, what=f"verify limits B={B} W={W}")


def test_verify_width_one_is_decode_bit_exact(dev):
    """W = 1 runs the decode attention's plan and kernel: identical bits."""
    import mk.gqa_ops as gqa

    rng = np.random.default_rng(5)
    B, Hq, Hkv, D, P, mb = 6, 32, 8, 128, 16, 64
    K, V, bt = _pages(rng, B, mb, P, Hkv, D)
    q = _t(rng.standard_normal((B, 1, Hq, D)), dev, torch.float16)
    lengths = rng.integers(1, mb * P + 1, size=B)
    args = (_t(K, dev, torch.float16), _t(V, dev, torch.float16), _t(bt, dev, torch.int32))
    ln = _t(lengths, dev, torch.int32)
    assert torch.equal(sv.paged_verify_attention(q, *args, ln), gqa.paged_gqa_decode_attention(q, *args, ln))


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("W", [2, 4])
def test_quantized_verify_attention_vs_oracle(dev, bits, W):
    print(f"quantized verify bits={bits} W={W}", flush=True)
    rng = np.random.default_rng(40 + bits + W)
    B, Hq, Hkv, D, P, mb, g = 4, 32, 8, 128, 16, 48, 64
    K, V, bt = _pages(rng, B, mb, P, Hkv, D)
    kq, vq, ks, vs = op.quantize_pages(K.astype(np.float16), V.astype(np.float16), g, bits)
    lengths = rng.integers(W, mb * P + 1, size=B)
    cache = pq.PagedQuantizedKVCache(
        k_pages_q=torch.from_numpy(kq).to(dev), v_pages_q=torch.from_numpy(vq).to(dev),
        k_scales=torch.from_numpy(ks).to(torch.float16).to(dev), v_scales=torch.from_numpy(vs).to(torch.float16).to(dev),
        block_table=_t(bt, dev, torch.int32), lengths=_t(lengths, dev, torch.int32), bits=bits, page_size=P,
        group_size=g, original_page_shape=K.shape)
    q = rng.standard_normal((B, W, Hq, D)).astype(np.float16)
    got = sv.paged_quantized_verify_attention(_t(q, dev, torch.float16), cache)
    ref = op.quantized_paged_verify_attention(q, kq, vq, ks.astype(np.float16).astype(np.float32),
                                              vs.astype(np.float16).astype(np.float32), bt, lengths, g, bits)
    assert_close(got, ref, what=f"q{bits} verify W={W}")


def test_verify_errors(dev):
    q = torch.zeros(1, 65, 8, 64, dtype=torch.float16, device=dev)
    K = torch.zeros(4, 16, 8, 64, dtype=torch.float16, device=dev)
    bt = torch.zeros(1, 4, dtype=torch.int32, device=dev)
    with pytest.raises(ValueError, match="verify width"):
        sv.paged_verify_attention(q, K, K, bt, 64)
    with pytest.raises(ValueError, match="backend must be one of"):
        sv.paged_verify_attention(q[:, :4], K, K, bt, 64, backend="metal_q8")


# ------------------------------------------------------------ stack pass


def _stack(rng, dev, cfg, bits, g, P, mb, B=1):
    layers = [_np_layer(rng, cfg, bits, g) for _ in range(cfg.num_hidden_layers)]
    emb = rng.standard_normal((cfg.vocab_size, cfg.hidden_size)).astype(np.float16)
    head = _linear(rng, cfg.vocab_size, cfg.hidden_size, bits, g)
    fnorm = np.ones(cfg.hidden_size, np.float16)
    hc, hs, hz = head
    wts = ls.LlamaStackWeights(
        layers=[_t_layer(lw, dev, bits, g) for lw in layers], final_norm_weight=torch.from_numpy(fnorm).to(dev),
        lm_head=ls.QuantizedHead(torch.from_numpy(hc).to(dev), torch.from_numpy(hs).to(torch.float16).to(dev),
                                 torch.from_numpy(hz).to(torch.float16).to(dev), bits, g),
        embedding=torch.from_numpy(emb).to(dev)).validate(cfg)
    bt = rng.permutation(B * mb).astype(np.int32).reshape(B, mb)
    caches = [(rng.standard_normal((B * mb, P, cfg.num_key_value_heads, cfg.head_dim)).astype(np.float16),
               rng.standard_normal((B * mb, P, cfg.num_key_value_heads, cfg.head_dim)).astype(np.float16))
              for _ in range(cfg.num_hidden_layers)]
    return layers, emb, head, fnorm, wts, bt, caches


def _dev_cache(caches, bt, dev, mb, P):
    btt = torch.from_numpy(bt).to(dev)
    return ls.LlamaStackCache([(torch.from_numpy(K.copy()).to(dev), torch.from_numpy(V.copy()).to(dev), btt)
                               for K, V in caches], "paged", mb * P, P)


@pytest.mark.parametrize("W", [1, 2, 4, 8])
def test_stack_verify_step_matches_staged_decode_steps(dev, W):
    """One W-row pass against W staged HIP decode steps (the reference's
    loop, run on this package's decode step) and against the oracle's staged
    loop: logits, final caches."""
    print(f"stack verify W={W}", flush=True)
    rng = np.random.default_rng(900 + W)
    cfg, bits, g, P, mb = _cfg(2, vocab=512), 4, 32, 16, 8
    layers, emb, head, fnorm, wts, bt, caches = _stack(rng, dev, cfg, bits, g, P, mb)
    cos, sin = op.rope_tables(cfg.max_position_embeddings, cfg.head_dim, cfg.rope_theta)
    tc, ts = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)
    p = 57
    drafts = rng.integers(0, cfg.vocab_size, size=W)
    # one pass
    cache1 = _dev_cache(caches, bt, dev, mb, P)
    x = sv.embed_proposed_tokens(drafts.tolist(), wts.embedding)
    logits, _, cache1 = sv.llama_stack_verify_step(x, wts, cache1, tc, ts, p, cfg)
    # W staged decode steps
    cache2 = _dev_cache(caches, bt, dev, mb, P)
    staged = []
    for i in range(W):
        xi = ls.embed_token_ids(torch.tensor([int(drafts[i])], device=dev), wts.embedding)
        lg, _, cache2 = ls.llama_stack_decode_step(xi, wts, cache2, tc, ts, torch.tensor([p + i], device=dev), cfg)
        staged.append(lg[0, 0].float().cpu().numpy())
    staged = np.stack(staged)
    got = logits[0].float().cpu().numpy()
    rms = float(np.sqrt(np.mean(staged.astype(np.float64) ** 2)))
    # same arithmetic per row up to the matvec kernels' row batching: the
    # K/V written and attended agree to fp16 rounding
    assert_close(got / rms, staged / rms, atol=8 * 2.0 ** -11, what=f"verify pass vs staged W={W}")
    for (K1, V1, _), (K2, V2, _) in zip(cache1.layer_caches, cache2.layer_caches):
        assert_close(K1, K2.float().cpu().numpy(), what="staged K")
        assert_close(V1, V2.float().cpu().numpy(), what="staged V")
    # the oracle's staged loop (ops/speculative_verify_ops.py:228-262)
    oc = caches
    ref = []
    for i in range(W):
        _, lg, oc = ol.stack_decode_step(np.array([drafts[i]]), {"layers": layers, "embedding": emb,
                                                                 "final_norm": fnorm, "lm_head": head},
                                         oc, bt, cos, sin, np.array([p + i]), cfg.num_attention_heads,
                                         cfg.num_key_value_heads, cfg.head_dim, bits, g)
        ref.append(lg[0])
    ref = np.stack(ref)
    assert_close(got / rms, ref / rms, atol=8 * 2.0 ** -11, what=f"verify pass vs oracle W={W}")


def test_parallel_verify_tokens_accept_replace_commit(dev):
    """The verify pass's targets against the staged decode loop's greedy
    tokens (a flip is allowed only at a near tie of the staged logits); the
    accept mask, accepted prefix and replacement follow
    models/speculative_decoding.py:163-228 on those targets; the live cache is
    untouched and commit copies exactly the accepted drafts' rows."""
    print("parallel_verify_tokens", flush=True)
    rng = np.random.default_rng(77)
    cfg, bits, g, P, mb = _cfg(2, vocab=512), 4, 32, 16, 8
    layers, emb, head, fnorm, wts, bt, caches = _stack(rng, dev, cfg, bits, g, P, mb)
    tc, ts = (torch.from_numpy(a).to(dev) for a in op.rope_tables(cfg.max_position_embeddings, cfg.head_dim,
                                                                   cfg.rope_theta))
    p, W = 40, 5
    drafts = [int(t) for t in rng.integers(0, cfg.vocab_size, size=W)]
    probe = _dev_cache(caches, bt, dev, mb, P)
    staged_logits = []
    for i in range(W):
        lg, _, probe = ls.llama_stack_decode_step(
            ls.embed_token_ids(torch.tensor([drafts[i]], device=dev), wts.embedding), wts, probe, tc, ts,
            torch.tensor([p + i], device=dev), cfg)
        staged_logits.append(lg[0, 0].float().cpu().numpy())
    staged_targets = [int(np.argmax(lg)) for lg in staged_logits]
    live = _dev_cache(caches, bt, dev, mb, P)
    res = sv.parallel_verify_tokens(context_token_ids=[1, 2, 3], proposed_token_ids=drafts, model_config=cfg,
                                    stack_weights=wts, stack_cache=live, cos=tc, sin=ts, position=p)
    assert res.metadata["verification_path"] == "multi_row_pass" and len(res.logits) == W
    for i, (a, b) in enumerate(zip(res.target_token_ids, staged_targets)):
        if a != b:
            lg = staged_logits[i]
            assert abs(lg[a] - lg[b]) <= 1e-2 * max(1.0, abs(lg[b])), (i, a, b)
    mask = sv.compute_accept_mask(drafts, res.target_token_ids)
    acc = sv.accepted_prefix_length(mask)
    assert res.accept_mask == mask and res.accepted_count == acc
    if acc < W:
        assert res.replacement_token_id == res.target_token_ids[acc]
        assert res.committed_tokens() == drafts[:acc] + [res.replacement_token_id]
    vr = res.to_verification_result()
    assert vr.accepted_count == acc and vr.rejected_count == W - acc
    # the live cache is untouched; commit copies exactly the given drafts' rows
    fresh = _dev_cache(caches, bt, dev, mb, P)
    for (K1, V1, _), (K0, V0, _) in zip(live.layer_caches, fresh.layer_caches):
        assert torch.equal(K1, K0) and torch.equal(V1, V0)
    n = 3
    sv.commit_parallel_verification_cache(live, res.staged_cache, start_position=p, accepted_count=n)
    for li in range(cfg.num_hidden_layers):
        K_live, K_st, K0 = live.layer_caches[li][0], res.staged_cache.layer_caches[li][0], fresh.layer_caches[li][0]
        for t in range(p - 2, p + W + 2):
            page, off = int(bt[0, t // P]), t % P
            want = K_st if p <= t < p + n else K0
            assert torch.equal(K_live[page, off], want[page, off]), (li, t)
