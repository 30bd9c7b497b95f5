"""Contiguous-cache neighbours on the GPU: decode attention / step and the
contiguous KV update (ops/decode_ops.py, ops/kv_cache_ops.py), the contiguous
q8/q4 KV cache and its GQA decode attention (ops/quantized_kv_cache_ops.py),
and the layer / stack decode loops (ops/llama_layer_ops.py:431,
ops/llama_stack_ops.py:439) -- against the oracle."""

import numpy as np
import pytest
import torch

import mk.decode_ops as dec
import mk.kv_cache_ops as kvc
import mk.quantized_kv_cache_ops as qkc
from mk import llama_layer_ops as ll
from mk import llama_stack_ops as ls
from oracle import paged as op
from tests._data import assert_close, to_dev
from tests.test_gpu_llama import _cfg, _np_layer, _t_layer

pytestmark = pytest.mark.gpu


def _kv(seed, B, S, H, D):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((B, 1, H, D)).astype(np.float16), rng.standard_normal((B, S, H, D)).astype(np.float16),
            rng.standard_normal((B, S, H, D)).astype(np.float16), rng)


@pytest.mark.parametrize("backend", ["auto", "metal", "metal_threadgroup", "metal_d128"])
@pytest.mark.parametrize("S,lengths", [(2048, [1, 700, 2048]), (100, [3, 99, 100]), (37, [37, 1, 20])])
def test_decode_attention(dev, backend, S, lengths):
    D = 128
    q, K, V, _ = _kv(S, 3, S, 8, D)
    got = dec.decode_attention(to_dev(q, dev), to_dev(K, dev), to_dev(V, dev), lengths, backend=backend)
    assert tuple(got.shape) == (3, 1, 8, D)
    assert_close(got[:, 0], op.contiguous_attention(q[:, 0], K, V, lengths), what=f"decode attention S{S}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_decode_step_in_place(dev, dtype):
    B, S, H, D = 4, 64, 4, 64
    q, K, V, rng = _kv(7, B, S, H, D)
    kn = rng.standard_normal((B, H, D)).astype(np.float16)
    vn = rng.standard_normal((B, 1, H, D)).astype(np.float16)
    Kt, Vt = to_dev(K, dev, dtype), to_dev(V, dev, dtype)
    pos = [0, 5, 63, 30]
    out, K2, V2 = dec.decode_step(to_dev(q, dev, dtype), to_dev(kn, dev, dtype), to_dev(vn, dev, dtype), Kt, Vt, pos,
                                  backend="metal_d64")
    assert K2 is Kt and V2 is Vt  # written in place
    Kf, Vf = to_dev(K, dev, dtype).float().cpu().numpy(), to_dev(V, dev, dtype).float().cpu().numpy()
    knf = to_dev(kn, dev, dtype).float().cpu().numpy()
    vnf = to_dev(vn, dev, dtype).float().cpu().numpy()[:, 0]
    rK, rV = op.contiguous_update(Kf, Vf, knf, vnf, pos)
    assert np.array_equal(K2.float().cpu().numpy(), rK) and np.array_equal(V2.float().cpu().numpy(), rV)
    qf = to_dev(q, dev, dtype).float().cpu().numpy()[:, 0]
    tol = (1e-2, 1e-3) if dtype == torch.float16 else (3e-2, 4e-3)
    assert_close(out[:, 0], op.contiguous_attention(qf, rK, rV, np.asarray(pos) + 1), rtol=tol[0], atol=tol[1],
                 what="decode step")
    # copy=True leaves the input alone
    Kc, Vc = to_dev(K, dev, dtype), to_dev(V, dev, dtype)
    K3, _ = kvc.kv_cache_update(Kc, Vc, to_dev(kn, dev, dtype), to_dev(vn, dev, dtype), 3, copy=True)
    assert torch.equal(Kc, to_dev(K, dev, dtype)) and not torch.equal(K3, Kc)


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("D,S,lengths", [(128, 4096, [4096, 1, 3000]), (64, 1000, [999, 1000, 17]),
                                         (128, 48, [48, 0, 5])])
def test_quantized_kv_cache_attention(dev, bits, D, S, lengths):
    B, Hq, Hkv, g = 3, 32, 8, 64
    rng = np.random.default_rng(bits + D + S)
    K = rng.standard_normal((B, S, Hkv, D)).astype(np.float16)
    V = rng.standard_normal((B, S, Hkv, D)).astype(np.float16)
    cfg = qkc.QuantizedKVCacheConfig(bits=bits, group_size=g)
    c = qkc.quantize_kv_cache(to_dev(K, dev), to_dev(V, dev), cfg, lengths=lengths)
    kq, vq, ks, vs = op.quantize_contiguous(K, V, g, bits, lengths)
    assert np.array_equal(c.k_q.cpu().numpy(), kq) and np.array_equal(c.v_q.cpu().numpy(), vq)
    assert np.array_equal(c.k_scales.cpu().numpy(), ks) and np.array_equal(c.v_scales.cpu().numpy(), vs)
    q = rng.standard_normal((B, 1, Hq, D)).astype(np.float16)
    got = qkc.quantized_kv_gqa_decode_attention(to_dev(q, dev), c, lengths, backend=f"metal_q{bits}")
    rK, rV = op.dequantize_pages(kq, vq, ks, vs, g, bits, D)
    ref = op.contiguous_attention(q[:, 0], rK, rV, lengths)
    assert_close(got[:, 0], ref, what=f"contiguous q{bits} D{D} S{S}")
    assert torch.all(got[np.asarray(lengths) == 0] == 0)
    Kd, _ = qkc.dequantize_kv_cache(c)
    assert np.array_equal(Kd.cpu().numpy(), rK)


def test_layer_contiguous_equals_paged(dev):
    """The layer on a contiguous cache (identity-paged view, P = 16) and on the
    same positions stored in permuted pages gives bit-identical outputs and
    writes the same K/V row."""
    rng = np.random.default_rng(5)
    cfg, g, B, S = _cfg(1), 32, 3, 128
    lw = _t_layer(_np_layer(rng, cfg, 4, g), dev, 4, g)
    Hkv, D, P = cfg.num_key_value_heads, cfg.head_dim, 16
    Kc = rng.standard_normal((B, S, Hkv, D)).astype(np.float16)
    Vc = rng.standard_normal((B, S, Hkv, D)).astype(np.float16)
    mb = S // P
    perm = rng.permutation(B * mb)
    bt = perm.reshape(B, mb).astype(np.int32)
    Kp = np.empty((B * mb, P, Hkv, D), np.float16)
    Vp = np.empty_like(Kp)
    Kp[perm] = Kc.reshape(B * mb, P, Hkv, D)
    Vp[perm] = Vc.reshape(B * mb, P, Hkv, D)
    x = to_dev(rng.standard_normal((B, 1, cfg.hidden_size)).astype(np.float16), dev)
    cos, sin = op.rope_tables(cfg.max_position_embeddings, D, cfg.rope_theta)
    tc, ts = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)
    pos = torch.tensor([0, 77, 127], dtype=torch.int32, device=dev)
    out_c, (K2, V2) = ll.llama_layer_decode_step(x, lw, (to_dev(Kc, dev), to_dev(Vc, dev)), tc, ts, pos, cfg)
    out_p, (Kp2, _, _) = ll.llama_layer_decode_step(x, lw, (to_dev(Kp, dev), to_dev(Vp, dev), to_dev(bt, dev)), tc,
                                                    ts, pos, cfg, cache_layout="paged")
    assert tuple(K2.shape) == (B, S, Hkv, D)
    assert torch.equal(out_c, out_p)
    # page i of the contiguous cache lives in physical page perm[i]
    assert torch.equal(K2.reshape(B * mb, P, Hkv, D), Kp2[torch.from_numpy(perm).to(dev)])


@pytest.mark.parametrize("preset", ["fused_experimental", "tiled", "reference"])
def test_layer_decode_loop(dev, preset):
    """llama_layer_decode_loop: T steps at positions 0..T-1, against stepping
    the layer by hand (bit-identical for the HIP presets) and against the
    reference preset at tolerance."""
    rng = np.random.default_rng(9)
    cfg, g, B, T, S = _cfg(1), 32, 2, 5, 32
    lw = _t_layer(_np_layer(rng, cfg, 4, g), dev, 4, g)
    inputs = to_dev(rng.standard_normal((B, T, cfg.hidden_size)).astype(np.float16), dev)
    cos, sin = op.rope_tables(cfg.max_position_embeddings, cfg.head_dim, cfg.rope_theta)
    tc, ts = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)
    cache = ll.init_llama_layer_cache(cfg, B, S, device=dev)
    out, (K, V) = ll.llama_layer_decode_loop(inputs, lw, cache, tc, ts, cfg, backend_preset=preset)
    assert tuple(out.shape) == (B, T, cfg.hidden_size)
    cache2 = ll.init_llama_layer_cache(cfg, B, S, device=dev)
    step = ll.reference_llama_layer_decode_step if preset == "reference" else ll.llama_layer_decode_step
    outs = []
    for t in range(T):
        o, cache2 = step(inputs[:, t:t + 1], lw, cache2, tc, ts, t, cfg)
        outs.append(o)
    assert torch.equal(out, torch.cat(outs, dim=1)) and torch.equal(K, cache2[0])
    assert not K[:, T:].any() and K[:, :T].abs().sum() > 0
    if preset != "reference":
        ref, _ = ll.llama_layer_decode_loop(inputs, lw, ll.init_llama_layer_cache(cfg, B, S, device=dev), tc, ts, cfg,
                                            backend_preset="reference")
        assert_close(out, ref.float().cpu().numpy(), what="loop vs reference preset")
    assert ll.llama_layer_decode_loop(inputs, lw, ll.init_llama_layer_cache(cfg, B, S, device=dev), tc, ts, cfg,
                                      T=2, return_final_cache=False).shape == (B, 2, cfg.hidden_size)


@pytest.mark.parametrize("layout", ["contiguous", "paged"])
def test_stack_decode_loop(dev, layout):
    """llama_stack_decode_loop over a 2-layer stack with a q4 head: logits of
    every step against the reference preset, and the final caches."""
    cfg = _cfg(2, vocab=256)
    B, T, S = 2, 4, 48
    w = ls.create_random_quantized_llama_stack_weights(cfg, bits=4, group_size=32, seed=3, device=dev)
    rng = np.random.default_rng(11)
    inputs = to_dev(rng.standard_normal((B, T, cfg.hidden_size)).astype(np.float16), dev)
    cos, sin = op.rope_tables(cfg.max_position_embeddings, cfg.head_dim, cfg.rope_theta)
    tc, ts = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)
    c1 = ls.init_llama_stack_cache(cfg, B, S, cache_layout=layout, device=dev)
    logits, c1 = ls.llama_stack_decode_loop(inputs, w, c1, tc, ts, cfg, cache_layout=layout)
    assert tuple(logits.shape) == (B, T, cfg.vocab_size) and logits.dtype == torch.float32
    c2 = ls.init_llama_stack_cache(cfg, B, S, cache_layout=layout, device=dev)
    ref, c2 = ls.reference_llama_stack_decode_loop(inputs, w, c2, tc, ts, cfg, cache_layout=layout)
    rms = float(ref.float().pow(2).mean().sqrt())
    assert_close(logits / rms, (ref / rms).float().cpu().numpy(), what=f"stack loop {layout}")
    for (Ka, _, *_), (Kb, _, *_) in zip(c1.layer_caches, c2.layer_caches):
        assert_close(Ka, Kb.float().cpu().numpy(), what="caches")
    hid, _ = ls.llama_stack_decode_loop(inputs[:, :, None], w, ls.init_llama_stack_cache(cfg, B, S, cache_layout=layout,
                                                                                        device=dev),
                                        tc, ts, cfg, cache_layout=layout, return_logits=False, T=2)
    assert tuple(hid.shape) == (B, 2, cfg.hidden_size)
    with pytest.raises(ValueError, match="does not match"):
        ls.llama_stack_decode_loop(inputs, w, c1, tc, ts, cfg,
                                   cache_layout="paged" if layout == "contiguous" else "contiguous")
