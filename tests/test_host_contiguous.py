"""Host (CPU tensor) paths of the contiguous-cache neighbours -- decode
attention / step, the contiguous KV update, the contiguous quantized KV cache
and its GQA decode attention -- against the oracle; the identity-paged view
they share; the decode loops' and registry's host-side behaviour.  No GPU."""

import numpy as np
import pytest
import torch

import mk.backend_registry as reg
import mk.decode_ops as dec
import mk.kv_cache_ops as kvc
import mk.quantized_kv_cache_ops as qkc
from mk import _contig
from oracle import paged as op
from tests._data import assert_close


def test_page_size_and_view():
    assert [_contig.page_size_for(s) for s in (16, 8192, 24, 100, 7, 2)] == [16, 16, 8, 4, 1, 2]
    K = torch.arange(2 * 24 * 3 * 4, dtype=torch.float32).reshape(2, 24, 3, 4)
    pages = _contig.as_pages(K, 8)
    assert pages.data_ptr() == K.data_ptr() and tuple(pages.shape) == (6, 8, 3, 4)
    bt = _contig.identity_table(2, 24, 8, "cpu")
    assert np.array_equal(bt.numpy(), op.identity_block_table(2, 24, 8))
    g, valid = op.gather(pages.numpy(), bt.numpy(), 24)
    assert valid.all() and np.array_equal(g, K.numpy())
    assert _contig.identity_table(2, 24, 8, "cpu") is bt  # cached
    with pytest.raises(ValueError, match="dense"):
        _contig.as_pages(K[:, ::2], 4)


@pytest.mark.parametrize("lengths", [None, [5, 24], 9])
def test_reference_decode_attention_matches_oracle(lengths):
    rng = np.random.default_rng(1)
    B, S, H, D = 2, 24, 4, 32
    q = rng.standard_normal((B, 1, H, D)).astype(np.float16)
    K = rng.standard_normal((B, S, H, D)).astype(np.float16)
    V = rng.standard_normal((B, S, H, D)).astype(np.float16)
    t = torch.from_numpy
    for fn in (lambda: dec.reference_decode_attention(t(q), t(K), t(V), lengths),
               lambda: dec.decode_attention(t(q), t(K), t(V), lengths, backend="reference")):
        got = fn()
        ln = S if lengths is None else lengths
        assert_close(got[:, 0], op.contiguous_attention(q[:, 0], K, V, ln), what=f"decode attention {lengths}")


def test_decode_attention_validation():
    q = torch.zeros(2, 1, 4, 32, dtype=torch.float16)
    K = torch.zeros(2, 8, 2, 32, dtype=torch.float16)
    with pytest.raises(ValueError, match="GQA"):
        dec.decode_attention(q, K, K)
    with pytest.raises(ValueError, match="q.shape\\[1\\] == 1"):
        dec.decode_attention(torch.zeros(2, 2, 2, 32, dtype=torch.float16), K, K)
    with pytest.raises(ValueError, match="D <= 128"):
        big = torch.zeros(1, 1, 1, 256, dtype=torch.float16)
        dec.decode_attention(big, big.expand(1, 4, 1, 256).contiguous(), big.expand(1, 4, 1, 256).contiguous())
    with pytest.raises(TypeError):
        f = torch.zeros(2, 1, 2, 32)
        dec.decode_attention(f, K.float(), K.float())
    with pytest.raises(ValueError, match="metal_d64"):
        dec.decode_attention(q[:, :, :2], K, K, backend="metal_d64")
    with pytest.raises(ValueError, match="positions must be in"):
        dec.decode_attention(q[:, :, :2], K, K, lengths=[3, 10])


def test_reference_decode_step_and_update():
    rng = np.random.default_rng(2)
    B, S, H, D = 2, 16, 2, 16
    K = rng.standard_normal((B, S, H, D)).astype(np.float16)
    V = rng.standard_normal((B, S, H, D)).astype(np.float16)
    kn = rng.standard_normal((B, 1, H, D)).astype(np.float16)
    vn = rng.standard_normal((B, H, D)).astype(np.float16)
    q = rng.standard_normal((B, 1, H, D)).astype(np.float16)
    t = torch.from_numpy
    K2, V2 = kvc.kv_cache_update(t(K), t(V), t(kn), t(vn), [0, 15], backend="reference")
    rK, rV = op.contiguous_update(K, V, kn[:, 0], vn, [0, 15])
    assert np.array_equal(K2.numpy(), rK) and np.array_equal(V2.numpy(), rV)
    out, K3, _ = dec.decode_step(t(q), t(kn), t(vn), t(K), t(V), [0, 15], backend="reference")
    assert np.array_equal(K3.numpy(), rK)
    assert_close(out[:, 0], op.contiguous_attention(q[:, 0], rK, rV, [1, 16]), what="decode step")
    assert np.array_equal(out[0, 0].numpy(), vn[0])  # position 0: the new token alone
    with pytest.raises(ValueError, match="positions must be in"):
        kvc.kv_cache_update(t(K), t(V), t(kn), t(vn), 16, backend="reference")
    with pytest.raises(ValueError, match="backend must be one of"):
        kvc.kv_cache_update(t(K), t(V), t(kn), t(vn), 1, backend="metal_d64")


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("lengths", [None, [3, 10]])
def test_host_quantized_kv_cache_bit_exact(bits, lengths):
    rng = np.random.default_rng(3 + bits)
    B, S, H, D, g = 2, 10, 2, 96, 32
    K = rng.standard_normal((B, S, H, D)).astype(np.float16)
    V = rng.standard_normal((B, S, H, D)).astype(np.float16)
    cfg = qkc.QuantizedKVCacheConfig(bits=bits, group_size=g)
    c = qkc.quantize_kv_cache(torch.from_numpy(K), torch.from_numpy(V), cfg, lengths=lengths)
    kq, vq, ks, vs = op.quantize_contiguous(K, V, g, bits, lengths)
    assert np.array_equal(c.k_q.numpy(), kq) and np.array_equal(c.v_q.numpy(), vq)
    assert np.array_equal(c.k_scales.numpy().view(np.uint16), ks.view(np.uint16))
    assert np.array_equal(c.v_scales.numpy().view(np.uint16), vs.view(np.uint16))
    Kd, Vd = qkc.dequantize_kv_cache(c)
    rK, rV = op.dequantize_pages(kq, vq, ks, vs, g, bits, D)
    assert np.array_equal(Kd.numpy(), rK) and np.array_equal(Vd.numpy(), rV)
    err = qkc.quantized_kv_error(torch.from_numpy(K), torch.from_numpy(V), c)
    if lengths is None:  # reference tests' bound (tests/test_quantized_kv_cache*.py: rmse < 1)
        assert err["k_rmse"] < 1.0 and err["v_rmse"] < 1.0
    assert 1.0 < err["compression_ratio"] < 10.0
    q = rng.standard_normal((B, 1, 4, D)).astype(np.float16)
    ln = [10, 10] if lengths is None else lengths
    got = qkc.quantized_kv_gqa_decode_attention(torch.from_numpy(q), c, ln)
    assert_close(got[:, 0], op.contiguous_attention(q[:, 0], rK, rV, ln), what="reference backend")


def test_quantized_kv_config_and_validation():
    with pytest.raises(NotImplementedError):
        qkc.QuantizedKVCacheConfig(symmetric=False).validate()
    with pytest.raises(NotImplementedError):
        qkc.QuantizedKVCacheConfig(layout="paged").validate()
    with pytest.raises(ValueError, match="bits must be 4 or 8"):
        qkc.QuantizedKVCacheConfig(bits=3).validate()
    K = torch.zeros(1, 4, 2, 32, dtype=torch.float16)
    c = qkc.quantize_kv_cache(K, K, qkc.QuantizedKVCacheConfig(bits=8, group_size=32))
    q = torch.zeros(1, 1, 4, 32, dtype=torch.float16)
    with pytest.raises(ValueError, match="metal_q4 backend requires bits=4"):
        qkc.quantized_kv_gqa_decode_attention(q, c, backend="metal_q4")
    with pytest.raises(ValueError, match="backend must be one of"):
        qkc.quantized_kv_gqa_decode_attention(q, c, backend="metal")
    with pytest.raises(ValueError, match="head_dim mismatch"):
        qkc.quantized_kv_gqa_decode_attention(torch.zeros(1, 1, 4, 16, dtype=torch.float16), c)
    import dataclasses
    bad = dataclasses.replace(c, k_scales=c.k_scales[:, :2].contiguous(), v_scales=c.v_scales[:, :2].contiguous())
    with pytest.raises(ValueError, match="must have shape"):
        qkc._check_kernel_layout(bad, 1, 4, 2, 32)


def test_registry_contiguous_and_loop_entries():
    for name in ("decode_attention", "quantized_kv_decode_attention", "llama_layer_decode", "llama_stack_decode"):
        assert name in reg.list_ops()
    assert reg.get_candidate_backends("llama_stack_decode") == ["metal", "tiled", "fused_experimental"]
    assert reg.filter_backends_for_shape("quantized_kv_decode_attention", {"Hq": 32, "Hkv": 8, "D": 128, "bits": 4},
                                         "float16", ["reference", "metal_q8", "metal_q4"]) == ["reference", "metal_q4"]
    assert reg.filter_backends_for_shape("llama_layer_decode", {"bits": 4}, "bfloat16",
                                         ["metal", "tiled", "fused_experimental"]) == ["metal", "tiled"]
    assert reg.filter_backends_for_shape("llama_stack_decode", {"bits": 3}, "float16", ["metal"]) == []
    assert reg.filter_backends_for_shape("decode_attention", {"D": 64}, "float16",
                                         ["metal", "metal_d64", "metal_d128"]) == ["metal", "metal_d64"]
