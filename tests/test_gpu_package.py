"""A written quantized package brought into HBM: the chunked pinned-buffer
loader copies payload files bit-exactly, and a 2-layer q4 package loaded with
load_quantized_stack decodes to the same final hidden state, bit for bit, as
the same arrays moved to the device directly; its first layer meets the
oracle's within the layer tests' tolerance."""

import numpy as np
import pytest
import torch

from mk import llama_layer_ops as ll
from mk import llama_stack_ops as ls
from mk import quantized_layer_package as qlp
from mk import quantized_package_io as qpio
from mk import quantized_package_writer as qpw
from mk import tensor_data_io as tdio
from oracle import llama as ol
from oracle import paged as op
from tests._data import assert_close
from tests.test_gpu_llama_fullshape import _ulp16

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shape,dtype,chunk", [((1000, 37), np.uint8, 4096), ((513, 64), np.float16, 1000),
                                               ((3, 5, 7), np.float32, 64 << 20), ((0, 4), np.float16, 256)])
def test_chunked_device_load_bit_exact(dev, tmp_path, shape, dtype, chunk):
    print(f"device load {shape} {np.dtype(dtype)} chunk {chunk}", flush=True)
    rng = np.random.default_rng(3)
    arr = (rng.integers(0, 256, size=shape).astype(np.uint8) if dtype == np.uint8
           else rng.standard_normal(shape).astype(dtype))
    info = tdio.save_tensor_npy(arr, tmp_path / "a.npy")
    got = tdio.load_tensor_to_device(info.file_path, dev, expected_shape=shape, expected_checksum=info.checksum,
                                     chunk_bytes=chunk)
    assert got.device.type == "cuda" and tuple(got.shape) == shape
    assert np.array_equal(got.cpu().numpy().view(np.uint8), arr.view(np.uint8))


def test_device_load_with_conversion_in_a_row(dev, tmp_path):
    """fp32 scales / zeros loaded with dtype=float16, several in a row behind
    queued work on the current stream: each load's staging copies wait for
    that stream, so the block freed by the previous call's conversion is not
    overwritten while the conversion still reads it -- every result equals
    numpy's fp16 rounding, bit for bit."""
    print("fp32 -> fp16 loads in a row", flush=True)
    rng = np.random.default_rng(7)
    arrays = [rng.standard_normal((1024, 256)).astype(np.float32) for _ in range(6)]
    infos = [tdio.save_tensor_npy(a, tmp_path / f"s{i}.npy") for i, a in enumerate(arrays)]
    got = []
    for info in infos:
        torch.cuda._sleep(2_000_000)  # keep work queued on the current stream
        got.append(tdio.load_tensor_to_device(info.file_path, dev, dtype=torch.float16, chunk_bytes=256 << 10))
    torch.cuda.synchronize()
    for a, t in zip(arrays, got):
        assert t.dtype == torch.float16
        assert np.array_equal(t.cpu().numpy().view(np.uint16), a.astype(np.float16).view(np.uint16))


def _np_linear(rng, n, k, g):
    codes = rng.integers(0, 16, size=(n, k // 2), dtype=np.uint8) | (rng.integers(0, 16, size=(n, k // 2),
                                                                                   dtype=np.uint8) << 4)
    # the statistics of N(0, 0.02) weights quantized at this group size, as the
    # full-shape layer tests draw them
    s = rng.uniform(0.002, 0.004, size=(n, k // g)).astype(np.float16)
    return codes.astype(np.uint8), s


def test_loaded_package_decodes_like_direct_weights(dev, tmp_path):
    print("package -> HBM -> decode step", flush=True)
    rng = np.random.default_rng(11)
    cfg = ll.LlamaLikeConfig(hidden_size=256, intermediate_size=512, num_attention_heads=4, num_key_value_heads=2,
                             head_dim=64, num_hidden_layers=2, max_position_embeddings=256, vocab_size=384).validate()
    g, B, P, mb = 32, 2, 16, 8
    H, I = cfg.hidden_size, cfg.intermediate_size
    layers = []
    for i in range(2):
        lin = {}
        for key, (n, k) in {"qkv": (cfg.qkv_output_dim(), H), "o_proj": (H, H), "gate_proj": (I, H),
                            "up_proj": (I, H), "down_proj": (H, I)}.items():
            w, s = _np_linear(rng, n, k, g)
            lin[key] = qlp.QuantizedLinearPackage(f"layers.{i}.{key}", w, s, None, 4, g, (n, k))
        layers.append(qlp.QuantizedLlamaLayerPackage(
            i, (1 + 0.1 * rng.standard_normal(H)).astype(np.float16),
            (1 + 0.1 * rng.standard_normal(H)).astype(np.float16), **lin))
    emb = rng.standard_normal((cfg.vocab_size, H)).astype(np.float16)
    fnorm = (1 + 0.1 * rng.standard_normal(H)).astype(np.float16)
    pkg = qpio.package_from_quantized_layers(cfg, layers, bits=4, group_size=g)
    pkg.global_tensors["norm"] = qpio.QuantizedTensorMetadata("norm", "norm", 0, 0, (H,), (H,), (0,))
    pkg.global_tensors["embedding"] = qpio.QuantizedTensorMetadata("embedding", "embedding", 0, 0,
                                                                   emb.shape, emb.shape, (0,))
    qpw.QuantizedPackageWriter().write_tensors(pkg, layers, tmp_path, global_tensors={
        "norm": fnorm, "embedding": emb}).raise_for_errors()

    cfg2, loaded = qpio.load_quantized_stack(tmp_path, dev)
    assert cfg2 == cfg
    direct = ls.LlamaStackWeights(layers=[lp.to_device(dev).to_kernel_weights(cfg) for lp in layers],
                                  final_norm_weight=torch.from_numpy(fnorm).to(dev),
                                  embedding=torch.from_numpy(emb).to(dev)).validate(cfg)
    for a, b in zip(loaded.layers, direct.layers):
        for f in ("qkv_w", "qkv_scales", "qkv_zeros", "down_w", "down_scales", "input_layernorm_weight"):
            assert torch.equal(getattr(a, f), getattr(b, f)), f
    bt = rng.permutation(B * mb).astype(np.int32).reshape(B, mb)
    caches = [(rng.standard_normal((B * mb, P, 2, 64)).astype(np.float16),
               rng.standard_normal((B * mb, P, 2, 64)).astype(np.float16)) for _ in range(2)]
    cos, sin = op.rope_tables(cfg.max_position_embeddings, cfg.head_dim, cfg.rope_theta)
    tc, ts = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)
    btt = torch.from_numpy(bt).to(dev)
    pos = np.array([30, 101], np.int32)
    tokens = np.array([5, 300])
    outs = []
    for w in (loaded, direct):
        cache = ls.LlamaStackCache([(torch.from_numpy(K.copy()).to(dev), torch.from_numpy(V.copy()).to(dev), btt)
                                    for K, V in caches], "paged", mb * P, P)
        x = ls.embed_token_ids(torch.from_numpy(tokens).to(dev), w.embedding)
        hidden, _ = ls.llama_stack_decode_step(x, w, cache, tc, ts, torch.from_numpy(pos).to(dev), cfg)
        outs.append(hidden)
    assert torch.equal(outs[0], outs[1])
    # and the loaded stack's layer 0 against the oracle
    lw0 = {k: (layers[0].__dict__[n].weight, layers[0].__dict__[n].scales.astype(np.float32),
               np.full(layers[0].__dict__[n].scales.shape, 8.0, np.float32))
           for k, n in (("qkv", "qkv"), ("o", "o_proj"), ("gate", "gate_proj"), ("up", "up_proj"),
                        ("down", "down_proj"))}
    lw0["ln1"], lw0["ln2"] = layers[0].input_layernorm_weight, layers[0].post_attention_layernorm_weight
    cache = ls.LlamaStackCache([(torch.from_numpy(caches[0][0].copy()).to(dev),
                                 torch.from_numpy(caches[0][1].copy()).to(dev), btt)], "paged", mb * P, P)
    one = ls.LlamaStackWeights(layers=loaded.layers[:1], final_norm_weight=loaded.final_norm_weight)
    _, _, inter = ls.llama_stack_decode_step(ls.embed_token_ids(torch.from_numpy(tokens).to(dev), loaded.embedding),
                                             one, cache, tc, ts, torch.from_numpy(pos).to(dev),
                                             ll.LlamaLikeConfig(**{**cfg.to_dict(), "num_hidden_layers": 1}),
                                             return_intermediates=True)
    ref, _, _ = ol.layer_decode_step(emb[tokens], lw0, caches[0][0], caches[0][1], bt, cos, sin, pos, 4, 2, 64, 4, g)
    # out = h + down with h = x + o-proj: where they cancel, ulps of the
    # residual stream show (as in the layer tests)
    assert_close(inter["layers"][0][:, 0], ref, what="loaded layer 0 vs oracle",
                 extra=2 * _ulp16(emb[tokens]) + 2 * _ulp16(ref))
