"""Drop-in entry points that wrap the hot-path kernels -- groupwise_dequant,
quantized_linear, quantized_gate_up_projection (every backend),
swiglu_down_project / fused_swiglu, the identity table and cache allocation,
paged_decode_step, dequantize_kv_pages / paged_quantized_kv_error,
contiguous <-> pages, and the reference backend of the quantized attention --
called through their reference signatures on the GPU and checked against the
oracle (or the reference tests' own checks)."""

import numpy as np
import pytest
import torch

import mk.activation_ops as act
import mk.mlp_block_ops as mlp
import mk.paged_kv_ops as pk
import mk.paged_quantized_kv_ops as pq
import mk.quant_ops as qo
from oracle import paged as op
from oracle import quant as oq
from tests._data import assert_close, quant_weight, to_dev

pytestmark = pytest.mark.gpu


# ------------------------------------------------------------ a6 groupwise_dequant

@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("zeros_kind", ["none", "affine"])
def test_groupwise_dequant_bit_exact(dev, bits, zeros_kind):
    # ops/quant_ops.py:319-333 dispatches to dequant_q4 / dequant_q8
    rng = np.random.default_rng(3 + bits)
    N, K, g = 40, 256, 32
    codes, stored, s, z = quant_weight(rng, N, K, g, bits, zeros_kind, "normal")
    s16 = s.astype(np.float16)
    got = qo.groupwise_dequant(to_dev(stored, dev), to_dev(s16, dev), None if z is None else to_dev(z, dev),
                               bits=bits, group_size=g)
    ref = oq.dequant(codes, s16.astype(np.float32), z, g, np.float16)
    assert got.dtype == torch.float16 and np.array_equal(got.cpu().numpy(), ref)
    with pytest.raises(ValueError, match="bits must be 4 or 8"):
        qo.groupwise_dequant(to_dev(stored, dev), to_dev(s16, dev), bits=3, group_size=g)


# ------------------------------------------------------------ a12 quantized_linear

@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("backend", ["auto", "metal", "metal_tiled", "metal_parallel", "reference"])
def test_quantized_linear_3d_input(dev, bits, backend):
    # ops/mlp_block_ops.py:77-101: [B,S,K] -> [B,S,N] through the matvec of `bits`
    rng = np.random.default_rng(12 + bits)
    B, S, K, N, g = 2, 3, 512, 96, 64
    codes, stored, s, z = quant_weight(rng, N, K, g, bits, "sym")
    s = s.astype(np.float16).astype(np.float32)
    x = rng.standard_normal((B, S, K)).astype(np.float16)
    y = mlp.quantized_linear(to_dev(x, dev), to_dev(stored, dev), to_dev(s, dev, torch.float16),
                             to_dev(z, dev, torch.float16), bits=bits, group_size=g, backend=backend)
    assert tuple(y.shape) == (B, S, N) and y.dtype == torch.float16
    mv = oq.q4_matvec if bits == 4 else oq.q8_matvec
    assert_close(y.reshape(B * S, N), mv(x.reshape(B * S, K), stored, s, z, g), what=f"linear {backend}")
    with pytest.raises(ValueError):
        mlp.quantized_linear(to_dev(x[..., :-64], dev), to_dev(stored, dev), to_dev(s, dev, torch.float16),
                             bits=bits, group_size=g, backend=backend)


# ------------------------------------------------------------ a13 gate/up projection

@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("backend", ["reference", "metal_tiled", "metal_parallel", "metal_gate_up_tiled"])
def test_quantized_gate_up_projection_backends(dev, bits, backend):
    # ops/mlp_block_ops.py:128-233
    rng = np.random.default_rng(20 + bits)
    B, S, K, N, g = 2, 1, 1024, 320, 64
    _, gst, gs, gz = quant_weight(rng, N, K, g, bits, "sym")
    _, ust, us, uz = quant_weight(rng, N, K, g, bits, "sym")
    gs, us = gs.astype(np.float16).astype(np.float32), us.astype(np.float16).astype(np.float32)
    x = rng.standard_normal((B, S, K)).astype(np.float16)
    gate, up = mlp.quantized_gate_up_projection(
        to_dev(x, dev), to_dev(gst, dev), to_dev(gs, dev, torch.float16), to_dev(ust, dev),
        to_dev(us, dev, torch.float16), gate_zeros=to_dev(gz, dev, torch.float16),
        up_zeros=to_dev(uz, dev, torch.float16), bits=bits, group_size=g, backend=backend)
    assert tuple(gate.shape) == (B, S, N) and tuple(up.shape) == (B, S, N)
    mv = oq.q4_matvec if bits == 4 else oq.q8_matvec
    xf = x.reshape(B * S, K)
    assert_close(gate.reshape(B * S, N), mv(xf, gst, gs, gz, g), what=f"gate {backend}")
    assert_close(up.reshape(B * S, N), mv(xf, ust, us, uz, g), what=f"up {backend}")


def test_quantized_gate_up_projection_rejects_unknown_backend(dev):
    x = torch.zeros((1, 1, 64), dtype=torch.float16, device=dev)
    w = torch.zeros((8, 32), dtype=torch.uint8, device=dev)
    s = torch.ones((8, 2), dtype=torch.float16, device=dev)
    with pytest.raises(ValueError, match="backend must be one of 'reference', 'metal_tiled', 'metal_parallel', "
                                         "'metal_gate_up_tiled'"):
        mlp.quantized_gate_up_projection(x, w, s, w, s, bits=4, group_size=32, backend="metal")


# ------------------------------------------------------------ a14 / a15 SwiGLU

@pytest.mark.parametrize("shape", [(5, 300), (2, 3, 128)])
@pytest.mark.parametrize("backend", ["metal_fused", "metal", "auto", "reference"])
def test_fused_swiglu(dev, shape, backend):
    # ops/activation_ops.py:117-153: [rows,D] or [B,S,D]; 'metal' needs 3-D
    rng = np.random.default_rng(30 + len(shape))
    g = (rng.standard_normal(shape) * 3).astype(np.float16)
    u = rng.standard_normal(shape).astype(np.float16)
    if backend == "metal" and len(shape) != 3:
        with pytest.raises(ValueError, match="requires \\[B,S,D\\]"):
            act.fused_swiglu(to_dev(g, dev), to_dev(u, dev), backend=backend)
        return
    out = act.fused_swiglu(to_dev(g, dev), to_dev(u, dev), backend=backend)
    assert tuple(out.shape) == shape
    ref = oq.swiglu(g.reshape(-1, shape[-1]), u.reshape(-1, shape[-1])).reshape(shape)
    assert_close(out, ref, rtol=2e-3, what=f"fused_swiglu {backend}")


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("activation_backend,matvec_backend", [("metal", "metal_tiled"), ("metal", "metal_parallel"),
                                                               ("reference", "reference")])
def test_swiglu_down_project(dev, bits, activation_backend, matvec_backend):
    # ops/mlp_block_ops.py:104-125: SwiGLU then the down quantized_linear
    rng = np.random.default_rng(40 + bits)
    B, S, I, D, g = 2, 1, 512, 128, 64
    gate = (rng.standard_normal((B, S, I)) * 2).astype(np.float16)
    up = rng.standard_normal((B, S, I)).astype(np.float16)
    _, dst, ds, dz = quant_weight(rng, D, I, g, bits, "sym")
    ds = ds.astype(np.float16).astype(np.float32)
    out = mlp.swiglu_down_project(to_dev(gate, dev), to_dev(up, dev), to_dev(dst, dev), to_dev(ds, dev, torch.float16),
                                  to_dev(dz, dev, torch.float16), bits=bits, group_size=g,
                                  activation_backend=activation_backend, matvec_backend=matvec_backend)
    assert tuple(out.shape) == (B, S, D)
    m = oq.swiglu(gate.reshape(-1, I), up.reshape(-1, I))
    mv = oq.q4_matvec if bits == 4 else oq.q8_matvec
    assert_close(out.reshape(-1, D), mv(m, dst, ds, dz, g), what="swiglu_down_project")


# ------------------------------------------------------------ a18 identity table / allocation

def test_identity_table_and_allocation_on_device(dev):
    # ops/paged_kv_ops.py:99-115
    for B, MAX_S, P in ((1, 16, 4), (3, 50, 16), (16, 8192, 16)):
        bt = pk.make_identity_block_table(B, MAX_S, P, device=dev)
        assert bt.dtype == torch.int32 and bt.device.type == "cuda"
        assert np.array_equal(bt.cpu().numpy(), op.identity_block_table(B, MAX_S, P))
    K, V, bt = pk.allocate_paged_kv_cache(3, 50, 4, 64, 16, torch.bfloat16, device=dev)
    assert tuple(K.shape) == (12, 16, 4, 64) and K.dtype == torch.bfloat16 and V.shape == K.shape
    assert not K.any() and not V.any()
    assert np.array_equal(bt.cpu().numpy(), op.identity_block_table(3, 50, 16))
    with pytest.raises(TypeError):
        pk.allocate_paged_kv_cache(1, 16, 1, 16, 4, torch.float32, device=dev)
    with pytest.raises(ValueError):
        pk.make_identity_block_table(0, 16, 4, device=dev)
    # an allocated cache written through the update and read by the attention
    K, V, bt = pk.allocate_paged_kv_cache(2, 32, 4, 64, 8, torch.float16, device=dev)
    k = torch.randn((2, 4, 64), device=dev).to(torch.float16)
    K, V = pk.paged_kv_cache_update(K, V, k, k, bt, [0, 0])
    out = pk.paged_decode_attention(k[:, None], K, V, bt, [1, 1])
    assert torch.equal(out[:, 0], k)


# ------------------------------------------------------------ a22 paged_decode_step

@pytest.mark.parametrize("backend", ["auto", "metal", "metal_threadgroup", "metal_d64", "reference"])
def test_paged_decode_step(dev, backend):
    # ops/paged_kv_ops.py:363-404: update at `position`, then attention over
    # lengths = position + 1
    rng = np.random.default_rng(50)
    B, H, D, P, mb = 3, 4, 64, 8, 6
    NP = B * mb
    Kp = rng.standard_normal((NP, P, H, D)).astype(np.float16)
    Vp = rng.standard_normal((NP, P, H, D)).astype(np.float16)
    bt = rng.permutation(NP).astype(np.int32).reshape(B, mb)
    pos = [0, 17, 47]
    q = rng.standard_normal((B, 1, H, D)).astype(np.float16)
    kn = rng.standard_normal((B, 1, H, D)).astype(np.float16)
    vn = rng.standard_normal((B, 1, H, D)).astype(np.float16)
    out, K2, V2 = pk.paged_decode_step(to_dev(q, dev), to_dev(kn, dev), to_dev(vn, dev), to_dev(Kp, dev),
                                       to_dev(Vp, dev), to_dev(bt, dev), pos, backend=backend)
    rK, rV = op.paged_kv_update(Kp, Vp, kn[:, 0], vn[:, 0], bt, pos)
    assert np.array_equal(K2.cpu().numpy(), rK) and np.array_equal(V2.cpu().numpy(), rV)
    ref = op.paged_attention(q[:, 0], rK, rV, bt, np.asarray(pos) + 1)
    assert_close(out[:, 0], ref, what=f"paged_decode_step {backend}")
    # position 0 attends to the new token alone: out = v_new exactly
    assert torch.equal(out[0, 0], to_dev(vn, dev)[0, 0])
    # a scalar position (int) broadcasts to every sequence
    out_i, _, _ = pk.paged_decode_step(to_dev(q, dev), to_dev(kn, dev), to_dev(vn, dev), to_dev(Kp, dev),
                                       to_dev(Vp, dev), to_dev(bt, dev), 9, backend=backend)
    rK, rV = op.paged_kv_update(Kp, Vp, kn[:, 0], vn[:, 0], bt, [9] * B)
    assert_close(out_i[:, 0], op.paged_attention(q[:, 0], rK, rV, bt, [10] * B), what="scalar position")


# ------------------------------------------------------------ a30 dequantize / error

@pytest.mark.parametrize("bits", [8, 4])
def test_dequantize_kv_pages_and_error(dev, bits):
    # ops/paged_quantized_kv_ops.py:295-367
    rng = np.random.default_rng(60 + bits)
    NP, P, Hkv, D, g = 6, 4, 2, 128, 64
    K = rng.standard_normal((NP, P, Hkv, D)).astype(np.float16)
    V = (rng.standard_normal((NP, P, Hkv, D)) * 0.01).astype(np.float16)
    bt = np.arange(NP, dtype=np.int32).reshape(2, 3)
    cfg = pq.PagedQuantizedKVConfig(bits=bits, page_size=P, group_size=g)
    c = pq.quantize_kv_pages(to_dev(K, dev), to_dev(V, dev), to_dev(bt, dev), to_dev(np.array([12, 12]), dev), cfg)
    Kd, Vd = pq.dequantize_kv_pages(c)
    kq, vq, ks, vs = op.quantize_pages(K, V, g, bits)
    rK, rV = op.dequantize_pages(kq, vq, ks, vs, g, bits, D)
    assert Kd.dtype == torch.float16 and np.array_equal(Kd.cpu().numpy(), rK) and np.array_equal(Vd.cpu().numpy(), rV)
    err = pq.paged_quantized_kv_error(to_dev(K, dev), to_dev(V, dev), c)
    kd = K.astype(np.float64) - rK.astype(np.float64)
    vd = V.astype(np.float64) - rV.astype(np.float64)
    want = {"k_max_abs_error": np.abs(kd).max(), "k_mean_abs_error": np.abs(kd).mean(),
            "k_rmse": np.sqrt((kd ** 2).mean()), "v_max_abs_error": np.abs(vd).max(),
            "v_mean_abs_error": np.abs(vd).mean(), "v_rmse": np.sqrt((vd ** 2).mean())}
    for k, v in want.items():
        assert abs(err[k] - v) <= 1e-6 + 1e-5 * abs(v), k
    # tests/test_paged_quantized_kv_ops.py:168-186 of the reference: rmse < 1.0
    assert err["k_rmse"] < 1.0 and err["v_rmse"] < 1.0
    assert 1.0 < err["compression_ratio"] < 10.0


# ------------------------------------------------------------ a31 contiguous <-> pages

def test_contiguous_pages_roundtrip_on_device(dev):
    # tests/test_paged_quantized_kv_ops.py:277-313 of the reference
    g = torch.Generator(device=dev).manual_seed(15)
    B, MAX_S, Hkv, D = 2, 8, 2, 16
    Kc = torch.randn((B, MAX_S, Hkv, D), generator=g, device=dev).to(torch.float16)
    Vc = torch.randn((B, MAX_S, Hkv, D), generator=g, device=dev).to(torch.float16)
    Kp, Vp, bt, ln = pq.contiguous_kv_to_pages(Kc, Vc, [6, 8], page_size=4)
    Kr, Vr = pq.pages_to_contiguous_kv(Kp, Vp, bt, ln, max_seq_len=MAX_S)
    for b, valid in enumerate([6, 8]):
        assert torch.equal(Kr[b, :valid], Kc[b, :valid]) and torch.equal(Vr[b, :valid], Vc[b, :valid])
        assert not Kr[b, valid:].any()
    assert bt.cpu().tolist() == [[0, 1], [2, 3]] and ln.cpu().tolist() == [6, 8]
    # the identity paging feeds the paged attention like the contiguous cache
    q = torch.randn((B, 1, 4, D), generator=g, device=dev).to(torch.float16)
    from mk import gqa_ops
    got = gqa_ops.paged_gqa_decode_attention(q, Kp, Vp, bt, ln)
    ref = op.attention(q[:, 0].float().cpu().numpy(), Kc.float().cpu().numpy(), Vc.float().cpu().numpy(),
                       np.array([6, 8]), np.ones((B, MAX_S), bool), 1.0 / 4.0)
    assert_close(got[:, 0], ref, what="attention over converted pages")


# ------------------------------------------------------------ a32 reference backend

@pytest.mark.parametrize("bits", [8, 4])
def test_quantized_attention_reference_backend(dev, bits):
    # the drop-in backend="reference" (ops/paged_quantized_kv_ops.py:469-515,
    # per-sequence lengths) on device tensors, against the oracle and the HIP
    # backend
    rng = np.random.default_rng(70 + bits)
    B, Hq, Hkv, D, P, mb, g = 3, 8, 2, 64, 16, 5, 32
    NP = B * mb + 1
    K = rng.standard_normal((NP, P, Hkv, D)).astype(np.float16)
    V = rng.standard_normal((NP, P, Hkv, D)).astype(np.float16)
    bt = rng.permutation(NP)[:B * mb].astype(np.int32).reshape(B, mb)
    lengths = np.array([1, 40, 80], np.int32)
    kq, vq, ks, vs = op.quantize_pages(K, V, g, bits)
    cache = pq.PagedQuantizedKVCache(k_pages_q=to_dev(kq, dev), v_pages_q=to_dev(vq, dev), k_scales=to_dev(ks, dev),
                                     v_scales=to_dev(vs, dev), block_table=to_dev(bt, dev),
                                     lengths=to_dev(lengths, dev), bits=bits, page_size=P, group_size=g,
                                     original_page_shape=K.shape)
    q = to_dev(rng.standard_normal((B, 1, Hq, D)).astype(np.float16), dev)
    ref_b = pq.paged_quantized_kv_gqa_decode_attention(q, cache)  # default backend "reference"
    hip = pq.paged_quantized_kv_gqa_decode_attention(q, cache, backend=f"metal_q{bits}")
    ref = op.quantized_paged_attention(q[:, 0].float().cpu().numpy(), kq, vq, ks, vs, bt, lengths, g, bits)
    assert tuple(ref_b.shape) == (B, 1, Hq, D) and ref_b.dtype == torch.float16
    assert_close(ref_b[:, 0], ref, what="reference backend")
    assert_close(hip[:, 0], ref, what="HIP backend")
    with pytest.raises(ValueError, match="metal_q8 backend requires bits=8|metal_q4 backend requires bits=4"):
        pq.paged_quantized_kv_gqa_decode_attention(q, cache, backend=f"metal_q{12 - bits}")
