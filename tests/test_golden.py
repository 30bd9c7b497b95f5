"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle re-derives every stored output from the stored inputs
(bit-exact for integer/byte work and elementwise float; matmul-based outputs
to a tight tolerance, since BLAS may sum in another order).
GPU: the HIP path, called through the drop-in API, reproduces the stored
outputs to the same bar as the other parity tests.
"""

import os

import numpy as np
import pytest
import torch

from oracle import paged as op
from oracle import quant as oq
from tests._data import assert_close, to_dev

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    with np.load(os.path.join(GOLDEN, f"{name}.npz")) as f:
        return {k: f[k] for k in f.files}


def _bits_equal(a, b):
    a, b = np.asarray(a), np.asarray(b)
    return a.shape == b.shape and a.dtype == b.dtype and np.array_equal(a.view(np.uint8), b.view(np.uint8))


# ------------------------------------------------------------------ CPU: oracle vs fixtures


def test_oracle_reproduces_quant_fixtures():
    f = _load("q4_pack")
    assert _bits_equal(oq.pack_q4(f["codes"]), f["packed"])
    assert _bits_equal(oq.unpack_q4(f["packed"], 33), f["codes"])
    d = _load("dequant")
    assert _bits_equal(oq.dequant_q4(d["q4_packed"], d["q4_scales"], d["q4_zeros"], 32), d["q4_out"])
    assert _bits_equal(oq.dequant_q8(d["q8_codes"], d["q8_scales"], d["q8_zeros"], 32), d["q8_out"])
    for bits in (4, 8):
        m = _load(f"q{bits}_matvec_llama_slice")
        w, s = oq.quantize_weight_groupwise(m["W_fp32_rows"], bits, 64)
        assert _bits_equal(w, m["weight"][:8]) and _bits_equal(s, m["scales_fp32_rows"])
        mv = oq.q4_matvec if bits == 4 else oq.q8_matvec
        y = mv(m["x"], m["weight"], m["scales"].astype(np.float32), m["zeros"].astype(np.float32), 64)
        assert_close(y.astype(np.float32), m["y"].astype(np.float32), rtol=1e-3, atol=1e-4, what=f"q{bits} slice")


def test_oracle_reproduces_mlp_fixture():
    f = _load("q4_mlp_block")
    trip = lambda n: (f[f"{n}_w"], f[f"{n}_s"].astype(np.float32), f[f"{n}_z"].astype(np.float32))  # noqa: E731
    out, inter = oq.mlp_block(f["x"], f["residual"], f["norm_w"], trip("gate"), trip("up"), trip("down"), bits=4,
                              group_size=64, intermediates=True)
    assert _bits_equal(inter["z"], f["i_z"])
    assert_close(out.astype(np.float32), f["out"].astype(np.float32), rtol=1e-3, atol=1e-4, what="mlp out")


def test_oracle_reproduces_paged_fixtures():
    f = _load("paged_gqa")
    page, off = op.block_table_lookup(f["block_table"], f["positions"], 16)
    assert _bits_equal(page, f["page"]) and _bits_equal(off, f["offset"])
    K2, V2 = op.paged_kv_update(f["K_pages"], f["V_pages"], f["k_new"], f["v_new"], f["block_table"], f["positions"])
    assert _bits_equal(K2, f["K_updated"]) and _bits_equal(V2, f["V_updated"])
    att = op.paged_attention(f["q"], f["K_pages"], f["V_pages"], f["block_table"], f["lengths"])
    assert np.allclose(att, f["attention"], rtol=1e-9, atol=1e-12)
    r = _load("qkv_rope_update")
    q_r, K3, V3 = op.qkv_rope_paged_update(r["qkv"], r["cos"], r["sin"], f["positions"], f["block_table"],
                                           f["K_pages"], f["V_pages"], 8, 2, 64)
    assert _bits_equal(q_r, r["q_rope"]) and _bits_equal(K3, r["K_updated"]) and _bits_equal(V3, r["V_updated"])
    for bits in (8, 4):
        qf = _load(f"paged_q{bits}")
        kq, vq, ks, vs = op.quantize_pages(f["K_pages"], f["V_pages"], 32, bits)
        for a, k in ((kq, "k_q"), (vq, "v_q"), (ks, "k_s"), (vs, "v_s")):
            assert _bits_equal(a, qf[k]), (bits, k)
        res = op.qkv_rope_paged_update_quant(r["qkv"], r["cos"], r["sin"], f["positions"], f["block_table"], kq, vq,
                                             ks, vs, 8, 2, 64, 32, bits)
        for a, k in zip(res[1:], ("k_q_updated", "v_q_updated", "k_s_updated", "v_s_updated")):
            assert _bits_equal(a, qf[k]), (bits, k)


# ------------------------------------------------------------------ GPU: HIP vs fixtures


@pytest.mark.gpu
def test_hip_quant_fixtures(dev):
    import mk.quant_ops as qo

    f = _load("q4_pack")
    assert _bits_equal(qo.pack_q4(to_dev(f["codes"], dev)).cpu().numpy(), f["packed"])
    d = _load("dequant")
    got4 = qo.dequant_q4(to_dev(d["q4_packed"], dev), to_dev(d["q4_scales"], dev), to_dev(d["q4_zeros"], dev),
                         group_size=32)
    assert _bits_equal(got4.cpu().numpy(), d["q4_out"])
    got8 = qo.dequant_q8(to_dev(d["q8_codes"], dev), to_dev(d["q8_scales"], dev), to_dev(d["q8_zeros"], dev),
                         group_size=32)
    assert _bits_equal(got8.cpu().numpy(), d["q8_out"])
    for bits in (4, 8):
        m = _load(f"q{bits}_matvec_llama_slice")
        fn = qo.q4_matvec_decode if bits == 4 else qo.q8_matvec_decode
        for M in (1, 4):
            y = fn(to_dev(m["x"][:M], dev), to_dev(m["weight"], dev), to_dev(m["scales"], dev),
                   to_dev(m["zeros"], dev), group_size=64)
            assert_close(y, m["y"][:M].astype(np.float32), what=f"q{bits} slice M={M}")


@pytest.mark.gpu
def test_hip_mlp_fixture(dev):
    import mk.mlp_block_ops as mlp

    f = _load("q4_mlp_block")
    t = lambda k: to_dev(f[k], dev)  # noqa: E731
    out = mlp.quantized_mlp_block(t("x")[:, None], t("residual")[:, None], t("norm_w"), t("gate_w"), t("gate_s"),
                                  t("up_w"), t("up_s"), t("down_w"), t("down_s"), gate_zeros=t("gate_z"),
                                  up_zeros=t("up_z"), down_zeros=t("down_z"), bits=4, group_size=64,
                                  backend_preset="fused_experimental")
    # the kernels see the same rounded intermediates as the oracle up to one
    # fp16 ulp of the down projection, added to the residual
    ulp = np.abs(f["i_down"].astype(np.float32)) * 2.0 ** -10
    assert_close(out[:, 0], f["out"].astype(np.float32), what="q4 MLP block", extra=4 * ulp + 1e-3)


@pytest.mark.gpu
def test_hip_paged_fixtures(dev):
    import mk.gqa_ops as gqa
    import mk.paged_kv_ops as pk

    f = _load("paged_gqa")
    bt = to_dev(f["block_table"], dev)
    page, off = pk.block_table_lookup(bt, to_dev(f["positions"], dev), 16, backend="metal")
    assert _bits_equal(page.cpu().numpy(), f["page"]) and _bits_equal(off.cpu().numpy(), f["offset"])
    q = to_dev(f["q"], dev)[:, None]
    att = gqa.paged_gqa_decode_attention(q, to_dev(f["K_pages"], dev), to_dev(f["V_pages"], dev), bt,
                                         to_dev(f["lengths"], dev))
    assert_close(att[:, 0], f["attention"], what="paged GQA attention")
    att_h = gqa.paged_gqa_decode_attention(q, to_dev(f["K_pages"], dev), to_dev(f["V_pages"], dev),
                                           to_dev(f["block_table_holes"], dev),
                                           to_dev(np.array([1, 37, 20], np.int32), dev))
    assert_close(att_h[:, 0], f["attention_holes"], what="paged GQA attention, unmapped block")
    Kp, Vp = to_dev(f["K_pages"], dev), to_dev(f["V_pages"], dev)
    K2, V2 = pk.paged_kv_cache_update(Kp, Vp, to_dev(f["k_new"], dev), to_dev(f["v_new"], dev), bt,
                                      to_dev(f["positions"], dev))
    assert _bits_equal(K2.cpu().numpy(), f["K_updated"]) and _bits_equal(V2.cpu().numpy(), f["V_updated"])

    r = _load("qkv_rope_update")
    Kp, Vp = to_dev(f["K_pages"], dev), to_dev(f["V_pages"], dev)
    out, K3, V3 = gqa.paged_gqa_decode_block_from_qkv(
        to_dev(r["qkv"], dev)[:, None], Kp, Vp, bt, torch.from_numpy(r["cos"]), torch.from_numpy(r["sin"]),
        to_dev(f["positions"], dev), num_attention_heads=8, num_key_value_heads=2, head_dim=64)
    assert _bits_equal(K3.cpu().numpy(), r["K_updated"]) and _bits_equal(V3.cpu().numpy(), r["V_updated"])
    ref = op.paged_attention(r["q_rope"], r["K_updated"], r["V_updated"], f["block_table"], f["positions"] + 1)
    assert_close(out[:, 0], ref, what="decode block from qkv")


@pytest.mark.gpu
@pytest.mark.parametrize("bits", [8, 4])
def test_hip_quantized_kv_fixtures(dev, bits):
    import mk.paged_quantized_kv_ops as pq

    f = _load("paged_gqa")
    r = _load("qkv_rope_update")
    qf = _load(f"paged_q{bits}")
    c = pq.quantize_kv_pages(to_dev(f["K_pages"], dev), to_dev(f["V_pages"], dev), to_dev(f["block_table"], dev),
                             to_dev(f["lengths"], dev), pq.PagedQuantizedKVConfig(bits=bits, page_size=16,
                                                                                 group_size=32))
    for a, k in ((c.k_pages_q, "k_q"), (c.v_pages_q, "v_q"), (c.k_scales, "k_s"), (c.v_scales, "v_s")):
        assert _bits_equal(a.cpu().numpy(), qf[k]), k
    got = pq.paged_quantized_kv_gqa_decode_attention(to_dev(f["q"], dev)[:, None], c, backend=f"metal_q{bits}")
    assert_close(got[:, 0], qf["attention"], what=f"q{bits} paged attention")
    q_out, c = pq.paged_quantized_kv_update_from_qkv(
        to_dev(r["qkv"], dev)[:, None], c, torch.from_numpy(r["cos"]), torch.from_numpy(r["sin"]),
        f["positions"].tolist(), num_attention_heads=8, num_key_value_heads=2, head_dim=64)
    assert _bits_equal(q_out[:, 0].cpu().numpy(), qf["q_rope"])
    for a, k in ((c.k_pages_q, "k_q_updated"), (c.v_pages_q, "v_q_updated"), (c.k_scales, "k_s_updated"),
                 (c.v_scales, "v_s_updated")):
        assert _bits_equal(a.cpu().numpy(), qf[k]), k
