"""Host (CPU tensor) side of the decode-block callers from a packed qkv row:
``paged_decode_block_from_qkv`` (ops/decode_block_ops.py:174-257) and
``gqa_decode_block_from_qkv`` (ops/gqa_ops.py:345-444).  Their 'reference'
backends against the oracle's composition, the MHA/GQA routing, and the
validation messages the reference raises.  No GPU."""

import numpy as np
import pytest
import torch

import mk.decode_block_ops as dbo
import mk.gqa_ops as gqa
from oracle import paged as op
from tests._data import assert_close


def _f16(a):
    return a.astype(np.float16).astype(np.float32)


def _case(seed, B, H, D, P, mb):
    rng = np.random.default_rng(seed)
    NP = B * mb
    Kp = rng.standard_normal((NP, P, H, D)).astype(np.float16)
    Vp = rng.standard_normal((NP, P, H, D)).astype(np.float16)
    bt = rng.permutation(NP).astype(np.int32).reshape(B, mb)
    pos = rng.integers(0, mb * P, size=B)
    return rng, Kp, Vp, bt, pos


@pytest.mark.parametrize("layout", ["packed", "explicit"])
@pytest.mark.parametrize("int_pos", [False, True])
def test_reference_paged_block_mha_matches_oracle(layout, int_pos):
    B, H, D, P, mb = 3, 4, 16, 4, 3
    rng, Kp, Vp, bt, pos = _case(11, B, H, D, P, mb)
    if int_pos:
        pos[:] = 5
    qkv = rng.standard_normal((B, 1, 3 * H * D)).astype(np.float16)
    cos, sin = op.rope_tables(mb * P, D, 10000.0)
    t = torch.from_numpy
    q_in = t(qkv) if layout == "packed" else t(qkv).reshape(B, 1, 3, H, D)
    kw = dict(H=H, D=D) if layout == "packed" else {}
    position = 5 if int_pos else t(pos)
    out, K1, V1 = dbo.paged_decode_block_from_qkv(q_in, t(Kp), t(Vp), t(bt), t(cos), t(sin), position,
                                                  backend="reference", **kw)
    q, k, v = op.qkv_split_rope(qkv[:, 0], cos, sin, pos, H, H, D)
    rK, rV = op.paged_kv_update(Kp, Vp, k, v, bt, pos)
    assert np.array_equal(K1.numpy(), rK) and np.array_equal(V1.numpy(), rV)
    ref = op.paged_attention(q.astype(np.float32), rK, rV, bt, pos + 1)
    assert_close(out[:, 0], ref, what="reference paged block", extra=1e-3)
    assert tuple(out.shape) == (B, 1, H, D) and out.dtype == torch.float16


def test_reference_paged_block_routes_gqa():
    B, Hq, Hkv, D, P, mb = 2, 8, 2, 16, 4, 3
    rng, Kp, Vp, bt, pos = _case(12, B, Hkv, D, P, mb)
    qkv = rng.standard_normal((B, 1, (Hq + 2 * Hkv) * D)).astype(np.float16)
    cos, sin = op.rope_tables(mb * P, D, 500000.0)
    t = torch.from_numpy
    out, K1, _ = dbo.paged_decode_block_from_qkv(t(qkv), t(Kp), t(Vp), t(bt), t(cos), t(sin), t(pos), H=Hq,
                                                 backend="reference")
    q, k, v = op.qkv_split_rope(qkv[:, 0], cos, sin, pos, Hq, Hkv, D)
    rK, rV = op.paged_kv_update(Kp, Vp, k, v, bt, pos)
    assert np.array_equal(K1.numpy(), rK)
    assert_close(out[:, 0], op.paged_attention(q.astype(np.float32), rK, rV, bt, pos + 1), what="gqa route",
                 extra=1e-3)


def test_reference_contiguous_gqa_block_matches_oracle():
    B, Hq, Hkv, D, S = 2, 8, 2, 16, 24
    rng = np.random.default_rng(13)
    K = rng.standard_normal((B, S, Hkv, D)).astype(np.float16)
    V = rng.standard_normal((B, S, Hkv, D)).astype(np.float16)
    qkv = rng.standard_normal((B, 1, (Hq + 2 * Hkv) * D)).astype(np.float16)
    cos, sin = op.rope_tables(S, D, 500000.0)
    pos = np.array([0, 23])
    t = torch.from_numpy
    for fn in (gqa.reference_gqa_decode_block_from_qkv,
               lambda *a, **k: gqa.gqa_decode_block_from_qkv(*a, backend="reference", **k)):
        Kt, Vt = t(K.copy()), t(V.copy())
        out, K1, V1 = fn(t(qkv), Kt, Vt, t(cos), t(sin), t(pos), num_attention_heads=Hq, num_key_value_heads=Hkv,
                         head_dim=D)
        assert np.array_equal(Kt.numpy(), K)  # functional: the inputs stay
        q, k, v = op.qkv_split_rope(qkv[:, 0], cos, sin, pos, Hq, Hkv, D)
        rK, rV = op.contiguous_update(K, V, k, v, pos)
        assert np.array_equal(K1.numpy(), rK) and np.array_equal(V1.numpy(), rV)
        assert_close(out[:, 0], op.contiguous_attention(q.astype(np.float32), rK, rV, pos + 1),
                     what="contiguous gqa block", extra=1e-3)


def test_paged_block_validation_messages():
    t = torch.zeros
    K = t(6, 4, 2, 16, dtype=torch.float16)
    bt = torch.zeros(2, 3, dtype=torch.int32)
    cos = sin = t(12, 8)
    qkv = t(2, 1, 3 * 2 * 16, dtype=torch.float16)
    with pytest.raises(ValueError, match="K_pages and V_pages must be matching"):
        dbo.paged_decode_block_from_qkv(qkv, K, K[:, :2], bt, cos, sin, 0, H=2, D=16)
    with pytest.raises(ValueError, match="block_table must be"):
        dbo.paged_decode_block_from_qkv(qkv, K, K, bt[0], cos, sin, 0, H=2, D=16)
    with pytest.raises(ValueError, match="H and D are required"):
        dbo.paged_decode_block_from_qkv(qkv, K, K, bt, cos, sin, 0)
    with pytest.raises(ValueError, match="3\\*H\\*D"):
        dbo.paged_decode_block_from_qkv(qkv[..., :-16], K, K, bt, cos, sin, 0, H=2, D=16)
    with pytest.raises(TypeError, match="qkv dtype"):
        dbo.paged_decode_block_from_qkv(qkv.float(), K, K, bt, cos, sin, 0, H=2, D=16)
    # the reference's split step takes only these names; its attention step rejects the GQA ones
    with pytest.raises(ValueError, match="'reference', 'metal', 'auto'"):
        dbo.paged_decode_block_from_qkv(qkv, K, K, bt, cos, sin, 0, H=2, D=16, backend="metal_threadgroup")
    with pytest.raises(ValueError, match="metal_d128"):
        dbo.paged_decode_block_from_qkv(qkv, K, K, bt, cos, sin, 0, H=2, D=16, backend="metal_gqa")
    with pytest.raises(ValueError, match="must normalize to"):
        dbo.paged_decode_block_from_qkv(t(2, 1, 3, 2, 8, dtype=torch.float16), K, K, bt, cos, sin, 0)
    with pytest.raises(ValueError, match="metal_gqa_threadgroup"):  # GQA route, unknown backend
        dbo.paged_decode_block_from_qkv(qkv, K, K, bt, cos, sin, 0, H=4, D=16, backend="bogus")


def test_contiguous_gqa_block_validation_messages():
    K = torch.zeros(2, 8, 2, 16, dtype=torch.float16)
    qkv = torch.zeros(2, 1, 8 * 16, dtype=torch.float16)
    cos = sin = torch.zeros(8, 8)
    kw = dict(num_attention_heads=4, num_key_value_heads=2, head_dim=16)
    with pytest.raises(ValueError, match="metal_gqa_threadgroup"):
        gqa.gqa_decode_block_from_qkv(qkv, K, K, cos, sin, 0, backend="metal_d64", **kw)
    with pytest.raises(ValueError, match="divisible"):
        gqa.gqa_decode_block_from_qkv(qkv, K, K, cos, sin, 0, num_attention_heads=3, num_key_value_heads=2,
                                      head_dim=16)
    with pytest.raises(ValueError, match="matching"):
        gqa.gqa_decode_block_from_qkv(qkv, K, K[:1], cos, sin, 0, **kw)
    with pytest.raises(ValueError, match="cache batch/head/head_dim"):
        gqa.gqa_decode_block_from_qkv(qkv[:1], K, K, cos, sin, 0, **kw)
