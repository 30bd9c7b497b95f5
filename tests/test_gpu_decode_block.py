"""The two decode-block callers from a packed qkv row on the GPU:
``paged_decode_block_from_qkv`` (ops/decode_block_ops.py:198-257; MHA on the
pages, or routed to the paged GQA block when H differs from the cache's head
count) and ``gqa_decode_block_from_qkv`` (ops/gqa_ops.py:391-444, contiguous
cache).  Each is checked against the oracle's composition of the same steps
-- split + RoPE, the cache write, decode attention over position + 1 --
with the cache bytes bit-exact and the attention output at rtol 1e-2 / atol
1e-3 (fp16; 3e-2 / 4e-3 for bf16, whose q and values carry 8 mantissa bits)."""

import numpy as np
import pytest
import torch

import mk.decode_block_ops as dbo
import mk.gqa_ops as gqa
from oracle import paged as op
from oracle.quant import round_bf16
from tests._data import assert_close, to_dev

pytestmark = pytest.mark.gpu


def _tol(dtype):
    return dict(rtol=1e-2, atol=1e-3) if dtype == torch.float16 else dict(rtol=3e-2, atol=4e-3)


def _round(a, dtype):
    """Round fp32 values to the device dtype, kept as float32."""
    return a.astype(np.float16).astype(np.float32) if dtype == torch.float16 else round_bf16(a.astype(np.float32))


def _oracle_block(x, cos, sin, pos, bt, K0, V0, Hq, Hkv, D, dtype):
    """Oracle composition in float32 on values that are already device-dtype:
    split + RoPE (each rotated value rounded to the dtype, as the reference's
    rope returns it), the paged scatter, attention over pos + 1."""
    q, k, v = op.qkv_split_rope(x, cos, sin, pos, Hq, Hkv, D)
    q, k = _round(q, dtype), _round(k, dtype)
    K1, V1 = op.paged_kv_update(K0, V0, k, v, bt, pos)
    return q, K1, V1, op.paged_attention(q, K1, V1, bt, np.asarray(pos) + 1)


def _pages(rng, NP, P, H, D, dev, dtype):
    K = to_dev(rng.standard_normal((NP, P, H, D)).astype(np.float32), dev, dtype)
    V = to_dev(rng.standard_normal((NP, P, H, D)).astype(np.float32), dev, dtype)
    return K, V


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("layout", ["packed", "explicit"])
@pytest.mark.parametrize("B,H,D,P,mb,int_pos", [(3, 8, 128, 16, 8, False), (2, 4, 64, 8, 5, True),
                                                 (1, 32, 128, 16, 130, False), (4, 2, 16, 4, 3, False)])
def test_paged_decode_block_mha(dev, dtype, layout, B, H, D, P, mb, int_pos):
    rng = np.random.default_rng(B * 1000 + H * 10 + D + mb)
    NP = B * mb + 3
    Kp, Vp = _pages(rng, NP, P, H, D, dev, dtype)
    bt = rng.permutation(NP)[:B * mb].astype(np.int32).reshape(B, mb)
    pos = rng.integers(0, mb * P, size=B)
    pos[0] = mb * P - 1  # the last slot of the table
    if int_pos:
        pos[:] = pos[0]
    qkv_flat = rng.standard_normal((B, 1, 3 * H * D)).astype(np.float32)
    qkv = to_dev(qkv_flat, dev, dtype)
    if layout == "explicit":
        qkv = qkv.reshape(B, 1, 3, H, D)
    cos, sin = op.rope_tables(mb * P, D, 10000.0)
    K0, V0 = Kp.float().cpu().numpy(), Vp.float().cpu().numpy()
    position = int(pos[0]) if int_pos else to_dev(pos, dev)
    kw = dict(H=H, D=D) if layout == "packed" else {}
    out, K1, V1 = dbo.paged_decode_block_from_qkv(qkv, Kp, Vp, to_dev(bt, dev), torch.from_numpy(cos),
                                                  torch.from_numpy(sin), position, **kw)
    assert K1 is Kp and V1 is Vp and tuple(out.shape) == (B, 1, H, D) and out.dtype == dtype
    x = qkv.reshape(B, -1).float().cpu().numpy()
    _, rK, rV, ref = _oracle_block(x, cos, sin, pos, bt, K0, V0, H, H, D, dtype)
    assert np.array_equal(K1.float().cpu().numpy(), rK) and np.array_equal(V1.float().cpu().numpy(), rV)
    assert_close(out[:, 0], ref, what=f"mha block {layout} B{B} H{H} D{D}", **_tol(dtype))


@pytest.mark.parametrize("Hq,Hkv,D", [(32, 8, 128), (8, 1, 64)])
def test_paged_decode_block_routes_gqa(dev, Hq, Hkv, D):
    """H given and unequal to the cache's heads: the GQA block runs, with
    head_dim taken from the pages when D is not given."""
    rng = np.random.default_rng(Hq + Hkv + D)
    B, P, mb = 3, 16, 6
    NP = B * mb
    Kp, Vp = _pages(rng, NP, P, Hkv, D, dev, torch.float16)
    bt = rng.permutation(NP).astype(np.int32).reshape(B, mb)
    pos = rng.integers(0, mb * P, size=B)
    qkv = to_dev(rng.standard_normal((B, 1, (Hq + 2 * Hkv) * D)).astype(np.float16), dev)
    cos, sin = op.rope_tables(mb * P, D, 500000.0)
    K0, V0 = Kp.float().cpu().numpy(), Vp.float().cpu().numpy()
    out, K1, V1 = dbo.paged_decode_block_from_qkv(qkv, Kp, Vp, to_dev(bt, dev), torch.from_numpy(cos),
                                                  torch.from_numpy(sin), to_dev(pos, dev), H=Hq)
    assert tuple(out.shape) == (B, 1, Hq, D)
    _, rK, rV, ref = _oracle_block(qkv[:, 0].float().cpu().numpy(), cos, sin, pos, bt, K0, V0, Hq, Hkv, D,
                                   torch.float16)
    assert np.array_equal(K1.float().cpu().numpy(), rK) and np.array_equal(V1.float().cpu().numpy(), rV)
    assert_close(out[:, 0], ref, what=f"gqa route Hq{Hq} Hkv{Hkv}")


def test_paged_decode_block_reference_backend_agrees(dev):
    """backend='reference' (tensor ops, functional update) and the HIP block
    give the same caches bit for bit and the same output to tolerance; the
    reference backend leaves its inputs alone."""
    rng = np.random.default_rng(5)
    B, H, D, P, mb = 2, 4, 64, 16, 4
    NP = B * mb
    Kp, Vp = _pages(rng, NP, P, H, D, dev, torch.float16)
    Kr, Vr = Kp.clone(), Vp.clone()
    bt = to_dev(rng.permutation(NP).astype(np.int32).reshape(B, mb), dev)
    qkv = to_dev(rng.standard_normal((B, 1, 3 * H * D)).astype(np.float16), dev)
    cos, sin = (torch.from_numpy(t) for t in op.rope_tables(mb * P, D, 10000.0))
    pos = to_dev(np.array([7, 63]), dev)
    ref_out, rK, rV = dbo.paged_decode_block_from_qkv(qkv, Kr, Vr, bt, cos, sin, pos, H=H, D=D, backend="reference")
    assert torch.equal(Kr, Kp) and rK is not Kr
    out, K1, V1 = dbo.paged_decode_block_from_qkv(qkv, Kp, Vp, bt, cos, sin, pos, H=H, D=D)
    assert torch.equal(K1, rK) and torch.equal(V1, rV)
    assert_close(out[:, 0], ref_out[:, 0].float().cpu().numpy(), what="hip vs reference backend", extra=1e-3)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("B,Hq,Hkv,D,S,int_pos", [(3, 32, 8, 128, 2048, False), (2, 8, 2, 64, 100, True),
                                                  (2, 4, 4, 32, 37, False), (1, 16, 1, 128, 8192, True)])
def test_gqa_decode_block_contiguous(dev, dtype, B, Hq, Hkv, D, S, int_pos):
    """Contiguous cache [B, MAX_S, Hkv, D] (MAX_S 100 and 37 view as pages of
    4 and 1 positions): in-place write of the roped k / v at row pos[b], then
    GQA attention over pos + 1."""
    rng = np.random.default_rng(S + D + Hq)
    K = to_dev(rng.standard_normal((B, S, Hkv, D)).astype(np.float32), dev, dtype)
    V = to_dev(rng.standard_normal((B, S, Hkv, D)).astype(np.float32), dev, dtype)
    pos = np.full(B, S - 1) if int_pos else rng.integers(0, S, size=B)
    qkv = to_dev(rng.standard_normal((B, 1, (Hq + 2 * Hkv) * D)).astype(np.float32), dev, dtype)
    cos, sin = op.rope_tables(S, D, 500000.0)
    K0, V0 = K.float().cpu().numpy(), V.float().cpu().numpy()
    position = int(pos[0]) if int_pos else to_dev(pos, dev)
    out, K1, V1 = gqa.gqa_decode_block_from_qkv(qkv, K, V, torch.from_numpy(cos), torch.from_numpy(sin), position,
                                                num_attention_heads=Hq, num_key_value_heads=Hkv, head_dim=D)
    assert K1 is K and V1 is V and tuple(out.shape) == (B, 1, Hq, D)
    q, k, v = op.qkv_split_rope(qkv[:, 0].float().cpu().numpy(), cos, sin, pos, Hq, Hkv, D)
    q, k = _round(q, dtype), _round(k, dtype)
    rK, rV = op.contiguous_update(K0, V0, k, v, pos)
    assert np.array_equal(K1.float().cpu().numpy(), rK) and np.array_equal(V1.float().cpu().numpy(), rV)
    assert_close(out[:, 0], op.contiguous_attention(q, rK, rV, pos + 1), what=f"contiguous gqa block S{S}",
                 **_tol(dtype))
