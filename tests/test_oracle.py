"""Pins the CPU oracle against the reference tests' known answers, closed
forms, invariants and brute-force loops (no GPU, no torch)."""

import math

import numpy as np
import pytest

from oracle import paged as op
from oracle import quant as oq


# ------------------------------------------------------------ pack / unpack

def test_pack_q4_known_answers():
    # low nibble = even column (ops/quant_ops.py:172-175)
    assert oq.pack_q4(np.array([[1, 2]])).tolist() == [[0x21]]
    assert oq.pack_q4(np.array([[15, 0, 3]])).tolist() == [[0x0F, 0x03]]
    assert oq.unpack_q4(np.array([[0xA5]], dtype=np.uint8)).tolist() == [[5, 10]]


def test_pack_unpack_roundtrip_reference_shape():
    # tests/test_quant_ops.py:20-26: pack then unpack (K=64) returns the codes
    q = np.random.default_rng(60).integers(0, 16, size=(4, 64), dtype=np.uint8)
    assert np.array_equal(oq.unpack_q4(oq.pack_q4(q), 64), q)


def test_pack_little_endian_word_view():
    # 8 nibbles per uint32, nibble i at bits 4i -- the layout the kernels load
    q = np.arange(8, dtype=np.uint8)[None, :]
    word = oq.pack_q4(q).view("<u4")[0, 0]
    assert [(int(word) >> (4 * i)) & 15 for i in range(8)] == list(range(8))


# ------------------------------------------------------------ dequant

def test_dequant_identity_and_zero_point():
    q = np.random.default_rng(1).integers(0, 16, size=(3, 64), dtype=np.uint8)
    ones = np.ones((3, 2), np.float32)
    assert np.array_equal(oq.dequant(q, ones, None, 32).astype(np.float32), q.astype(np.float32))
    z = np.full((3, 2), 8.0, np.float32)
    assert np.array_equal(oq.dequant(q, ones, z, 32).astype(np.float32), q.astype(np.float32) - 8)


def test_dequant_group_boundaries():
    # K=80, g=32 -> 3 groups, the last one partial: each column must use the
    # scale of group k // 32
    q = np.ones((1, 80), dtype=np.uint8)
    s = np.array([[1.0, 2.0, 4.0]], np.float32)
    w = oq.dequant(q, s, None, 32).astype(np.float32)[0]
    assert np.all(w[:32] == 1) and np.all(w[32:64] == 2) and np.all(w[64:] == 4)


def test_dequant_single_rounding_fp16():
    # (q - z) * s is formed in fp32 then rounded once: pick s so the product
    # needs rounding and compare with Python's exact arithmetic + one RNE step
    q = np.array([[3, 13]], dtype=np.uint8)
    s = np.array([[0.1]], np.float32)
    z = np.array([[0.3]], np.float32)
    got = oq.dequant(q, s, z, 64)
    for j in range(2):
        exact = (float(q[0, j]) - float(z[0, 0])) * float(s[0, 0])
        assert abs(float(got[0, j]) - exact) <= 2.0 ** -11 * abs(exact) + 1e-7


# ------------------------------------------------------------ matvec

def _metal_scalar_matvec(x, codes, s, z, g):
    """Brute force mirroring kernels/q4_matvec_decode.metal: one serial loop
    per output, w = (q - z) * s, fp64 accumulation."""
    M, K = x.shape
    N = codes.shape[0]
    y = np.zeros((M, N))
    for m in range(M):
        for n in range(N):
            acc = 0.0
            for k in range(K):
                w = (float(codes[n, k]) - (float(z[n, k // g]) if z is not None else 0.0)) * float(s[n, k // g])
                acc += float(x[m, k]) * w
            y[m, n] = acc
    return y


@pytest.mark.parametrize("with_zero", [False, True])
def test_q4_matvec_matches_scalar_kernel_loop(with_zero):
    rng = np.random.default_rng(3)
    M, N, K, g = 2, 5, 96, 32
    codes = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    s = (rng.standard_normal((N, K // g)) * 0.1).astype(np.float32)
    z = rng.uniform(0, 15, (N, K // g)).astype(np.float32) if with_zero else None
    x = rng.standard_normal((M, K)).astype(np.float16)
    got = oq.q4_matvec(x, oq.pack_q4(codes), s, z, g).astype(np.float64)
    ref = _metal_scalar_matvec(x, codes, s, z, g)
    assert np.allclose(got, ref, rtol=1e-2, atol=1e-2)


def test_matvec_one_hot_selects_weight_column():
    # x = e_k picks W[:, k]: pins the n/k orientation and the nibble order
    rng = np.random.default_rng(4)
    N, K, g = 6, 64, 32
    codes = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    s = rng.uniform(0.5, 1.0, (N, 2)).astype(np.float32)
    W = oq.dequant(codes, s, None, g)
    for k in (0, 1, 31, 32, 63):
        x = np.zeros((1, K), np.float16)
        x[0, k] = 1.0
        assert np.array_equal(oq.q4_matvec(x, oq.pack_q4(codes), s, None, g)[0], W[:, k])


def test_matvec_saturates():
    x = np.full((1, 64), 60000.0, np.float16)
    codes = np.full((2, 64), 15, np.uint8)
    s = np.ones((2, 1), np.float32)
    y = oq.q8_matvec(x, codes, s, None, 64)
    assert np.all(y == np.float16(65504.0))


# ------------------------------------------------------------ elementwise / block

def test_swiglu_closed_form():
    g = np.array([0.0, 1.0, -2.0, 30.0], np.float16)
    u = np.array([5.0, 2.0, 1.0, 1.0], np.float16)
    exp = [0.0, 2.0 / (1 + math.exp(-1.0)), -2.0 / (1 + math.exp(2.0)), 30.0]
    assert np.allclose(oq.swiglu(g, u).astype(np.float64), exp, rtol=1e-3)


def test_rms_norm_constant_row():
    x = np.full((1, 16), 3.0, np.float16)
    w = np.full((16,), 2.0, np.float16)
    y = oq.rms_norm(x, w, 1e-5).astype(np.float64)
    assert np.allclose(y, 2.0 * 3.0 / math.sqrt(9.0 + 1e-5), rtol=1e-3)


def test_rms_norm_eps_dominates_small_rows():
    """Rows of amplitude ~1e-3, where eps (1e-5, ops/norm_ops.py:47) is ten
    times mean(x^2): a constant row c gives c / sqrt(c^2 + eps) -- 0.30151
    for c = 1e-3 (without eps it would be 1.0, with eps 1e-6 0.7071) -- and
    the default eps is the reference's.  An all-zero row stays zero."""
    x = np.full((1, 64), 1e-3, np.float16)
    w = np.ones(64, np.float16)
    c = float(np.float16(1e-3))
    assert np.allclose(oq.rms_norm(x, w).astype(np.float64), c / math.sqrt(c * c + 1e-5), rtol=2e-3)
    assert np.allclose(oq.rms_norm(x, w).astype(np.float64), 0.30151, rtol=2e-3)
    # alternating signs: mean(x^2) is the same, the signs carry through
    xs = x * np.where(np.arange(64) % 2 == 0, 1, -1).astype(np.float16)
    ys = oq.rms_norm(xs, w).astype(np.float64)
    assert np.allclose(np.abs(ys), 0.30151, rtol=2e-3) and np.all(np.sign(ys) == np.sign(xs))
    assert np.array_equal(oq.rms_norm(np.zeros((2, 64), np.float16), w), np.zeros((2, 64), np.float16))


def test_mlp_block_zero_weights_is_residual_sum():
    rng = np.random.default_rng(5)
    D, I, g = 64, 128, 32
    x = rng.standard_normal((2, D)).astype(np.float16)
    r = rng.standard_normal((2, D)).astype(np.float16)
    w = np.ones(D, np.float16)
    zero_pt = lambda n, k: (oq.pack_q4(np.full((n, k), 8, np.uint8)), np.ones((n, k // g), np.float32),
                            np.full((n, k // g), 8.0, np.float32))
    out = oq.mlp_block(x, r, w, zero_pt(I, D), zero_pt(I, D), zero_pt(D, I), bits=4, group_size=g)
    assert np.array_equal(out, oq.residual_add(x, r))


def test_decode_layer_zero_projections_is_identity():
    """A layer whose projections all dequantize to 0 (codes at the zero
    point) returns its input exactly and writes k = v = 0 at the new slot."""
    from oracle import llama as ol

    rng = np.random.default_rng(8)
    B, H, Hq, Hkv, D, I, g, P, mb = 2, 64, 4, 2, 16, 128, 32, 4, 4
    zero_pt = lambda n, k: (oq.pack_q4(np.full((n, k), 8, np.uint8)), np.ones((n, k // g), np.float32),
                            np.full((n, k // g), 8.0, np.float32))
    w = {"qkv": zero_pt((Hq + 2 * Hkv) * D, H), "o": zero_pt(H, Hq * D), "gate": zero_pt(I, H),
         "up": zero_pt(I, H), "down": zero_pt(H, I), "ln1": np.ones(H, np.float16), "ln2": np.ones(H, np.float16)}
    K = rng.standard_normal((B * mb, P, Hkv, D)).astype(np.float16)
    V = rng.standard_normal((B * mb, P, Hkv, D)).astype(np.float16)
    bt = np.arange(B * mb, dtype=np.int32).reshape(B, mb)
    x = rng.standard_normal((B, H)).astype(np.float16)
    cos, sin = op.rope_tables(64, D, 500000.0)
    pos = [3, 9]
    out, K2, V2 = ol.layer_decode_step(x, w, K, V, bt, cos, sin, pos, Hq, Hkv, D)
    assert np.array_equal(out, x)
    for b, p in enumerate(pos):
        assert not K2[bt[b, p // P], p % P].any() and not V2[bt[b, p // P], p % P].any()
    keep = np.ones(K.shape[:2], bool)
    keep[[bt[b, p // P] for b, p in enumerate(pos)], [p % P for p in pos]] = False
    assert np.array_equal(K2[keep], K[keep]) and np.array_equal(V2[keep], V[keep])


# ------------------------------------------------------------ weight quantizer

def test_weight_quantizer_reference_shapes_and_error():
    # tests/test_quantize_weights.py:18-34
    w = np.random.default_rng(10).normal(size=(16, 64)).astype(np.float32)
    packed, s = oq.quantize_weight_groupwise(w, 4, 32)
    assert packed.shape == (16, 32) and s.shape == (16, 2)
    deq = oq.dequant_q4(packed, s, np.full_like(s, 8.0), 32, np.float32)
    rmse = float(np.sqrt(np.mean((deq - w) ** 2)))
    assert rmse < 0.25 and rmse / float(np.sqrt(np.mean(w * w))) < 0.25
    packed, s = oq.quantize_weight_groupwise(np.random.default_rng(11).normal(size=(16, 65)).astype(np.float32), 4, 32)
    assert packed.shape == (16, 33) and s.shape == (16, 3)


@pytest.mark.parametrize("bits", [4, 8])
def test_weight_quantizer_error_bound_and_tie_rule(bits):
    w = np.random.default_rng(12).normal(size=(8, 64)).astype(np.float32)
    codes, s = oq.quantize_weight_groupwise(w, bits, 32)
    zp = 8 if bits == 4 else 128
    deq = (oq.dequant_q4 if bits == 4 else oq.dequant_q8)(codes, s, np.full_like(s, zp), 32, np.float32)
    assert np.all(np.abs(deq - w) <= np.repeat(s, 32, axis=1) * 0.5 * (1 + 1e-6))
    # half-way value rounds to even: group max 7 -> scale 1, value 2.5 -> 2
    t = np.zeros((1, 32), np.float32)
    t[0, 0], t[0, 1] = 7.0 if bits == 4 else 127.0, 2.5
    c, _ = oq.quantize_weight_groupwise(t, bits, 32)
    c = oq.unpack_q4(c, 32) if bits == 4 else c
    assert int(c[0, 1]) - zp == 2


# ------------------------------------------------------------ paged plumbing

def test_block_table_lookup_reference_cases():
    # tests/test_paged_kv_cache.py:19-27 on the identity table
    bt = op.identity_block_table(1, 16, 4)
    assert [a.tolist() for a in op.block_table_lookup(bt, [3], 4)] == [[0], [3]]
    bt = op.identity_block_table(2, 32, 8)
    assert [a.tolist() for a in op.block_table_lookup(bt, [2, 17], 8)] == [[0, 6], [2, 1]]


def test_paged_update_touches_only_target_slots_and_later_b_wins():
    rng = np.random.default_rng(6)
    Kp = rng.standard_normal((6, 4, 2, 8)).astype(np.float16)
    Vp = rng.standard_normal((6, 4, 2, 8)).astype(np.float16)
    bt = np.array([[0, 1, 2], [0, 4, 5]], np.int32)
    k = rng.standard_normal((2, 2, 8)).astype(np.float16)
    v = rng.standard_normal((2, 2, 8)).astype(np.float16)
    K2, V2 = op.paged_kv_update(Kp, Vp, k, v, bt, [1, 1])  # both hit page 0 slot 1
    assert np.array_equal(K2[0, 1], k[1]) and np.array_equal(V2[0, 1], v[1])
    changed = (K2 != Kp).any(axis=(2, 3))
    assert changed.sum() == 1 and changed[0, 1]


def test_identity_paging_roundtrip():
    # tests/test_paged_quantized_kv_ops.py:277-295 (identity paging of [6, 8])
    rng = np.random.default_rng(15)
    K = rng.standard_normal((2, 8, 2, 16)).astype(np.float16)
    bt = op.identity_block_table(2, 8, 4)
    pages = K.reshape(2, 2, 4, 2, 16).reshape(4, 4, 2, 16)
    g, valid = op.gather(pages, bt, 8)
    assert valid.all() and np.array_equal(g, K)


# ------------------------------------------------------------ attention

def _online_softmax_scalar(q, K, V, n, scale):
    """Brute force mirroring kernels/paged_decode_attention.metal:43-57."""
    m, l = -math.inf, 0.0
    acc = np.zeros(q.shape[-1])
    for j in range(n):
        s = float(np.dot(q.astype(np.float64), K[j].astype(np.float64))) * scale
        m_new = max(m, s)
        alpha = math.exp(m - m_new) if math.isfinite(m) else 0.0
        beta = math.exp(s - m_new)
        l = l * alpha + beta
        acc = acc * alpha + beta * V[j].astype(np.float64)
        m = m_new
    return acc / max(l, 1e-20)


def _paged_case(seed, B=3, Hq=4, Hkv=2, D=16, P=4, mb=5):
    rng = np.random.default_rng(seed)
    NP = B * mb
    Kp = rng.standard_normal((NP, P, Hkv, D)).astype(np.float16)
    Vp = rng.standard_normal((NP, P, Hkv, D)).astype(np.float16)
    bt = rng.permutation(NP).astype(np.int32).reshape(B, mb)
    q = rng.standard_normal((B, Hq, D)).astype(np.float16)
    lengths = rng.integers(1, mb * P + 1, size=B)
    return q, Kp, Vp, bt, lengths


def test_paged_attention_matches_online_softmax_loop():
    q, Kp, Vp, bt, lengths = _paged_case(7)
    got = op.paged_attention(q, Kp, Vp, bt, lengths)
    K, _ = op.gather(Kp, bt, bt.shape[1] * Kp.shape[1])
    V, _ = op.gather(Vp, bt, bt.shape[1] * Kp.shape[1])
    for b in range(q.shape[0]):
        for h in range(q.shape[1]):
            ref = _online_softmax_scalar(q[b, h], K[b, :, h // 2], V[b, :, h // 2], lengths[b], 1 / math.sqrt(16))
            assert np.allclose(got[b, h], ref, rtol=1e-9, atol=1e-12)


def test_paged_attention_invariants():
    q, Kp, Vp, bt, lengths = _paged_case(8)
    base = op.paged_attention(q, Kp, Vp, bt, lengths)
    # physical page permutation leaves the result unchanged
    perm = np.random.default_rng(9).permutation(Kp.shape[0])
    inv = np.argsort(perm)
    same = op.paged_attention(q, Kp[perm], Vp[perm], inv[bt].astype(np.int32), lengths)
    assert np.array_equal(base, same)
    # length 1 returns V at position 0 of the head's kv head
    one = op.paged_attention(q, Kp, Vp, bt, np.ones_like(lengths))
    for b in range(q.shape[0]):
        for h in range(q.shape[1]):
            assert np.allclose(one[b, h], Vp[bt[b, 0], 0, h // 2].astype(np.float64))
    # GQA equals MHA over heads-expanded pages
    Kx = np.repeat(Kp, 2, axis=2)
    Vx = np.repeat(Vp, 2, axis=2)
    assert np.allclose(base, op.paged_attention(q, Kx, Vx, bt, lengths), rtol=1e-12, atol=1e-12)
    # zero keys give the mean of the valid values
    z = op.paged_attention(q, np.zeros_like(Kp), Vp, bt, lengths)
    V, _ = op.gather(Vp, bt, bt.shape[1] * Kp.shape[1])
    for b in range(q.shape[0]):
        assert np.allclose(z[b, 0], V[b, :lengths[b], 0].astype(np.float64).mean(axis=0))
    # no position -> zeros
    assert np.all(op.paged_attention(q, Kp, Vp, bt, np.zeros_like(lengths)) == 0)


# ------------------------------------------------------------ RoPE

def test_rope_tables_and_rotation():
    c, s = op.rope_tables(64, 16, 500000.0)
    assert np.allclose(c * c + s * s, 1.0, atol=1e-6)
    for pos in (0, 5, 63):
        for i in range(8):
            ang = pos * 500000.0 ** (-2 * i / 16)
            assert abs(c[pos, i] - math.cos(ang)) < 1e-5 and abs(s[pos, i] - math.sin(ang)) < 1e-5
    x = np.random.default_rng(2).standard_normal((3, 16)).astype(np.float16)
    assert np.array_equal(op.apply_rope(x, c[0], s[0]), x)  # angle 0
    y = op.apply_rope(x, c[7], s[7]).astype(np.float64)
    xx = x.astype(np.float64)
    assert np.allclose(y[:, 0::2] ** 2 + y[:, 1::2] ** 2, xx[:, 0::2] ** 2 + xx[:, 1::2] ** 2, rtol=3e-3)
    # interleaved pairs: pair (0,1) at 90 degrees maps (a, b) -> (-b, a)
    cq, sq = np.zeros(8, np.float32), np.ones(8, np.float32)
    t = np.arange(16, dtype=np.float16)[None]
    r = op.apply_rope(t, cq, sq)
    assert r[0, 0] == -1 and r[0, 1] == 0 and r[0, 2] == -3 and r[0, 3] == 2


# ------------------------------------------------------------ KV quantizer

@pytest.mark.parametrize("bits", [8, 4])
def test_kv_quantizer_bounds(bits):
    rng = np.random.default_rng(13)
    v = rng.standard_normal((5, 3, 128)).astype(np.float16)
    codes, s = op.quantize_groups(v, 64, bits)
    qmax, off = (127, 128) if bits == 8 else (7, 8)
    assert codes.min() >= off - qmax and codes.max() <= off + qmax
    deq = op.dequantize(codes, s, 64, bits).astype(np.float64)
    bound = np.repeat(np.abs(s.astype(np.float64)), 64, axis=-1) * (0.5 + 2.0 ** -10) + 1e-3
    assert np.all(np.abs(deq - v.astype(np.float64)) <= bound)
    # each group's max |v| lands on the extreme code
    g0 = np.abs(v[..., :64].astype(np.float32))
    at = np.argmax(g0, axis=-1)
    ext = np.take_along_axis(codes[..., :64].astype(int), at[..., None], -1)[..., 0]
    assert np.all(np.abs(ext - off) == qmax)
    # all-zero group: scale 1e-8/qmax, every code at the offset
    zc, zs = op.quantize_groups(np.zeros((1, 64), np.float16), 64, bits)
    assert np.all(zc == off) and np.isclose(float(zs[0, 0]), np.float16(1e-8 / qmax))


def test_quantized_attention_close_to_fp16():
    # tests/test_paged_quantized_kv_decode_reference.py tolerances 0.15 (q8) / 0.3 (q4)
    q, Kp, Vp, bt, lengths = _paged_case(14, D=64)
    ref = op.paged_attention(q, Kp, Vp, bt, lengths)
    for bits, tol in ((8, 0.15), (4, 0.3)):
        kq, vq, ks, vs = op.quantize_pages(Kp, Vp, 32, bits)
        got = op.quantized_paged_attention(q, kq, vq, ks, vs, bt, lengths, 32, bits)
        assert np.allclose(got, ref, atol=tol, rtol=tol)


def test_round_bf16_matches_torch_cast():
    # a library routine pins the bf16 rounding used by the bf16 matvec oracle
    torch = pytest.importorskip("torch")
    v = (np.random.default_rng(0).standard_normal(20000) * 300).astype(np.float32)
    v[:4] = [0.0, -0.0, 1e-40, 3.0e38]
    assert np.array_equal(oq.round_bf16(v), torch.from_numpy(v).to(torch.bfloat16).float().numpy())


# ------------------------------------------------------------ contiguous caches

def test_contiguous_attention_equals_identity_paged_and_scalar_loop():
    # a contiguous cache is the paged layout under the identity table
    # (ops/paged_kv_ops.py:99-105): the two statements must agree exactly
    rng = np.random.default_rng(30)
    B, S, Hq, Hkv, D, P = 3, 24, 4, 2, 16, 4
    K = rng.standard_normal((B, S, Hkv, D)).astype(np.float16)
    V = rng.standard_normal((B, S, Hkv, D)).astype(np.float16)
    q = rng.standard_normal((B, Hq, D)).astype(np.float16)
    lengths = np.array([1, 13, 40])  # the last one clips to MAX_S
    got = op.contiguous_attention(q, K, V, lengths)
    bt = op.identity_block_table(B, S, P)
    paged = op.paged_attention(q, K.reshape(B * S // P, P, Hkv, D), V.reshape(B * S // P, P, Hkv, D), bt, lengths)
    assert np.array_equal(got, paged)
    for b in range(B):
        for h in range(Hq):
            n = min(lengths[b], S)
            ref = _online_softmax_scalar(q[b, h], K[b, :, h // 2], V[b, :, h // 2], n, 1 / math.sqrt(D))
            assert np.allclose(got[b, h], ref, rtol=1e-9, atol=1e-12)


def test_contiguous_update_touches_one_row_per_sequence():
    rng = np.random.default_rng(31)
    K = rng.standard_normal((2, 8, 2, 4)).astype(np.float16)
    kn = rng.standard_normal((2, 2, 4)).astype(np.float16)
    K2, V2 = op.contiguous_update(K, K, kn, kn, [3, 7])
    assert np.array_equal(K2[0, 3], kn[0]) and np.array_equal(K2[1, 7], kn[1])
    mask = np.ones(K.shape[:2], bool)
    mask[0, 3] = mask[1, 7] = False
    assert np.array_equal(K2[mask], K[mask])
    K3, _ = op.contiguous_update(K, K, kn, kn, 5)  # a scalar position broadcasts
    assert np.array_equal(K3[:, 5], kn)


@pytest.mark.parametrize("bits", [8, 4])
def test_quantize_contiguous_respects_lengths(bits):
    rng = np.random.default_rng(32 + bits)
    B, S, H, D, g = 2, 6, 2, 64, 32
    K = rng.standard_normal((B, S, H, D)).astype(np.float16)
    kq, vq, ks, vs = op.quantize_contiguous(K, K, g, bits, lengths=[4, 6])
    full = op.quantize_contiguous(K, K, g, bits)
    assert np.array_equal(kq[0, :4], full[0][0, :4]) and np.array_equal(kq[1], full[0][1])
    assert not kq[0, 4:].any() and not ks[0, 4:].any()
    # dequantized rows past the length are 0; valid rows within the bound
    D_ = D
    deq = op.dequantize(op.unpack_last(kq, D_) if bits == 4 else kq, ks, g, bits)
    assert not deq[0, 4:].any()
    assert np.all(np.abs(deq[0, :4].astype(np.float64) - K[0, :4]) <=
                  np.repeat(np.abs(ks[0, :4].astype(np.float64)), g, axis=-1) * 0.51 + 1e-3)


# ------------------------------------------------------- multi-row verify

def _dense_causal_verify(q, K, V, lengths, scale):
    """Brute force over a dense [W, S] score matrix with the causal mask
    written out (j visible to row w iff j <= lengths[b] - W + w), scalar
    softmax loops -- a different formulation from the oracle's per-row calls."""
    B, W, Hq, D = q.shape
    g = Hq // K.shape[2]
    out = np.zeros(q.shape)
    for b in range(B):
        for w in range(W):
            last = int(lengths[b]) - W + w  # the row's own position
            for h in range(Hq):
                scores = []
                for j in range(K.shape[1]):
                    if j <= last:
                        scores.append((j, float(np.dot(q[b, w, h].astype(np.float64),
                                                       K[b, j, h // g].astype(np.float64))) * scale))
                if not scores:
                    continue
                mx = max(sc for _, sc in scores)
                den = sum(math.exp(sc - mx) for _, sc in scores)
                for j, sc in scores:
                    out[b, w, h] += math.exp(sc - mx) / den * V[b, j, h // g].astype(np.float64)
    return out


def test_verify_attention_brute_force_and_row_lengths():
    rng = np.random.default_rng(90)
    B, W, Hq, Hkv, D, P, mb = 3, 4, 4, 2, 8, 4, 4
    Kp = rng.standard_normal((B * mb, P, Hkv, D)).astype(np.float16)
    Vp = rng.standard_normal((B * mb, P, Hkv, D)).astype(np.float16)
    bt = rng.permutation(B * mb).astype(np.int32).reshape(B, mb)
    q = rng.standard_normal((B, W, Hq, D)).astype(np.float16)
    lengths = np.array([16, 7, 2])  # the last: rows 0 and 1 see nothing
    assert op.verify_row_lengths(lengths, W).tolist() == [[13, 14, 15, 16], [4, 5, 6, 7], [0, 0, 1, 2]]
    got = op.paged_verify_attention(q, Kp, Vp, bt, lengths)
    K, _ = op.gather(Kp, bt, mb * P)
    V, _ = op.gather(Vp, bt, mb * P)
    ref = _dense_causal_verify(q, K, V, lengths, 1.0 / math.sqrt(D))
    assert np.allclose(got, ref, rtol=1e-12, atol=1e-12)
    assert np.all(got[2, :2] == 0.0)
    # W = 1 is the decode attention; the last row always is
    assert np.array_equal(op.paged_verify_attention(q[:, -1:], Kp, Vp, bt, lengths)[:, 0],
                          op.paged_attention(q[:, -1], Kp, Vp, bt, lengths))
    assert np.array_equal(got[:, -1], op.paged_attention(q[:, -1], Kp, Vp, bt, lengths))


def test_verify_attention_equals_staged_decode_loop_and_is_causal():
    """The staged loop of parallel_verify_tokens (ops/speculative_verify_ops.py:
    228-262) -- write draft token i's K/V at position p + i, then attend with
    p + i + 1 positions -- against one multi-row call over the cache holding
    all W writes; and a change at the last position reaches only the last row."""
    rng = np.random.default_rng(91)
    B, W, Hq, Hkv, D, P, mb = 2, 5, 8, 2, 16, 8, 4
    Kp = rng.standard_normal((B * mb, P, Hkv, D)).astype(np.float16)
    Vp = rng.standard_normal((B * mb, P, Hkv, D)).astype(np.float16)
    bt = rng.permutation(B * mb).astype(np.int32).reshape(B, mb)
    p = np.array([9, 20])
    q = rng.standard_normal((B, W, Hq, D)).astype(np.float16)
    kn = rng.standard_normal((B, W, Hkv, D)).astype(np.float16)
    vn = rng.standard_normal((B, W, Hkv, D)).astype(np.float16)
    K1, V1 = Kp, Vp
    staged = []
    for i in range(W):
        K1, V1 = op.paged_kv_update(K1, V1, kn[:, i], vn[:, i], bt, p + i)
        staged.append(op.paged_attention(q[:, i], K1, V1, bt, p + i + 1))
    got = op.paged_verify_attention(q, K1, V1, bt, p + W)
    assert np.array_equal(got, np.stack(staged, axis=1))
    page, off = op.block_table_lookup(bt, p + W - 1, P)
    K2 = K1.copy()
    K2[page, off] += np.float16(1.0)
    got2 = op.paged_verify_attention(q, K2, V1, bt, p + W)
    assert np.array_equal(got2[:, :-1], got[:, :-1]) and not np.allclose(got2[:, -1], got[:, -1])


def test_quantized_verify_attention_is_verify_over_dequantized_pages():
    rng = np.random.default_rng(92)
    B, W, Hq, Hkv, D, P, mb, g = 2, 3, 4, 1, 32, 4, 3, 16
    Kp = rng.standard_normal((B * mb, P, Hkv, D)).astype(np.float16)
    Vp = rng.standard_normal((B * mb, P, Hkv, D)).astype(np.float16)
    bt = rng.permutation(B * mb).astype(np.int32).reshape(B, mb)
    q = rng.standard_normal((B, W, Hq, D)).astype(np.float16)
    for bits in (8, 4):
        kq, vq, ks, vs = op.quantize_pages(Kp, Vp, g, bits)
        Kd, Vd = op.dequantize_pages(kq, vq, ks, vs, g, bits, D)
        got = op.quantized_paged_verify_attention(q, kq, vq, ks, vs, bt, [12, 5], g, bits)
        assert np.array_equal(got, op.paged_verify_attention(q, Kd, Vd, bt, [12, 5]))


def test_metal_semantics_matvec_one_hot_and_w_rounding():
    """q4/q8_matvec_w32 (the reference's Metal kernels: fp32 W): a one-hot row
    e_k gives the fp32 dequant W[n, k] rounded once to fp16 (the dequant's
    closed form), and on random rows it differs from the pure-array oracle
    (fp16-rounded W) by no more than the W rounding can move a sum,
    2^-11 sum_k |x_k W_nk|, plus one output rounding each."""
    rng = np.random.default_rng(91)
    N, K, g = 48, 256, 32
    codes = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    s = (rng.standard_normal((N, K // g)) * 0.01).astype(np.float32)
    z = rng.integers(0, 16, size=(N, K // g)).astype(np.float32)
    W32 = oq.dequant(codes, s, z, g, np.float32)
    for k in (0, 1, 97, K - 1):
        x = np.zeros((1, K), np.float16)
        x[0, k] = 1.0
        assert np.array_equal(oq.q4_matvec_w32(x, oq.pack_q4(codes), s, z, g)[0], W32[:, k].astype(np.float16))
        assert np.array_equal(oq.q8_matvec_w32(x, codes, s, z, g)[0], W32[:, k].astype(np.float16))
    x = rng.standard_normal((3, K)).astype(np.float16)
    a = oq.q4_matvec_w32(x, oq.pack_q4(codes), s, z, g).astype(np.float64)
    b = oq.q4_matvec(x, oq.pack_q4(codes), s, z, g).astype(np.float64)
    bound = (np.abs(x.astype(np.float64)) @ np.abs(W32.astype(np.float64)).T) * 2.0 ** -11
    assert np.all(np.abs(a - b) <= bound + (np.abs(a) + np.abs(b)) * 2.0 ** -11 + 1e-7)
    assert not np.array_equal(a, b)  # the two semantics are distinguishable


def test_memoized_dequant_matches_and_reuses():
    """oracle.quant.memoized_dequant: the same matvec results as without it,
    one dequantization per weight array set, nothing kept after the block."""
    rng = np.random.default_rng(92)
    packed = rng.integers(0, 256, size=(32, 64), dtype=np.uint8)
    s = rng.uniform(0.01, 0.02, size=(32, 4)).astype(np.float32)
    z = np.full((32, 4), 8.0, np.float32)
    x = rng.standard_normal((2, 128)).astype(np.float16)
    plain = oq.q4_matvec(x, packed, s, z, 32)
    with oq.memoized_dequant():
        a = oq.q4_matvec(x, packed, s, z, 32)
        b = oq.q4_matvec(x[:1], packed, s, z, 32)
        assert len(oq._DEQ_MEMO) == 1
        oq.q8_matvec(x, rng.integers(0, 256, size=(8, 128), dtype=np.uint8), s[:8], z[:8], 32)
        assert len(oq._DEQ_MEMO) == 2
    assert oq._DEQ_MEMO is None
    assert np.array_equal(a, plain) and np.array_equal(b, plain[:1])
