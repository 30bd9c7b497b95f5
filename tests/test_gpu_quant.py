"""HIP q4/q8 pack, dequant, matvec, gate/up and MLP block vs the oracle."""

import numpy as np
import pytest
import torch

import mk.mlp_block_ops as mlp
import mk.quant_ops as qo
from oracle import quant as oq
from tests._data import assert_close, quant_weight, to_dev

pytestmark = pytest.mark.gpu

ACT = {"f16": torch.float16, "bf16": torch.bfloat16}


def _x(rng, M, K, act, dev):
    x = rng.standard_normal((M, K)).astype(np.float32)
    t = torch.from_numpy(x).to(ACT[act]).to(dev)
    return t, t.float().cpu().numpy()


# ------------------------------------------------------------ bit-exact integer paths

def test_pack_unpack_bit_exact(dev):
    rng = np.random.default_rng(60)
    for shape in ((4, 64), (3, 65), (1, 1), (7, 4096)):
        q = rng.integers(0, 16, size=shape, dtype=np.uint8)
        got = qo.pack_q4(to_dev(q, dev))
        assert np.array_equal(got.cpu().numpy(), oq.pack_q4(q))
        back = qo.unpack_q4(got, shape[1])
        assert np.array_equal(back.cpu().numpy(), q)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("zeros_kind", ["none", "sym", "affine"])
@pytest.mark.parametrize("out", ["f16", "bf16"])
@pytest.mark.parametrize("sdt", [torch.float32, torch.float16])
def test_dequant_bit_exact(dev, bits, zeros_kind, out, sdt):
    rng = np.random.default_rng(61)
    M, K, g = 5, 96, 32
    codes, stored, s, z = quant_weight(rng, M, K, g, bits, zeros_kind, "normal")
    s = torch.from_numpy(s).to(sdt).float().numpy()  # the values the kernel will see
    if z is not None:
        z = torch.from_numpy(z).to(sdt).float().numpy()
    fn = qo.dequant_q4 if bits == 4 else qo.dequant_q8
    got = fn(to_dev(stored, dev), to_dev(s, dev, sdt), to_dev(z, dev, sdt), group_size=g, out_dtype=ACT[out],
             backend="metal")
    ref = oq.dequant(codes, s, z, g, np.float32)
    ref = ref.astype(np.float16).astype(np.float32) if out == "f16" else oq.round_bf16(ref)
    assert np.array_equal(got.float().cpu().numpy(), ref)


# ------------------------------------------------------------ matvec

MATVEC_CASES = [
    # (M, N, K, g)  -- reference test shapes, generic-path shapes, fast-path shapes
    (1, 32, 64, 32),
    (2, 50, 96, 16),
    (2, 48, 128, 32),
    (1, 64, 64, 8),
    (3, 33, 256, 64),
    (1, 4096, 4096, 64),
    (4, 1000, 4096, 64),
    (8, 4096, 14336, 64),
    (16, 96, 512, 128),
    (17, 64, 256, 64),
    # M = 1 dot path with a partial last 2048-k slice (K % 2048 != 0)
    (1, 200, 3072, 64),
    (1, 77, 2560, 64),
    (1, 96, 512, 64),
    (1, 64, 5120, 32),
]


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M,N,K,g", MATVEC_CASES)
def test_matvec_f16(dev, bits, M, N, K, g):
    rng = np.random.default_rng(100 + M + N + K)
    codes, stored, s, z = quant_weight(rng, N, K, g, bits, "sym")
    xt, xf = _x(rng, M, K, "f16", dev)
    fn = qo.q4_matvec_decode if bits == 4 else qo.q8_matvec_decode
    got = fn(xt, to_dev(stored, dev), to_dev(s, dev, torch.float16), to_dev(z, dev, torch.float16), group_size=g,
             backend="metal")
    s16 = s.astype(np.float16).astype(np.float32)
    ref = (oq.q4_matvec if bits == 4 else oq.q8_matvec)(xf.astype(np.float16), stored, s16, z, g)
    assert_close(got, ref, what=f"q{bits} M{M} N{N} K{K} g{g}")


# batched decode rows (the v_dot2 kernel at M <= 4 (q8: 2), the MFMA kernel
# above, in 16-row passes): several passes, N not a multiple of 16, group
# 32-256, affine / absent zero points
TILE_CASES = [
    (2, 48, 128, 32, "sym"),
    (5, 70, 1152, 32, "affine"),
    (16, 100, 4096, 64, "none"),
    (17, 40, 640, 64, "sym"),
    (32, 48, 4096, 128, "affine"),
    (33, 130, 640, 64, "none"),
    (20, 16, 256, 256, "affine"),
    (4, 3000, 14336, 64, "sym"),
    (64, 96, 1536, 64, "sym"),
    # the activation-stationary kernel (q4, N % 16 == 0 with >= 512 row
    # tiles, K % 256 == 0, K <= 4096): two groups per lane's 64 k with an odd
    # tile count, one and two column tiles, no zero points, 32 + 1 rows, a
    # one-wave workgroup; N = 8200 takes the other kernels
    (5, 8208, 2048, 32, "affine"),
    (5, 8200, 2048, 32, "affine"),
    # the K-split kernel (q4, one matrix, N % 16 == 0, K % 128 == 0 with
    # 2048 <= K <= 16384): the down projection's 14336 k (7 halves per wave),
    # one half per wave with two groups per half, two column tiles with
    # uneven halves per wave and no zero points
    (8, 4096, 14336, 64, "sym"),
    (5, 1024, 2048, 32, "affine"),
    # ... at 6 and 7 rows with uneven halves per wave (2 or 3; 1 or 2)
    (6, 2048, 5120, 64, "none"),
    (7, 1040, 3072, 64, "affine"),
    (20, 2048, 6272, 128, "none"),
    (17, 8192, 4096, 128, "none"),
    (33, 8192, 1024, 64, "sym"),
    (12, 16384, 256, 64, "sym"),
]


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M,N,K,g,zk", TILE_CASES)
def test_batched_matvec(dev, bits, M, N, K, g, zk):
    rng = np.random.default_rng(300 + M + N + K + g)
    codes, stored, s, z = quant_weight(rng, N, K, g, bits, zk, "normal")
    s = (s * 0.01).astype(np.float16).astype(np.float32)
    xt, xf = _x(rng, M, K, "f16", dev)
    fn = qo.q4_matvec_decode if bits == 4 else qo.q8_matvec_decode
    got = fn(xt, to_dev(stored, dev), to_dev(s, dev, torch.float16), to_dev(z, dev, torch.float16), group_size=g)
    mv = oq.q4_matvec if bits == 4 else oq.q8_matvec
    ref = mv(xf.astype(np.float16), stored, s, z, g)
    assert_close(got, ref, what=f"q{bits} M{M} N{N} K{K} g{g} {zk}", rms_atol=True)
    # residual epilogue (the down projection's): y_mm and residual + y_mm
    res = torch.from_numpy(rng.standard_normal((M, N)).astype(np.float16)).to(dev)
    ymm, out = qo.q_matvec_residual(xt, to_dev(stored, dev), to_dev(s, dev, torch.float16),
                                    to_dev(z, dev, torch.float16), res, bits=bits, group_size=g, want_mm=True)
    assert torch.equal(ymm, got), "same kernel, same partial sums"
    assert_close(out, oq.residual_add(res.cpu().numpy(), ymm.cpu().numpy()), rtol=1e-3, what="residual epilogue")


# the v_dot2 kernel with 2-4 activation rows (q8: 2; 3 runs as 4 with the
# last row repeated): partial last 2048-k slice, N not a multiple of the
# rows per workgroup, group 32 / 128, zeros absent
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M,N,K,g,zk", [(2, 77, 2560, 64, "sym"), (3, 130, 4096, 32, "affine"),
                                        (4, 96, 6144, 128, "none"), (4, 4096, 14336, 64, "sym")])
def test_dot_rows_matvec_and_gate_up(dev, bits, M, N, K, g, zk):
    rng = np.random.default_rng(500 + M + N + K)
    codes, stored, s, z = quant_weight(rng, N, K, g, bits, zk, "normal")
    s = (s * 0.01).astype(np.float16).astype(np.float32)
    xt, xf = _x(rng, M, K, "f16", dev)
    x16 = xf.astype(np.float16)
    mv = oq.q4_matvec if bits == 4 else oq.q8_matvec
    fn = qo.q4_matvec_decode if bits == 4 else qo.q8_matvec_decode
    w = (to_dev(stored, dev), to_dev(s, dev, torch.float16), to_dev(z, dev, torch.float16))
    got = fn(xt, *w, group_size=g)
    ref = mv(x16, stored, s, z, g)
    assert_close(got, ref, what=f"matvec q{bits} M{M}", rms_atol=True)
    res = torch.from_numpy(rng.standard_normal((M, N)).astype(np.float16)).to(dev)
    ymm, out = qo.q_matvec_residual(xt, *w, res, bits=bits, group_size=g, want_mm=True)
    assert torch.equal(ymm, got)
    assert_close(out, oq.residual_add(res.cpu().numpy(), ymm.cpu().numpy()), rtol=1e-3, what="residual")
    _, su_stored, su, zu = quant_weight(rng, N, K, g, bits, zk, "normal")
    su = (su * 0.01).astype(np.float16).astype(np.float32)
    gfn = qo.q4_gate_up_matvec_tiled if bits == 4 else qo.q8_gate_up_matvec_tiled
    gate, up = gfn(xt, w[0], to_dev(su_stored, dev), w[1], to_dev(su, dev, torch.float16), w[2],
                   to_dev(zu, dev, torch.float16), group_size=g)
    assert_close(gate, ref, what="gate", rms_atol=True)
    assert_close(up, mv(x16, su_stored, su, zu, g), what="up", rms_atol=True)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M,N,K,g", [(4, 14336, 4096, 64), (8, 14336, 4096, 64), (32, 14336, 4096, 64),
                                     (6, 200, 1280, 64), (24, 90, 512, 32), (32, 64, 4096, 64)])
def test_batched_gate_up(dev, bits, M, N, K, g):
    rng = np.random.default_rng(400 + M + N)
    _, sg_stored, sg, zg = quant_weight(rng, N, K, g, bits, "sym")
    _, su_stored, su, zu = quant_weight(rng, N, K, g, bits, "affine", "normal")
    su = (su * 0.01).astype(np.float16).astype(np.float32)
    sg = sg.astype(np.float16).astype(np.float32)
    xt, xf = _x(rng, M, K, "f16", dev)
    args = (to_dev(sg_stored, dev), to_dev(su_stored, dev), to_dev(sg, dev, torch.float16),
            to_dev(su, dev, torch.float16), to_dev(zg, dev, torch.float16), to_dev(zu, dev, torch.float16))
    fn = qo.q4_gate_up_matvec_tiled if bits == 4 else qo.q8_gate_up_matvec_tiled
    gate, up = fn(xt, *args, group_size=g)
    mv = oq.q4_matvec if bits == 4 else oq.q8_matvec
    x16 = xf.astype(np.float16)
    assert_close(gate, mv(x16, sg_stored, sg, zg, g), what="gate")
    assert_close(up, mv(x16, su_stored, su, zu, g), what="up", rms_atol=True)
    mlp_out = qo.q_gate_up_swiglu(xt, *args, bits=bits, group_size=g)
    assert_close(mlp_out, oq.swiglu(gate.cpu().numpy(), up.cpu().numpy()), rtol=1e-3, what="swiglu epilogue")


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("act", ["f16", "bf16"])
@pytest.mark.parametrize("zeros_kind", ["none", "affine"])
@pytest.mark.parametrize("sdt", [torch.float16, torch.float32])
@pytest.mark.parametrize("M,N,K,g", [(2, 50, 96, 16), (3, 40, 512, 64), (1, 72, 3072, 64)])
def test_matvec_dtypes_and_zeros(dev, bits, act, zeros_kind, sdt, M, N, K, g):
    rng = np.random.default_rng(7)
    codes, stored, s, z = quant_weight(rng, N, K, g, bits, zeros_kind, "normal")
    s = torch.from_numpy(s).to(sdt).float().numpy()
    z = None if z is None else torch.from_numpy(z).to(sdt).float().numpy()
    xt, xf = _x(rng, M, K, act, dev)
    fn = qo.q4_matvec_decode if bits == 4 else qo.q8_matvec_decode
    got = fn(xt[:, None, :], to_dev(stored, dev), to_dev(s, dev, sdt), to_dev(z, dev, sdt), group_size=g,
             backend="metal_tiled")
    ref = (oq.q4_matvec if bits == 4 else oq.q8_matvec)(xf, stored, s, z, g, act=act)
    assert got.dtype == ACT[act] and tuple(got.shape) == (M, N)
    assert_close(got, ref, rtol=1e-2 if act == "f16" else 2e-2, what=f"q{bits} {act} {zeros_kind}", rms_atol=True)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M", [1, 3, 8, 24, 40])
@pytest.mark.parametrize("amp", [1.0, 1e-4])
def test_matvec_one_hot_rows_are_exact_dequant(dev, bits, M, amp):
    """x row m = e_{k_m}: y[m, n] is the dequantized weight W[n, k_m] rounded
    to fp16 once (the reference's dequant, ops/quant_ops.py:191-212), so every
    kernel path (v_dot2 rows, MFMA, two-column tiles) must reproduce it bit
    for bit -- including groups whose fp16 scale is below 2^-10 (amp 1e-4),
    where a scale pre-divided by 16 would become subnormal."""
    rng = np.random.default_rng(17 + M + bits)
    N, K, g = 160, 512, 64
    codes, stored, s, z = quant_weight(rng, N, K, g, bits, "affine", "normal")
    s = (s * amp).astype(np.float16).astype(np.float32)
    ks = rng.integers(0, K, size=M)
    ks[: min(M, 4)] = [0, 1, K - 2, K - 1][: min(M, 4)]  # even and odd columns, both ends
    x = np.zeros((M, K), np.float16)
    x[np.arange(M), ks] = 1.0
    fn = qo.q4_matvec_decode if bits == 4 else qo.q8_matvec_decode
    y = fn(to_dev(x, dev), to_dev(stored, dev), to_dev(s, dev, torch.float16), to_dev(z, dev, torch.float16),
           group_size=g).cpu().numpy()
    W = oq.dequant(codes, s, z, g, np.float16)
    # equal as numbers (a code at its zero point gives +0 from the sum where
    # the reference's (q - z) * s gives -0 for a negative scale)
    assert np.array_equal(y, W[:, ks].T)


@pytest.mark.parametrize("bits", [4, 8])
def test_matvec_saturates(dev, bits):
    K = 256
    x = torch.full((1, K), 200.0, dtype=torch.float16, device=dev)
    codes = np.full((16, K), 15 if bits == 4 else 255, np.uint8)
    stored = oq.pack_q4(codes) if bits == 4 else codes
    s = torch.full((16, K // 64), 4.0, dtype=torch.float16, device=dev)
    fn = qo.q4_matvec_decode if bits == 4 else qo.q8_matvec_decode
    y = fn(x, to_dev(stored, dev), s, None, group_size=64)
    assert torch.all(y == 65504.0)
    y = fn(-x, to_dev(stored, dev), s, None, group_size=64)
    assert torch.all(y == -65504.0)


# ------------------------------------------------------------ gate / up / MLP

@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("rows,N,K,g", [(3, 50, 96, 32), (1, 14336, 4096, 64), (8, 512, 4096, 64), (5, 64, 95, 32),
                                        (1, 300, 3072, 64), (1, 256, 4096, 32)])
def test_gate_up_and_swiglu_epilogue(dev, bits, rows, N, K, g):
    if bits == 8 and K % 2:
        pytest.skip("odd K only matters for the q4 ceil(K/2) packing")
    rng = np.random.default_rng(11 + rows + N)
    cg, sg_stored, sg, zg = quant_weight(rng, N, K, g, bits, "sym")
    cu, su_stored, su, zu = quant_weight(rng, N, K, g, bits, "sym")
    xt, xf = _x(rng, rows, K, "f16", dev)
    args = (to_dev(sg_stored, dev), to_dev(su_stored, dev), to_dev(sg, dev, torch.float16),
            to_dev(su, dev, torch.float16), to_dev(zg, dev, torch.float16), to_dev(zu, dev, torch.float16))
    fn = qo.q4_gate_up_matvec_tiled if bits == 4 else qo.q8_gate_up_matvec_tiled
    gate, up = fn(xt, *args, group_size=g)
    mv = oq.q4_matvec if bits == 4 else oq.q8_matvec
    x16 = xf.astype(np.float16)
    rg = mv(x16, sg_stored, sg.astype(np.float16).astype(np.float32), zg, g)
    ru = mv(x16, su_stored, su.astype(np.float16).astype(np.float32), zu, g)
    assert_close(gate, rg, what="gate")
    assert_close(up, ru, what="up")
    mlp_out = qo.q_gate_up_swiglu(xt, args[0], args[1], args[2], args[3], args[4], args[5], bits=bits, group_size=g)
    # the epilogue consumes the kernel's own rounded gate/up
    assert_close(mlp_out, oq.swiglu(gate.cpu().numpy(), up.cpu().numpy()), rtol=1e-3, what="swiglu epilogue")
    assert_close(mlp_out, oq.swiglu(rg, ru), what="swiglu vs oracle")


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("rows,N,K,g,act", [(1, 14336, 4096, 64, "f16"), (1, 300, 3072, 64, "f16"),
                                            (1, 256, 4096, 32, "f16"), (3, 50, 96, 32, "f16"),
                                            (1, 64, 512, 64, "bf16"),
                                            # 5..16 rows: norm kernel, then the activation-stationary
                                            # gate/up (two groups per run at g = 32)
                                            (8, 14336, 4096, 64, "f16"), (5, 8192, 2048, 32, "f16"),
                                            (16, 8192, 1024, 128, "f16")])
def test_rmsnorm_gate_up(dev, bits, rows, N, K, g, act):
    """mk_q{4,8}_rmsnorm_gate_up (one launch for an fp16 row, the norm and
    gate/up kernels otherwise) against the separate norm kernel and the oracle."""
    import mk.norm_ops as norm

    rng = np.random.default_rng(31 + rows + N + K)
    _, sg_stored, sg, zg = quant_weight(rng, N, K, g, bits, "sym")
    _, su_stored, su, zu = quant_weight(rng, N, K, g, bits, "sym")
    xt, xf = _x(rng, rows, K, act, dev)
    rt, rf = _x(rng, rows, K, act, dev)
    nw = torch.from_numpy((1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)).to(ACT[act]).to(dev)
    args = (to_dev(sg_stored, dev), to_dev(su_stored, dev), to_dev(sg, dev, torch.float16),
            to_dev(su, dev, torch.float16), to_dev(zg, dev, torch.float16), to_dev(zu, dev, torch.float16))
    z, normed, gate, up, mlp = qo.q_rmsnorm_gate_up_swiglu(xt, rt, nw, *args, bits=bits, group_size=g, eps=1e-5,
                                                           return_gate_up=True)
    z_ref, n_ref = norm.residual_rms_norm(xt[:, None], rt[:, None], nw, eps=1e-5)
    assert torch.equal(z, z_ref[:, 0])
    # the one-launch path sums z^2 in another order: the rsqrt can move by an
    # ulp, so a normalised element may land one fp16/bf16 step away
    nd = (normed.float() - n_ref[:, 0].float()).abs()
    step = n_ref[:, 0].float().abs() * (2.0 ** -10 if act == "f16" else 2.0 ** -7) + 1e-7
    assert torch.all(nd <= step)
    # gate/up/mlp against the oracle on the kernel's own normalised row
    mv = oq.q4_matvec if bits == 4 else oq.q8_matvec
    nf = normed.float().cpu().numpy()
    rg = mv(nf, sg_stored, sg.astype(np.float16).astype(np.float32), zg, g, act=act)
    ru = mv(nf, su_stored, su.astype(np.float16).astype(np.float32), zu, g, act=act)
    tol = 1e-2 if act == "f16" else 2e-2
    assert_close(gate, rg, rtol=tol, what="gate")
    assert_close(up, ru, rtol=tol, what="up")
    assert_close(mlp, oq.swiglu(gate.float().cpu().numpy(), up.float().cpu().numpy(), act=act), rtol=tol,
                 what="swiglu epilogue")
    if act == "f16":  # z against the oracle's residual add (bit-exact)
        zo = oq.residual_add(xf.astype(np.float16), rf.astype(np.float16))
        assert np.array_equal(z.cpu().numpy(), zo)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("rows,N,K,g,act", [(1, 6144, 4096, 64, "f16"), (1, 512, 4096, 32, "f16"),
                                            (1, 1000, 2048, 64, "f16"), (1, 300, 8192, 128, "f16"),
                                            (2, 64, 256, 32, "f16"), (1, 64, 512, 64, "bf16")])
def test_rmsnorm_matvec(dev, bits, rows, N, K, g, act):
    """mk_q{4,8}_rmsnorm_matvec (one launch for a q4 fp16 row: the norm as the
    dot kernel's prologue with no residual) against the norm kernel and the
    oracle on the kernel's own normalised rows."""
    import mk.norm_ops as norm

    rng = np.random.default_rng(41 + rows + N + K)
    _, stored, s, z = quant_weight(rng, N, K, g, bits, "sym")
    xt, xf = _x(rng, rows, K, act, dev)
    nw = torch.from_numpy((1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)).to(ACT[act]).to(dev)
    y, normed = qo.q_rmsnorm_matvec(xt, nw, to_dev(stored, dev), to_dev(s, dev, torch.float16),
                                    to_dev(z, dev, torch.float16), bits=bits, group_size=g, eps=1e-5,
                                    return_normed=True)
    n_ref = norm.rms_norm(xt[:, None], nw, eps=1e-5)[:, 0]
    nd = (normed.float() - n_ref.float()).abs()
    step = n_ref.float().abs() * (2.0 ** -10 if act == "f16" else 2.0 ** -7) + 1e-7
    assert torch.all(nd <= step), "normed within one step of the norm kernel"
    mv = oq.q4_matvec if bits == 4 else oq.q8_matvec
    ref = mv(normed.float().cpu().numpy(), stored, s.astype(np.float16).astype(np.float32), z, g, act=act)
    assert_close(y, ref, rtol=1e-2 if act == "f16" else 2e-2, what="rmsnorm matvec")


def _dot_kernel_path(bits, rows, K, g):
    """Whether a fp16 projection of ``rows`` rows over K runs on the v_dot2
    kernel (W exact) rather than an MFMA kernel (W rounded to fp16): the
    shape part of the dispatcher's test (gemv.hip, dot_eligible) -- at most
    4 rows (q4) / 2 (q8), group size 32..256, K % 32 == 0, K <= 16384 and a
    group count divisible by 8."""
    G = -(-K // g)
    return rows <= (4 if bits == 4 else 2) and 32 <= g <= 256 and K % 32 == 0 and K <= 16384 and G % 8 == 0


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("preset", ["tiled", "fused_experimental", "parallel", "metal"])
@pytest.mark.parametrize("B,S,D,I,g", [(1, 1, 64, 128, 32), (2, 1, 64, 130, 32), (1, 1, 4096, 14336, 64),
                                       (4, 1, 256, 512, 64)])
def test_mlp_block(dev, bits, preset, B, S, D, I, g):
    if I % 2 and bits == 4 and preset != "fused_experimental":
        pytest.skip("q4 matvec backends require even K (ops/quant_ops.py:543)")
    rng = np.random.default_rng(21 + D + I)
    x = rng.standard_normal((B, S, D)).astype(np.float16)
    r = rng.standard_normal((B, S, D)).astype(np.float16)
    nw = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float16)
    mats = [quant_weight(rng, I, D, g, bits, "sym"), quant_weight(rng, I, D, g, bits, "sym"),
            quant_weight(rng, D, I, g, bits, "sym")]
    dv = lambda m: (to_dev(m[1], dev), to_dev(m[2], dev, torch.float16), to_dev(m[3], dev, torch.float16))
    (gw, gs, gz), (uw, us, uz), (dw, ds, dz) = dv(mats[0]), dv(mats[1]), dv(mats[2])
    out, inter = mlp.quantized_mlp_block(
        to_dev(x, dev), to_dev(r, dev), to_dev(nw, dev), gw, gs, uw, us, dw, ds, gate_zeros=gz, up_zeros=uz,
        down_zeros=dz, bits=bits, group_size=g, backend_preset=preset, return_intermediates=True)
    trip = lambda m: (m[1], m[2].astype(np.float16).astype(np.float32), m[3])
    assert tuple(out.shape) == (B, S, D)
    gi = {k: v.reshape(B * S, -1).cpu().numpy() for k, v in inter.items()}
    # every stage against the oracle on the kernel's own inputs, at the plain
    # tolerance, each projection against the semantics its kernel implements:
    # the v_dot2 kernel keeps W exact in fp32 (the reference's Metal kernels,
    # q4/q8_matvec_w32), the MFMA kernels round W to fp16 (the reference's
    # pure-array matvec, q4/q8_matvec).  At 14336-term rows the two differ by
    # ~1e-3 on small outputs, so the choice matters at full size.
    w32_gu, w32_dn = _dot_kernel_path(bits, B * S, D, g), _dot_kernel_path(bits, B * S, I, g)
    pick = lambda exact: ((oq.q4_matvec_w32 if bits == 4 else oq.q8_matvec_w32) if exact
                          else (oq.q4_matvec if bits == 4 else oq.q8_matvec))
    assert np.array_equal(gi["z"], oq.residual_add(x.reshape(-1, D), r.reshape(-1, D))), "z"
    assert_close(gi["normed"], oq.rms_norm(gi["z"], nw), what="normed")
    assert_close(gi["gate"], pick(w32_gu)(gi["normed"], *trip(mats[0]), group_size=g), what="gate")
    assert_close(gi["up"], pick(w32_gu)(gi["normed"], *trip(mats[1]), group_size=g), what="up")
    assert_close(gi["mlp"], oq.swiglu(gi["gate"], gi["up"]), rtol=2e-3, what="mlp")
    assert_close(gi["down"], pick(w32_dn)(gi["mlp"], *trip(mats[2]), group_size=g), what="down")
    # the residual epilogue is exact given the kernel's own z and down
    assert np.array_equal(gi.get("out", out.reshape(-1, D).cpu().numpy()), oq.residual_add(gi["z"], gi["down"]))
    # end to end against the all-oracle composition with the same semantics
    # per projection: rounded intermediates (fp16 gate/up/mlp/down) can flip
    # by an ulp and out = z + down can cancel, so admit a few ulps of |down|
    x2, r2 = x.reshape(-1, D), r.reshape(-1, D)
    ref, rint = oq.mlp_block(x2, r2, nw, trip(mats[0]), trip(mats[1]), trip(mats[2]), bits=bits, group_size=g,
                             intermediates=True, w32=(w32_gu, w32_dn))
    ulp_down = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(rint["down"].astype(np.float64)), 2.0 ** -14))) - 10)
    assert_close(out.reshape(-1, D), ref, extra=4 * ulp_down, what="mlp out")
    # and against the reference preset's composition (W rounded to fp16 in
    # every projection), allowing on top the spread between the reference's
    # own two presets on this input: that rounding moves each I-term down sum
    # by ~2^-12 of the typical |down|, not of the local output, which z + down
    # can cancel to near zero
    ref16 = oq.mlp_block(x2, r2, nw, trip(mats[0]), trip(mats[1]), trip(mats[2]), bits=bits, group_size=g)
    spread = np.abs(ref.astype(np.float64) - ref16.astype(np.float64))
    assert_close(out.reshape(-1, D), ref16, extra=4 * ulp_down + spread, what="mlp out vs reference preset")


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("B", [8, 32])
def test_mlp_block_full_size_batched(dev, bits, B):
    """Config 2 at M = 8 and config 5's batch 32 through the all-HIP MLP block
    (norm kernel, batched gate/up + SwiGLU, down + residual) at 4096/14336."""
    test_mlp_block(dev, bits, "fused_experimental", B, 1, 4096, 14336, 64)


def test_mlp_decode_step(dev):
    rng = np.random.default_rng(31)
    D, I, g = 256, 512, 64
    x = rng.standard_normal((2, 1, D)).astype(np.float16)
    nw = np.ones(D, np.float16)
    mats = [quant_weight(rng, I, D, g, 4, "sym"), quant_weight(rng, I, D, g, 4, "sym"),
            quant_weight(rng, D, I, g, 4, "sym")]
    dv = lambda m: (to_dev(m[1], dev), to_dev(m[2], dev, torch.float16))
    out = mlp.quantized_mlp_decode_step(to_dev(x, dev), to_dev(nw, dev), *dv(mats[0]), *dv(mats[1]), *dv(mats[2]),
                                        gate_zeros=to_dev(mats[0][3], dev, torch.float16),
                                        up_zeros=to_dev(mats[1][3], dev, torch.float16),
                                        down_zeros=to_dev(mats[2][3], dev, torch.float16), bits=4, group_size=g,
                                        backend_preset="parallel")
    trip = lambda m: (m[1], m[2].astype(np.float16).astype(np.float32), m[3])
    ref = oq.mlp_block(x.reshape(-1, D), x.reshape(-1, D), nw, trip(mats[0]), trip(mats[1]), trip(mats[2]), bits=4,
                       group_size=g)
    assert_close(out.reshape(-1, D), ref, what="decode step")


def test_reference_backend_matches_oracle(dev):
    rng = np.random.default_rng(41)
    codes, stored, s, z = quant_weight(rng, 64, 128, 32, 4, "affine", "normal")
    xt, xf = _x(rng, 2, 128, "f16", dev)
    got = qo.q4_matvec_decode(xt, to_dev(stored, dev), to_dev(s, dev), to_dev(z, dev), group_size=32,
                              backend="reference")
    assert_close(got, oq.q4_matvec(xf.astype(np.float16), stored, s, z, 32), what="reference backend", rms_atol=True)
