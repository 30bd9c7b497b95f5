"""HIP rms_norm / residual + rms_norm / SwiGLU / residual add vs the oracle.

Hidden sizes cover both norm kernels: D % 8 == 0 up to 8192 takes the
register-resident vector kernel (1, 2 or 4 chunks of 8 per thread), other D
the strided one.
"""

import numpy as np
import pytest
import torch

import mk.activation_ops as act_ops
import mk.fused_ops as fused
import mk.norm_ops as norm
from oracle import quant as oq
from tests._data import assert_close

pytestmark = pytest.mark.gpu

DT = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}


def _rand(rng, shape, dt, dev, scale=1.0):
    t = torch.from_numpy((rng.standard_normal(shape) * scale).astype(np.float32)).to(DT[dt])
    return t.to(dev), t.float().numpy()


def _round(a: np.ndarray, dt: str) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(DT[dt]).float().numpy()


@pytest.mark.parametrize("D", [8, 1000, 2048, 4096, 4100, 6000, 8192, 12288])
@pytest.mark.parametrize("xdt,wdt", [("f16", "f16"), ("bf16", "bf16"), ("f16", "f32"), ("f32", "f32"),
                                     ("bf16", "f16")])
def test_rms_norm(dev, D, xdt, wdt):
    rng = np.random.default_rng(D)
    x, xf = _rand(rng, (3, 1, D), xdt, dev)
    w, wf = _rand(rng, (D,), wdt, dev, 0.5)
    got = norm.rms_norm(x, w)
    assert got.dtype == x.dtype
    ref = _round(oq.rms_norm(xf, wf), xdt)
    assert_close(got.float().cpu().numpy(), ref, what=f"rms_norm D={D}")


@pytest.mark.parametrize("D", [8, 1000, 4096, 6000, 12288])
@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_residual_rms_norm(dev, D, dt):
    rng = np.random.default_rng(100 + D)
    x, xf = _rand(rng, (2, 1, D), dt, dev)
    r, rf = _rand(rng, (2, 1, D), dt, dev)
    w, wf = _rand(rng, (D,), dt, dev, 0.5)
    z, y = norm.residual_rms_norm(x, r, w)
    zref = _round(xf + rf, dt)
    # z is one rounding of an exact fp32 sum: bit-exact
    assert np.array_equal(z.float().cpu().numpy(), zref)
    yref = _round(oq.rms_norm(zref.reshape(2, D), wf), dt).reshape(2, 1, D)
    assert_close(y.float().cpu().numpy(), yref, what=f"residual_rms_norm D={D}")


def test_rms_norm_unaligned_view_uses_strided_kernel(dev):
    # a view starting one element in is not 16-byte aligned
    rng = np.random.default_rng(7)
    base, bf = _rand(rng, (4097,), "f16", dev)
    w, wf = _rand(rng, (4096,), "f16", dev)
    x = base[1:].reshape(1, 1, 4096)
    assert x.data_ptr() % 16 != 0
    got = norm.rms_norm(x, w)
    ref = _round(oq.rms_norm(bf[1:].reshape(1, 1, 4096), wf), "f16")
    assert_close(got.float().cpu().numpy(), ref, what="unaligned rms_norm")


@pytest.mark.parametrize("n", [1, 4096, 14336, 100003])
@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_swiglu_and_residual_add(dev, n, dt):
    rng = np.random.default_rng(n)
    g, gf = _rand(rng, (1, 1, n), dt, dev, 3.0)
    u, uf = _rand(rng, (1, 1, n), dt, dev)
    got = act_ops.swiglu(g, u)
    ref = oq.swiglu(gf, uf, act=dt).astype(np.float32)
    assert_close(got.float().cpu().numpy(), ref, what="swiglu")
    s = fused.residual_add(g, u)
    assert np.array_equal(s.float().cpu().numpy(), _round(gf + uf, dt))


@pytest.mark.parametrize("rows,n,dt", [(1, 128256, torch.float16), (32, 128256, torch.float16),
                                       (3, 1000, torch.bfloat16), (2, 515, torch.float16),
                                       (4, 4096, torch.float32), (2, 7, torch.float32),
                                       (5, 40000, torch.float16), (5, 8, torch.float16)])
def test_argmax_rows(dev, rows, n, dt):
    """Greedy sampling (models/sampling.py:120-124) on device against
    np.argmax: random rows, planted ties (the first index must win), a NaN
    row (the first NaN wins, as in numpy), a row with both infinities (whose
    packed fp16 sums are NaN without a NaN in the row) and a row of signed
    zeros (equal: the first wins)."""
    from mk.llama_stack_ops import greedy_sample

    rng = np.random.default_rng(rows * 7 + n)
    x = rng.standard_normal((rows, n)).astype(np.float32)
    if rows > 1:  # a tie between two positions of the row's maximum
        x[1, n // 3] = x[1, n - 1] = x[1].max() + 1.0
    if rows > 2:
        x[2, n // 2] = np.nan
        x[2, n - 2] = np.nan
    if rows > 4:
        x[3, n // 4] = -np.inf
        x[3, n - 1] = x[3, n // 5 + 1] = np.inf
        x[4] = 0.0
        x[4, ::3] = -0.0
    xt = torch.from_numpy(x).to(dt)
    want = np.argmax(xt.float().numpy(), axis=-1)  # the rounded values' argmax
    got = greedy_sample(xt.to(dev)).cpu().numpy()
    assert got.dtype == np.int64
    assert np.array_equal(got, want), (got, want)
    # a 3-D [B, 1, vocab] input and a misaligned (offset) view take the same answer
    got3 = greedy_sample(xt.to(dev)[:, None]).cpu().numpy()
    assert np.array_equal(got3, want)
    if n > 1:
        xs = xt.to(dev)[:, 1:]
        assert np.array_equal(greedy_sample(xs).cpu().numpy(), np.argmax(xt.float().numpy()[:, 1:], axis=-1))
