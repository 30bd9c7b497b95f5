"""HIP weight quantizer (mk_quantize_weight) vs the oracle: bit-exact codes
and scales for q4/q8, odd K, odd group sizes, all-zero groups, fp32/fp16/bf16
weights and fp16/bf16/fp32 scales; and the quantized weights feeding the
matvec kernels."""

import numpy as np
import pytest
import torch

import mk.quant_ops as qo
import mk.quantize_weights as qw
from oracle import quant as oq
from tests._data import assert_close

pytestmark = pytest.mark.gpu

WDT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
SDT = {"float16": np.float16, "float32": np.float32}


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("n,k,g", [(8, 64, 32), (5, 67, 64), (3, 33, 7), (16, 4096, 64), (7, 1, 4), (2, 130, 130)])
@pytest.mark.parametrize("wdt", ["f32", "f16", "bf16"])
def test_quantize_weight_bit_exact(dev, bits, n, k, g, wdt):
    rng = np.random.default_rng(bits * 100 + k + g)
    W = torch.from_numpy((rng.standard_normal((n, k)) * 0.02).astype(np.float32)).to(WDT[wdt])
    W[0, : min(g, k)] = 0.0
    w32 = W.float().numpy()  # the oracle quantizes the (rounded) values the kernel reads
    p, s = oq.quantize_weight_groupwise(w32, bits, g)
    for sname in ("float16", "float32"):
        r = qw.quantize_weight_groupwise(W.to(dev), qw.QuantizationConfig(bits=bits, group_size=g, dtype=sname))
        assert np.array_equal(r.packed_weight.cpu().numpy(), p)
        got = r.scales.cpu().numpy()
        assert np.array_equal(got.view(np.uint16 if sname == "float16" else np.uint32),
                              s.astype(SDT[sname]).view(np.uint16 if sname == "float16" else np.uint32))
    rb = qw.quantize_weight_groupwise(W.to(dev), qw.QuantizationConfig(bits=bits, group_size=g, dtype="bfloat16"))
    ref_bf = torch.from_numpy(s).to(torch.bfloat16)
    assert torch.equal(rb.scales.cpu().view(torch.int16), ref_bf.view(torch.int16))


def test_quantized_weights_feed_the_matvec(dev):
    rng = np.random.default_rng(5)
    N, K, g = 256, 4096, 64
    W = torch.from_numpy((rng.standard_normal((N, K)) * 0.02).astype(np.float32)).to(dev)
    q = qw.quantize_weight_groupwise(W, qw.QuantizationConfig(bits=4, group_size=g))
    x = torch.from_numpy(rng.standard_normal((1, K)).astype(np.float16)).to(dev)
    y = qo.q4_matvec_decode(x, q.packed_weight, q.scales, q.kernel_zeros(), group_size=g)
    ref = oq.q4_matvec(x.cpu().numpy(), q.packed_weight.cpu().numpy(), q.scales.float().cpu().numpy(),
                       np.full((N, K // g), 8.0, np.float32), g)
    assert_close(y, ref.astype(np.float32), what="q4 matvec of quantized weights")
    deq = qw.dequantize_quantized_weight(q.packed_weight, q.scales, bits=4, group_size=g)
    # quantization error bound of the reference's test (tests/test_quantize_weights.py:18-27)
    rmse = float(torch.sqrt(torch.mean((deq.float() - W) ** 2)))
    assert rmse < 0.25 * float(W.abs().max())
