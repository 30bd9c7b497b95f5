"""Seeded input builders shared by the GPU parity tests."""

import numpy as np
import torch

from oracle import quant as oq


def quant_weight(rng, N, K, g, bits, zeros_kind="sym", scale_kind="weights"):
    """Codes + fp32 scales (+ zeros) in the layouts the ops take.
    scale_kind 'weights': symmetric quantization of W ~ N(0, 0.02) (the
    BASELINE configs); 'normal': random codes with N(0,1) scales, as the
    reference's kernel tests draw them."""
    G = -(-K // g)
    if scale_kind == "weights":
        W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        codes_packed, s = oq.quantize_weight_groupwise(W, bits, g)
        codes = oq.unpack_q4(codes_packed, K) if bits == 4 else codes_packed
    else:
        codes = rng.integers(0, 16 if bits == 4 else 256, size=(N, K), dtype=np.uint8)
        s = rng.standard_normal((N, G)).astype(np.float32)
    if zeros_kind == "none":
        z = None
    elif zeros_kind == "sym":
        z = np.full((N, G), 8.0 if bits == 4 else 128.0, np.float32)
    else:
        z = rng.integers(0, 16 if bits == 4 else 256, size=(N, G)).astype(np.float32)
    stored = oq.pack_q4(codes) if bits == 4 else codes
    return codes, stored, s, z


def to_dev(a, dev, dtype=None):
    if a is None:
        return None
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.to(dev)


def assert_close(got, ref, rtol=1e-2, atol=1e-3, what="", extra=0.0, rms_atol=False):
    """|got - ref| <= atol + rtol |ref| + extra, rtol
    1e-2 / atol 1e-3.  ``rms_atol`` scales atol by the output's rms (when
    above 1): only for the tests that draw N(0,1) scales as the reference's
    kernel tests do, whose outputs are O(10-100) -- there an absolute 1e-3 is
    below one fp16 ulp of a typical output.  ``extra`` adds a per-element
    allowance (e.g. one fp16 ulp of an intermediate that was rounded)."""
    g = got.detach().float().cpu().numpy().astype(np.float64) if isinstance(got, torch.Tensor) else np.asarray(got, np.float64)
    r = np.asarray(ref, dtype=np.float64)
    assert g.shape == r.shape, (what, g.shape, r.shape)
    scale = max(1.0, float(np.sqrt(np.mean(r * r)))) if (rms_atol and r.size) else 1.0
    err = np.abs(g - r)
    lim = atol * scale + rtol * np.abs(r) + extra
    bad = err > lim
    if bad.any():
        i = np.unravel_index(np.argmax(np.where(bad, err - lim, -np.inf)), err.shape)
        raise AssertionError(f"{what}: {int(bad.sum())}/{bad.size} out of tolerance, max err {err.max():.3g}; "
                             f"worst at {tuple(int(v) for v in i)}: got {g[i]:.6g} ref {r[i]:.6g} lim {lim[i]:.3g}")

