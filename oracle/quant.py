"""Oracle: q4/q8 packing, dequant, decode matvec family and the MLP block.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
"""

from __future__ import annotations

import contextlib
import math

import numpy as np

F16_MAX = 65504.0


def pack_q4(q: np.ndarray) -> np.ndarray:
    """ops/quant_ops.py:166-176: uint8 low + (high << 4), odd K padded with 0."""
    q = np.asarray(q).astype(np.uint8)
    if q.shape[1] % 2:
        q = np.pad(q, ((0, 0), (0, 1)))
    return (q[:, 0::2] + (q[:, 1::2] << 4)).astype(np.uint8)


def unpack_q4(packed: np.ndarray, K: int | None = None) -> np.ndarray:
    """ops/quant_ops.py:179-188."""
    p = np.asarray(packed).astype(np.uint8)
    out = np.stack([p & 0x0F, (p >> 4) & 0x0F], axis=-1).reshape(p.shape[0], p.shape[1] * 2)
    return out if K is None else out[:, :K]


def _expand(t: np.ndarray, g: int, K: int) -> np.ndarray:
    return np.repeat(np.asarray(t, dtype=np.float32), g, axis=1)[:, :K]


def dequant(codes_unpacked: np.ndarray, scales, zeros, group_size: int, out_dtype=np.float16) -> np.ndarray:
    """ops/quant_ops.py:191-212 / 256-276: (q - z) * s in fp32 (q * s without
    zeros), then one rounding into out_dtype."""
    q = codes_unpacked.astype(np.float32)
    K = q.shape[1]
    s = _expand(scales, group_size, K)
    w = q * s if zeros is None else (q - _expand(zeros, group_size, K)) * s
    return w.astype(out_dtype)


def dequant_q4(packed, scales, zeros=None, group_size=32, out_dtype=np.float16):
    return dequant(unpack_q4(packed), scales, zeros, group_size, out_dtype)


def dequant_q8(q, scales, zeros=None, group_size=32, out_dtype=np.float16):
    return dequant(np.asarray(q, dtype=np.uint8), scales, zeros, group_size, out_dtype)


BF16_MAX = 3.3895313892515355e38


def round_bf16(v: np.ndarray) -> np.ndarray:
    """fp32 -> nearest-even bfloat16, returned as fp32 (numpy has no bf16).
    NaN/inf are passed through."""
    f = np.ascontiguousarray(v, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32).view(np.float32)
    return np.where(np.isfinite(f), r, f)


def _cast(v: np.ndarray, act: str) -> np.ndarray:
    return v.astype(np.float16) if act == "f16" else round_bf16(v.astype(np.float32))


def matvec(x: np.ndarray, W_deq: np.ndarray, act: str = "f16") -> np.ndarray:
    """ops/quant_ops.py:509-526: fp32 matmul of x with W already rounded to
    x's dtype, clipped to the finite range of x's dtype, cast to it.
    act="bf16" returns bf16 values held in fp32."""
    y = x.astype(np.float32) @ np.asarray(W_deq, dtype=np.float32).T
    m = F16_MAX if act == "f16" else BF16_MAX
    return _cast(np.clip(y, -m, m), act)


def _deq_act(codes_unpacked, scales, zeros, group_size, act):
    w = dequant(codes_unpacked, scales, zeros, group_size, np.float32)
    return w.astype(np.float16) if act == "f16" else round_bf16(w)


# Dequantized weights of q4_matvec / q8_matvec, reused while a
# memoized_dequant() block is open: keyed by the identity of the code, scale
# and zero arrays (held by the memo, so the keys stay unique), for tests that
# run one weight set many times (a deep stack whose layers share weights).
_DEQ_MEMO = None


@contextlib.contextmanager
def memoized_dequant():
    global _DEQ_MEMO
    _DEQ_MEMO = {}
    try:
        yield
    finally:
        _DEQ_MEMO = None


def _deq_cached(make, arrays, key):
    if _DEQ_MEMO is None:
        return make()
    k = tuple(id(a) for a in arrays) + key
    if k not in _DEQ_MEMO:
        _DEQ_MEMO[k] = (make().astype(np.float32), arrays)
    return _DEQ_MEMO[k][0]


def q4_matvec(x, packed, scales, zeros=None, group_size=32, act="f16"):
    """ops/quant_ops.py:509-526 (W rounded to the activation dtype)."""
    K = x.shape[1]
    W = _deq_cached(lambda: _deq_act(unpack_q4(packed, K), scales, zeros, group_size, act), (packed, scales, zeros),
                    ("q4", K, group_size, act))
    return matvec(x, W, act)


def q8_matvec(x, q, scales, zeros=None, group_size=32, act="f16"):
    """ops/quant_ops.py:574-588."""
    W = _deq_cached(lambda: _deq_act(np.asarray(q, dtype=np.uint8), scales, zeros, group_size, act), (q, scales, zeros),
                    ("q8", group_size, act))
    return matvec(x, W, act)


def q4_matvec_w32(x, packed, scales, zeros=None, group_size=32, act="f16"):
    """The reference's Metal matvec backends (ops/quant_ops.py:529-571 running
    kernels/q4_matvec_decode.metal:17-28): w = (q - z) s kept in fp32, fp32
    accumulation, one rounding of each sum into x's dtype (clipped to its
    finite range, as the HIP kernels saturate).  It differs from q4_matvec,
    the pure-array reference, only by that path's fp16 rounding of W."""
    K = x.shape[1]
    return matvec(x, dequant(unpack_q4(packed, K), scales, zeros, group_size, np.float32), act)


def q8_matvec_w32(x, q, scales, zeros=None, group_size=32, act="f16"):
    """kernels/q8_matvec_decode.metal: the q8 twin of q4_matvec_w32."""
    return matvec(x, dequant(np.asarray(q, dtype=np.uint8), scales, zeros, group_size, np.float32), act)


def swiglu(gate: np.ndarray, up: np.ndarray, act: str = "f16") -> np.ndarray:
    """ops/activation_ops.py:83-88: g / (1 + exp(-g)) * u in fp32."""
    g = gate.astype(np.float32)
    return _cast(g / (np.float32(1.0) + np.exp(-g)) * up.astype(np.float32), act)


def residual_add(x: np.ndarray, r: np.ndarray) -> np.ndarray:
    """ops/fused_ops.py:149-152."""
    return (x.astype(np.float32) + r.astype(np.float32)).astype(x.dtype)


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    """ops/norm_ops.py:47-52: x * rsqrt(mean(x^2) + eps) * w in fp32."""
    xf = x.astype(np.float32)
    inv = np.float32(1.0) / np.sqrt(np.mean(xf * xf, axis=-1, keepdims=True) + np.float32(eps))
    return (xf * inv * w.astype(np.float32)).astype(x.dtype)


def mlp_block(x, residual, norm_w, gate, up, down, bits=4, group_size=32, eps=1e-5, intermediates=False,
              w32=False):
    """ops/mlp_block_ops.py:258-364: gate/up/down are (codes, scales, zeros)
    triples; x, residual [rows, D] fp16.  w32=False is the reference preset
    (:258-298, the pure-array matvecs, W rounded to fp16); w32=True the Metal
    presets (:301-364 with matvec backends metal_*), whose kernels keep W in
    fp32 (q4_matvec_w32 / q8_matvec_w32).  A pair (gate_up, down) picks the
    semantics per projection."""
    w32_gu, w32_dn = (w32, w32) if isinstance(w32, bool) else w32
    pick = lambda exact: ((q4_matvec_w32 if bits == 4 else q8_matvec_w32) if exact
                          else (q4_matvec if bits == 4 else q8_matvec))
    z = residual_add(x, residual)
    n = rms_norm(z, norm_w, eps)
    g = pick(w32_gu)(n, *gate, group_size=group_size)
    u = pick(w32_gu)(n, *up, group_size=group_size)
    m = swiglu(g, u)
    d = pick(w32_dn)(m, *down, group_size=group_size)
    out = residual_add(z, d)
    if intermediates:
        return out, {"z": z, "normed": n, "gate": g, "up": u, "mlp": m, "down": d}
    return out


def quantize_weight_groupwise(weight: np.ndarray, bits: int = 4, group_size: int = 32, eps: float = 1e-8):
    """models/quantize_weights.py:164-203: symmetric absmax per group,
    scale = max(max|w| / limit, eps) (Python float, then fp32 for the
    divide), codes rint(w / scale) clipped to +-limit plus zero point 8/128.
    Returns (packed_or_codes uint8, scales fp32 [out, G])."""
    w = np.asarray(weight, dtype=np.float32)
    out_dim, in_dim = w.shape
    G = math.ceil(in_dim / group_size)
    limit = 7 if bits == 4 else 127
    zp = 8 if bits == 4 else 128
    pad = G * group_size - in_dim
    wp = np.pad(w, ((0, 0), (0, pad))) if pad else w
    max_abs = np.abs(wp.reshape(out_dim, G, group_size)).max(axis=-1).astype(np.float64)
    scale64 = np.maximum(max_abs / float(limit), eps)
    scale32 = scale64.astype(np.float32)
    q = np.clip(np.rint(w / np.repeat(scale32, group_size, axis=1)[:, :in_dim]), -limit, limit)
    codes = (q.astype(np.int32) + zp).astype(np.uint8)
    return (pack_q4(codes) if bits == 4 else codes), scale32
