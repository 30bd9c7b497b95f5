"""Groupwise-affine q4/q8 pack, dequant and decode matvec -- drop-in for the
reference's ``ops/quant_ops.py`` over ``torch.Tensor``.

Every public name, argument, default, return arity and error message follows
the reference (file:line cited per function).  Backend names:

* ``"reference"`` -- the pure tensor-op path (the reference's pure-MLX
  ``reference_*`` functions restated with torch ops; runs on any device);
* ``"metal"``, ``"metal_parallel"``, ``"metal_tiled"``, ``"auto"`` -- accepted
  for drop-in compatibility and all run the single gfx950 HIP kernel of the op
  (``libmk_hip.so``).  They never fall back: a missing library or host tensors
  raise.

``MLX_METAL_CI_SAFE_MODE=1`` keeps the reference's explicit opt-in that routes
kernel backends to ``reference_*`` (ops/quant_ops.py:33-34).
"""

from __future__ import annotations

import math
import os

import torch

from . import _lib
from ._common import ACT_DTYPES, as_u8, ci_safe_mode_enabled, finfo_max, scales_for_kernel

_MATVEC_BACKENDS_MSG = "backend must be one of 'reference', 'metal', 'metal_parallel', 'metal_tiled', 'auto'"


def _ci_safe_mode_enabled() -> bool:
    return ci_safe_mode_enabled()


def _normalize_out_dtype(out_dtype):
    """ops/quant_ops.py:147-152."""
    if out_dtype is None:
        return torch.float16
    if out_dtype not in ACT_DTYPES:
        raise TypeError(f"out_dtype must be float16 or bfloat16, got {out_dtype}")
    return out_dtype


def _validate_group_params(M: int, K: int, scales, zeros, group_size: int):
    """ops/quant_ops.py:155-163."""
    if group_size <= 0:
        raise ValueError("group_size must be positive")
    groups = math.ceil(K / group_size)
    if tuple(scales.shape) != (M, groups):
        raise ValueError(f"scales must have shape {(M, groups)}, got {tuple(scales.shape)}")
    if zeros is not None and tuple(zeros.shape) != (M, groups):
        raise ValueError(f"zeros must have shape {(M, groups)}, got {tuple(zeros.shape)}")
    return groups


# ----------------------------------------------------------------- pack / unpack


def _pack_q4_torch(q_int: torch.Tensor) -> torch.Tensor:
    if q_int.shape[1] % 2 != 0:
        pad = torch.zeros((q_int.shape[0], 1), dtype=torch.uint8, device=q_int.device)
        q_int = torch.cat([q_int, pad], dim=1)
    low = q_int[:, 0::2]
    high = q_int[:, 1::2]
    return (low + (high << 4)).to(torch.uint8)


def pack_q4(q_unpacked: torch.Tensor) -> torch.Tensor:
    """ops/quant_ops.py:166-176: packed[m, j] = q[m, 2j] + (q[m, 2j+1] << 4)
    (uint8 arithmetic), odd K padded with a zero code.  Device tensors are
    packed by the HIP kernel, host tensors with tensor ops."""
    if q_unpacked.ndim != 2:
        raise ValueError(f"q_unpacked must be 2-D [M,K], got {tuple(q_unpacked.shape)}")
    q_int = as_u8(q_unpacked)
    if q_int.device.type != "cuda":
        return _pack_q4_torch(q_int)
    rows, K = q_int.shape
    out = torch.empty((rows, (K + 1) // 2), dtype=torch.uint8, device=q_int.device)
    _lib.launch("mk_pack_q4", q_int.device, _lib.ptr(q_int), _lib.ptr(out), rows, K)
    return out


def unpack_q4_reference(packed: torch.Tensor, K: int | None = None) -> torch.Tensor:
    """ops/quant_ops.py:179-188: low nibble -> even column, high -> odd."""
    if packed.ndim != 2:
        raise ValueError(f"packed must be 2-D [M,K_packed], got {tuple(packed.shape)}")
    p = packed.to(torch.uint8)
    low = p & 0x0F
    high = (p >> 4) & 0x0F
    unpacked = torch.stack([low, high], dim=-1).reshape(p.shape[0], p.shape[1] * 2)
    if K is not None:
        unpacked = unpacked[:, :K]
    return unpacked.to(torch.uint8)


def unpack_q4(packed: torch.Tensor, K: int | None = None) -> torch.Tensor:
    """HIP twin of ``unpack_q4_reference`` for device tensors."""
    if packed.ndim != 2:
        raise ValueError(f"packed must be 2-D [M,K_packed], got {tuple(packed.shape)}")
    p = as_u8(packed)
    rows, kp = p.shape
    k_out = 2 * kp if K is None else min(int(K), 2 * kp)
    out = torch.empty((rows, k_out), dtype=torch.uint8, device=p.device)
    _lib.launch("mk_unpack_q4", _lib.require_device(p), _lib.ptr(p), _lib.ptr(out), rows, kp, k_out)
    return out


# ----------------------------------------------------------------- dequant


def _expand_groups(t: torch.Tensor, group_size: int, K: int) -> torch.Tensor:
    return torch.repeat_interleave(t.to(torch.float32), group_size, dim=1)[:, :K]


def reference_dequant_q4(packed, scales, zeros=None, *, group_size: int = 32, out_dtype=None):
    """ops/quant_ops.py:191-212."""
    if packed.ndim != 2:
        raise ValueError(f"packed must be 2-D [M,K_packed], got {tuple(packed.shape)}")
    out_dtype = _normalize_out_dtype(out_dtype)
    M, K_packed = packed.shape
    K = K_packed * 2
    _validate_group_params(M, K, scales, zeros, group_size)
    q = unpack_q4_reference(packed, K=K).to(torch.float32)
    scale_full = _expand_groups(scales, group_size, K)
    if zeros is None:
        out = q * scale_full
    else:
        out = (q - _expand_groups(zeros, group_size, K)) * scale_full
    return out.to(out_dtype)


def _hip_dequant(name, codes, scales, zeros, rows, k_arg, group_size, out_dtype, K):
    codes = as_u8(codes)
    dev = _lib.require_device(codes, scales, zeros)
    s, z = scales_for_kernel(scales, zeros)
    out = torch.empty((rows, K), dtype=out_dtype, device=dev)
    _lib.launch(name, dev, _lib.ptr(codes), _lib.ptr(s), _lib.ptr(z), _lib.ptr(out), rows, k_arg,
                group_size, _lib.dtype_code(s.dtype), _lib.dtype_code(out_dtype))
    return out


def dequant_q4(packed, scales, zeros=None, *, group_size: int = 32, out_dtype=None, backend: str = "auto"):
    """ops/quant_ops.py:215-253."""
    if packed.ndim != 2:
        raise ValueError(f"packed must be 2-D [M,K_packed], got {tuple(packed.shape)}")
    out_dtype = _normalize_out_dtype(out_dtype)
    M, K_packed = packed.shape
    K = K_packed * 2
    _validate_group_params(M, K, scales, zeros, group_size)
    backend_name = backend.lower()
    if backend_name == "auto":
        backend_name = "metal"
    if _ci_safe_mode_enabled() or backend_name == "reference":
        return reference_dequant_q4(packed, scales, zeros, group_size=group_size, out_dtype=out_dtype)
    if backend_name != "metal":
        raise ValueError("backend must be one of 'reference', 'metal', 'auto'")
    return _hip_dequant("mk_dequant_q4", packed, scales, zeros, M, K_packed, group_size, out_dtype, K)


def reference_dequant_q8(q, scales, zeros=None, *, group_size: int = 32, out_dtype=None):
    """ops/quant_ops.py:256-276."""
    if q.ndim != 2:
        raise ValueError(f"q must be 2-D [M,K], got {tuple(q.shape)}")
    out_dtype = _normalize_out_dtype(out_dtype)
    M, K = q.shape
    _validate_group_params(M, K, scales, zeros, group_size)
    q_f = q.to(torch.float32)
    scale_full = _expand_groups(scales, group_size, K)
    if zeros is None:
        out = q_f * scale_full
    else:
        out = (q_f - _expand_groups(zeros, group_size, K)) * scale_full
    return out.to(out_dtype)


def dequant_q8(q, scales, zeros=None, *, group_size: int = 32, out_dtype=None, backend: str = "auto"):
    """ops/quant_ops.py:279-316."""
    if q.ndim != 2:
        raise ValueError(f"q must be 2-D [M,K], got {tuple(q.shape)}")
    out_dtype = _normalize_out_dtype(out_dtype)
    M, K = q.shape
    _validate_group_params(M, K, scales, zeros, group_size)
    backend_name = backend.lower()
    if backend_name == "auto":
        backend_name = "metal"
    if _ci_safe_mode_enabled() or backend_name == "reference":
        return reference_dequant_q8(q, scales, zeros, group_size=group_size, out_dtype=out_dtype)
    if backend_name != "metal":
        raise ValueError("backend must be one of 'reference', 'metal', 'auto'")
    return _hip_dequant("mk_dequant_q8", q, scales, zeros, M, K, group_size, out_dtype, K)


def groupwise_dequant(q, scales, zeros=None, *, bits, group_size: int = 32, out_dtype=None, backend: str = "auto"):
    """ops/quant_ops.py:319-333."""
    if bits == 4:
        return dequant_q4(q, scales, zeros, group_size=group_size, out_dtype=out_dtype, backend=backend)
    if bits == 8:
        return dequant_q8(q, scales, zeros, group_size=group_size, out_dtype=out_dtype, backend=backend)
    raise ValueError(f"bits must be 4 or 8, got {bits}")


# ----------------------------------------------------------------- shape helpers


def _normalize_x_2d(x):
    """ops/quant_ops.py:336-342."""
    if x.ndim == 2:
        return x, x.shape[0], x.shape[1]
    if x.ndim == 3 and x.shape[1] == 1:
        squeezed = x[:, 0, :]
        return squeezed, squeezed.shape[0], squeezed.shape[1]
    raise ValueError(f"x must have shape [B,K] or [B,1,K], got {tuple(x.shape)}")


def _validate_matvec_input_dtype(x2d):
    """ops/quant_ops.py:345-347."""
    if x2d.dtype not in ACT_DTYPES:
        raise TypeError(f"x dtype must be float16 or bfloat16, got {x2d.dtype}")


def _normalize_hidden_rows_input(x):
    """ops/quant_ops.py:350-356."""
    if x.ndim == 2:
        return x, tuple(x.shape), x.shape[0], x.shape[1]
    if x.ndim == 3:
        rows = x.shape[0] * x.shape[1]
        return x.reshape(rows, x.shape[2]), tuple(x.shape), rows, x.shape[2]
    raise ValueError(f"x must have shape [rows,K] or [B,S,K], got {tuple(x.shape)}")


def _restore_hidden_rows_output(y2d, original_shape):
    """ops/quant_ops.py:359-362."""
    if len(original_shape) == 2:
        return y2d
    return y2d.reshape(tuple(original_shape[:-1]) + (y2d.shape[-1],))


def _validate_gate_up_shapes(x2d, gate_w, up_w, gate_scales, up_scales, gate_zeros, up_zeros, *, bits, group_size):
    """ops/quant_ops.py:372-404."""
    _validate_matvec_input_dtype(x2d)
    if bits not in (4, 8):
        raise ValueError(f"bits must be 4 or 8, got {bits}")
    rows, k_dim = x2d.shape
    if gate_w.ndim != 2 or up_w.ndim != 2:
        raise ValueError(f"gate_w and up_w must be 2-D, got {tuple(gate_w.shape)}, {tuple(up_w.shape)}")
    if gate_w.shape != up_w.shape:
        raise ValueError(f"gate_w and up_w must have identical shapes, got {tuple(gate_w.shape)}, {tuple(up_w.shape)}")
    out_dim = gate_w.shape[0]
    if bits == 4:
        expected_cols = math.ceil(k_dim / 2)
        if gate_w.shape[1] != expected_cols:
            raise ValueError(f"q4 gate/up weights must have shape [{out_dim},{expected_cols}], got {tuple(gate_w.shape)}")
    else:
        if gate_w.shape[1] != k_dim:
            raise ValueError(f"q8 gate/up weights must have shape [{out_dim},{k_dim}], got {tuple(gate_w.shape)}")
    groups = _validate_group_params(out_dim, k_dim, gate_scales, gate_zeros, group_size)
    up_groups = _validate_group_params(out_dim, k_dim, up_scales, up_zeros, group_size)
    if groups != up_groups:
        raise ValueError(f"gate and up scale group counts must match, got {groups} and {up_groups}")
    return rows, k_dim, out_dim


# ----------------------------------------------------------------- matvec


def _hip_matvec(bits, x2d, w, scales, zeros, group_size, residual=None, want_mm=False):
    """Launch mk_q{4,8}_matvec.  Returns y (or (y_mm, y_out) with a residual)."""
    x2d = x2d.contiguous()
    w = as_u8(w)
    dev = _lib.require_device(x2d, w, scales, zeros, residual)
    s, z = scales_for_kernel(scales, zeros)
    M, K = x2d.shape
    N = w.shape[0]
    name = "mk_q4_matvec" if bits == 4 else "mk_q8_matvec"
    if residual is None:
        y = torch.empty((M, N), dtype=x2d.dtype, device=dev)
        _lib.launch(name, dev, _lib.ptr(x2d), _lib.ptr(w), _lib.ptr(s), _lib.ptr(z), None, None,
                    _lib.ptr(y), M, N, K, group_size, _lib.dtype_code(x2d.dtype), _lib.dtype_code(s.dtype))
        return y
    residual = residual.to(x2d.dtype).contiguous()
    y_out = torch.empty((M, N), dtype=x2d.dtype, device=dev)
    y_mm = torch.empty((M, N), dtype=x2d.dtype, device=dev) if want_mm else None
    _lib.launch(name, dev, _lib.ptr(x2d), _lib.ptr(w), _lib.ptr(s), _lib.ptr(z), _lib.ptr(residual),
                _lib.ptr(y_mm), _lib.ptr(y_out), M, N, K, group_size, _lib.dtype_code(x2d.dtype),
                _lib.dtype_code(s.dtype))
    return y_mm, y_out


def reference_q4_matvec_decode(x, packed_w, scales, zeros=None, *, group_size: int = 32):
    """ops/quant_ops.py:509-526: fp32 matmul of x with W dequantized and
    rounded to x's dtype, clipped to the finite range of x's dtype."""
    x2d, B, K = _normalize_x_2d(x)
    if packed_w.ndim != 2:
        raise ValueError(f"packed_w must be 2-D [N,K_packed], got {tuple(packed_w.shape)}")
    N, K_packed = packed_w.shape
    if K_packed * 2 != K:
        raise ValueError(f"packed_w implies K={K_packed * 2}, but x has K={K}")
    W = reference_dequant_q4(packed_w, scales, zeros, group_size=group_size, out_dtype=x2d.dtype)
    result = torch.matmul(x2d.to(torch.float32), W.to(torch.float32).t())
    m = finfo_max(x2d.dtype)
    return torch.clamp(result, -m, m).to(x2d.dtype)


def q4_matvec_decode(x, packed_w, scales, zeros=None, *, group_size: int = 32, backend: str = "auto"):
    """ops/quant_ops.py:529-571."""
    x2d, B, K = _normalize_x_2d(x)
    _validate_matvec_input_dtype(x2d)
    if packed_w.ndim != 2:
        raise ValueError(f"packed_w must be 2-D [N,K_packed], got {tuple(packed_w.shape)}")
    N, K_packed = packed_w.shape
    if K_packed * 2 != K:
        raise ValueError(f"packed_w implies K={K_packed * 2}, but x has K={K}")
    _validate_group_params(N, K, scales, zeros, group_size)
    backend_name = backend.lower()
    if backend_name == "auto":
        backend_name = "metal_tiled" if os.environ.get("MLX_METAL_USE_TILED_MATVEC", "0") == "1" else "metal"
    if backend_name == "reference" or _ci_safe_mode_enabled():
        return reference_q4_matvec_decode(x2d, packed_w, scales, zeros, group_size=group_size)
    if backend_name not in ("metal", "metal_parallel", "metal_tiled"):
        raise ValueError(_MATVEC_BACKENDS_MSG)
    return _hip_matvec(4, x2d, packed_w, scales, zeros, group_size)


def reference_q8_matvec_decode(x, q_w, scales, zeros=None, *, group_size: int = 32):
    """ops/quant_ops.py:574-588."""
    x2d, _, K = _normalize_x_2d(x)
    if q_w.ndim != 2 or q_w.shape[1] != K:
        raise ValueError(f"q_w must have shape [N,{K}], got {tuple(q_w.shape)}")
    W = reference_dequant_q8(q_w, scales, zeros, group_size=group_size, out_dtype=x2d.dtype)
    result = torch.matmul(x2d.to(torch.float32), W.to(torch.float32).t())
    m = finfo_max(x2d.dtype)
    return torch.clamp(result, -m, m).to(x2d.dtype)


def q8_matvec_decode(x, q_w, scales, zeros=None, *, group_size: int = 32, backend: str = "auto"):
    """ops/quant_ops.py:591-631."""
    x2d, B, K = _normalize_x_2d(x)
    _validate_matvec_input_dtype(x2d)
    if q_w.ndim != 2 or q_w.shape[1] != K:
        raise ValueError(f"q_w must have shape [N,{K}], got {tuple(q_w.shape)}")
    N = q_w.shape[0]
    _validate_group_params(N, K, scales, zeros, group_size)
    backend_name = backend.lower()
    if backend_name == "auto":
        backend_name = "metal_tiled" if os.environ.get("MLX_METAL_USE_TILED_MATVEC", "0") == "1" else "metal"
    if backend_name == "reference" or _ci_safe_mode_enabled():
        return reference_q8_matvec_decode(x2d, q_w, scales, zeros, group_size=group_size)
    if backend_name not in ("metal", "metal_parallel", "metal_tiled"):
        raise ValueError(_MATVEC_BACKENDS_MSG)
    return _hip_matvec(8, x2d, q_w, scales, zeros, group_size)


def q_matvec_residual(x, w, scales, zeros, residual, *, bits: int, group_size: int, want_mm: bool = False):
    """x @ W^T with the residual add fused into the epilogue:
    returns (y_mm or None, residual + y_mm).  Used by the MLP block's down
    projection (ops/mlp_block_ops.py:360-361); no standalone reference op."""
    x2d, _, _, _ = _normalize_hidden_rows_input(x)
    _validate_matvec_input_dtype(x2d)
    res2d = residual.reshape(x2d.shape[0], -1)
    return _hip_matvec(bits, x2d, w, scales, zeros, group_size, residual=res2d, want_mm=want_mm)


# ----------------------------------------------------------------- gate / up


def _hip_gate_up(bits, x, gate_w, up_w, gate_scales, up_scales, gate_zeros, up_zeros, group_size,
                 want_gate=True, want_up=True, want_mlp=False):
    x2d, original_shape, rows, k_dim = _normalize_hidden_rows_input(x)
    _, _, out_dim = _validate_gate_up_shapes(x2d, gate_w, up_w, gate_scales, up_scales, gate_zeros, up_zeros,
                                             bits=bits, group_size=group_size)
    x2d = x2d.contiguous()
    gw, uw = as_u8(gate_w), as_u8(up_w)
    dev = _lib.require_device(x2d, gw, uw, gate_scales, up_scales, gate_zeros, up_zeros)
    # both streams share one scale dtype
    all_f16 = all(t is None or t.dtype == torch.float16 for t in (gate_scales, up_scales, gate_zeros, up_zeros))
    tgt = torch.float16 if all_f16 else torch.float32

    def cvt(t):
        return None if t is None else t.to(tgt).contiguous()

    sg, su, zg, zu = cvt(gate_scales), cvt(up_scales), cvt(gate_zeros), cvt(up_zeros)
    outs = []
    gate = torch.empty((rows, out_dim), dtype=x2d.dtype, device=dev) if want_gate else None
    up = torch.empty((rows, out_dim), dtype=x2d.dtype, device=dev) if want_up else None
    mlp = torch.empty((rows, out_dim), dtype=x2d.dtype, device=dev) if want_mlp else None
    name = "mk_q4_gate_up" if bits == 4 else "mk_q8_gate_up"
    _lib.launch(name, dev, _lib.ptr(x2d), _lib.ptr(gw), _lib.ptr(uw), _lib.ptr(sg), _lib.ptr(su),
                _lib.ptr(zg), _lib.ptr(zu), _lib.ptr(gate), _lib.ptr(up), _lib.ptr(mlp), rows, out_dim,
                k_dim, group_size, _lib.dtype_code(x2d.dtype), _lib.dtype_code(tgt))
    for t in (gate, up, mlp):
        outs.append(None if t is None else _restore_hidden_rows_output(t, original_shape))
    return tuple(outs)


def q4_gate_up_matvec_tiled(x, gate_packed, up_packed, gate_scales, up_scales, gate_zeros=None, up_zeros=None, *,
                            group_size: int = 32):
    """ops/quant_ops.py:634-685: (gate, up) from one read of x.  Like the
    reference, this op has no CI-safe fallback."""
    gate, up, _ = _hip_gate_up(4, x, gate_packed, up_packed, gate_scales, up_scales, gate_zeros, up_zeros,
                               group_size)
    return gate, up


def q8_gate_up_matvec_tiled(x, gate_q, up_q, gate_scales, up_scales, gate_zeros=None, up_zeros=None, *,
                            group_size: int = 32):
    """ops/quant_ops.py:688-738."""
    gate, up, _ = _hip_gate_up(8, x, gate_q, up_q, gate_scales, up_scales, gate_zeros, up_zeros, group_size)
    return gate, up


def q_rmsnorm_gate_up_swiglu(x, residual, norm_weight, gate_w, up_w, gate_scales, up_scales, gate_zeros=None,
                             up_zeros=None, *, bits: int = 4, group_size: int = 32, eps: float = 1e-5,
                             return_gate_up: bool = False):
    """The front of the MLP block (ops/mlp_block_ops.py:343-356): z = x +
    residual, normed = rms_norm(z) * norm_weight, then gate/up and the SwiGLU
    epilogue -- one HIP launch for a q4 decode row (the norm runs inside the
    gate/up kernel), else the norm and gate/up kernels in turn.  Returns
    ``(z, normed, mlp)`` or ``(z, normed, gate, up, mlp)``."""
    if x.shape != residual.shape:
        raise ValueError(f"x and residual must have identical shapes, got {tuple(x.shape)}, {tuple(residual.shape)}")
    x2d, original_shape, rows, k_dim = _normalize_hidden_rows_input(x)
    _validate_matvec_input_dtype(x2d)
    if tuple(norm_weight.shape) != (k_dim,):
        raise ValueError(f"norm_weight must have shape {(k_dim,)}, got {tuple(norm_weight.shape)}")
    _, _, out_dim = _validate_gate_up_shapes(x2d, gate_w, up_w, gate_scales, up_scales, gate_zeros, up_zeros,
                                             bits=bits, group_size=group_size)
    x2d = x2d.contiguous()
    r2d = residual.reshape(rows, k_dim).to(x2d.dtype).contiguous()
    nw = norm_weight.contiguous()
    gw, uw = as_u8(gate_w), as_u8(up_w)
    dev = _lib.require_device(x2d, r2d, nw, gw, uw, gate_scales, up_scales, gate_zeros, up_zeros)
    all_f16 = all(t is None or t.dtype == torch.float16 for t in (gate_scales, up_scales, gate_zeros, up_zeros))
    tgt = torch.float16 if all_f16 else torch.float32

    def cvt(t):
        return None if t is None else t.to(tgt).contiguous()

    sg, su, zg, zu = cvt(gate_scales), cvt(up_scales), cvt(gate_zeros), cvt(up_zeros)
    z = torch.empty_like(x2d)
    normed = torch.empty_like(x2d)
    gate = torch.empty((rows, out_dim), dtype=x2d.dtype, device=dev) if return_gate_up else None
    up = torch.empty((rows, out_dim), dtype=x2d.dtype, device=dev) if return_gate_up else None
    mlp = torch.empty((rows, out_dim), dtype=x2d.dtype, device=dev)
    name = "mk_q4_rmsnorm_gate_up" if bits == 4 else "mk_q8_rmsnorm_gate_up"
    _lib.launch(name, dev, _lib.ptr(x2d), _lib.ptr(r2d), _lib.ptr(nw), float(eps), _lib.ptr(gw), _lib.ptr(uw),
                _lib.ptr(sg), _lib.ptr(su), _lib.ptr(zg), _lib.ptr(zu), _lib.ptr(z), _lib.ptr(normed),
                _lib.ptr(gate), _lib.ptr(up), _lib.ptr(mlp), rows, out_dim, k_dim, group_size,
                _lib.dtype_code(x2d.dtype), _lib.dtype_code(tgt), _lib.dtype_code(nw.dtype))
    outs = [z.reshape(x.shape), normed.reshape(x.shape)]
    if return_gate_up:
        outs += [_restore_hidden_rows_output(gate, original_shape), _restore_hidden_rows_output(up, original_shape)]
    outs.append(_restore_hidden_rows_output(mlp, original_shape))
    return tuple(outs)


def q_rmsnorm_matvec(x, norm_weight, w, scales, zeros=None, *, bits: int = 4, group_size: int = 32,
                     eps: float = 1e-5, return_normed: bool = False):
    """RMSNorm then the q4/q8 matvec, y = rms_norm(x) . W^T with the norm
    rounded to x's dtype first (ops/norm_ops.py:47-52 feeding
    ops/quant_ops.py:509-631) -- the decode layer's input norm + qkv
    projection and the stack's final norm + head.  One HIP launch for a q4
    fp16 decode row, the norm kernel then the matvec otherwise.  Returns y
    [rows, N] (and the normalised rows with ``return_normed``)."""
    x2d, original_shape, rows, k_dim = _normalize_hidden_rows_input(x)
    _validate_matvec_input_dtype(x2d)
    if tuple(norm_weight.shape) != (k_dim,):
        raise ValueError(f"norm_weight must have shape {(k_dim,)}, got {tuple(norm_weight.shape)}")
    if bits not in (4, 8):
        raise ValueError(f"bits must be 4 or 8, got {bits}")
    w8 = as_u8(w)
    cols = math.ceil(k_dim / 2) if bits == 4 else k_dim
    if w8.ndim != 2 or w8.shape[1] != cols:
        raise ValueError(f"w must have shape [N,{cols}], got {tuple(w8.shape)}")
    N = w8.shape[0]
    _validate_group_params(N, k_dim, scales, zeros, group_size)
    x2d = x2d.contiguous()
    nw = norm_weight.contiguous()
    dev = _lib.require_device(x2d, nw, w8, scales, zeros)
    s, z = scales_for_kernel(scales, zeros)
    normed = torch.empty_like(x2d)
    y = torch.empty((rows, N), dtype=x2d.dtype, device=dev)
    name = "mk_q4_rmsnorm_matvec" if bits == 4 else "mk_q8_rmsnorm_matvec"
    _lib.launch(name, dev, _lib.ptr(x2d), _lib.ptr(nw), float(eps), _lib.ptr(w8), _lib.ptr(s), _lib.ptr(z),
                _lib.ptr(normed), _lib.ptr(y), rows, N, k_dim, group_size, _lib.dtype_code(x2d.dtype),
                _lib.dtype_code(s.dtype), _lib.dtype_code(nw.dtype))
    y = _restore_hidden_rows_output(y, original_shape)
    if return_normed:
        return y, normed.reshape(x.shape)
    return y


def q_gate_up_swiglu(x, gate_w, up_w, gate_scales, up_scales, gate_zeros=None, up_zeros=None, *, bits: int = 4,
                     group_size: int = 32, return_gate_up: bool = False):
    """Gate/up projection with the SwiGLU epilogue fused in: silu(gate) * up
    computed from the rounded gate/up values (ops/activation_ops.py:83-88
    applied to the output of ops/quant_ops.py:634-738).  Returns ``mlp`` or
    ``(gate, up, mlp)``.  Extension of the reference API (its fused path runs
    gate/up and SwiGLU as two launches)."""
    gate, up, mlp = _hip_gate_up(bits, x, gate_w, up_w, gate_scales, up_scales, gate_zeros, up_zeros, group_size,
                                 want_gate=return_gate_up, want_up=return_gate_up, want_mlp=True)
    if return_gate_up:
        return gate, up, mlp
    return mlp
