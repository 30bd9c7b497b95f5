"""Position / token-shape normalisation shared by the paged ops -- the helper
part of ops/kv_cache_ops.py (:29-61)."""

from __future__ import annotations

import os

import torch


def _normalize_token_shape(x, name: str):
    """ops/kv_cache_ops.py:29-34: [B,H,D] -> [B,1,H,D]."""
    if x.ndim == 3:
        return x[:, None, :, :]
    if x.ndim == 4 and x.shape[1] == 1:
        return x
    raise ValueError(f"{name} must have shape [B,1,H,D] or [B,H,D], got {tuple(x.shape)}")


def host_checks_enabled(t: torch.Tensor) -> bool:
    """Whether the host-side range check may read device tensor ``t``.

    The reference reads positions back to the host on every call
    (ops/kv_cache_ops.py:55).  That read is a device synchronisation, and it
    is illegal while a HIP graph is being captured, so it is skipped for
    device tensors during capture and when MK_SKIP_DEVICE_RANGE_CHECKS=1.
    The kernels stay memory-safe without it: they skip positions and page
    ids outside the cache."""
    if t.device.type != "cuda":
        return True
    if os.environ.get("MK_SKIP_DEVICE_RANGE_CHECKS", "0") == "1":
        return False
    return not torch.cuda.is_current_stream_capturing()


def normalize_positions(positions, B: int, MAX_S: int, *, device=None) -> torch.Tensor:
    """ops/kv_cache_ops.py:37-61: scalar / list / tensor -> int32 [B], every
    value range-checked into [0, MAX_S) (a host read, as in the reference;
    see ``host_checks_enabled`` for when device tensors skip it).  The result
    lives on ``device`` (default: the input tensor's device, else the host)."""
    if isinstance(positions, bool):
        positions = int(positions)
    if isinstance(positions, int):
        pos = torch.full((B,), positions, dtype=torch.int32, device=device)
    elif isinstance(positions, torch.Tensor):
        dev = device if device is not None else positions.device
        if positions.ndim == 0:
            pos = positions.to(device=dev, dtype=torch.int32).reshape(1).expand(B).contiguous()
        elif positions.ndim == 1 and positions.shape[0] == B:
            pos = positions.to(device=dev, dtype=torch.int32)
        else:
            raise ValueError(f"positions must be scalar or shape [B], got {tuple(positions.shape)}")
    else:
        pos_arr = torch.as_tensor(positions, dtype=torch.int32)
        if pos_arr.ndim == 0:
            pos = torch.full((B,), int(pos_arr.item()), dtype=torch.int32, device=device)
        elif pos_arr.ndim == 1 and pos_arr.shape[0] == B:
            pos = pos_arr.to(device=device)
        else:
            raise ValueError(f"positions must be scalar or shape [B], got {tuple(pos_arr.shape)}")
    if host_checks_enabled(pos):
        for p in pos.tolist():
            if p < 0 or p >= MAX_S:
                raise ValueError(f"positions must be in [0, {MAX_S}), got {p}")
    return pos


# ----------------------------------------------------------------- contiguous update


def _validate_update_inputs(K_cache, V_cache, k_new, v_new, positions):
    """ops/kv_cache_ops.py:64-90."""
    if K_cache.ndim != 4 or V_cache.ndim != 4:
        raise ValueError(f"K_cache and V_cache must be 4-D [B,MAX_S,H,D], got {tuple(K_cache.shape)}, "
                         f"{tuple(V_cache.shape)}")
    if K_cache.shape != V_cache.shape:
        raise ValueError(f"K_cache and V_cache must have identical shapes, got {tuple(K_cache.shape)}, "
                         f"{tuple(V_cache.shape)}")
    k_new = _normalize_token_shape(k_new, "k_new")
    v_new = _normalize_token_shape(v_new, "v_new")
    B, MAX_S, H, D = K_cache.shape
    if tuple(k_new.shape) != (B, 1, H, D) or tuple(v_new.shape) != (B, 1, H, D):
        raise ValueError(
            "k_new and v_new must match cache batch/head/head_dim after normalization. "
            f"Got k_new={tuple(k_new.shape)}, v_new={tuple(v_new.shape)}, cache={tuple(K_cache.shape)}.")
    act = (torch.float16, torch.bfloat16)
    if K_cache.dtype not in act:
        raise TypeError(f"K_cache dtype must be float16 or bfloat16, got {K_cache.dtype}")
    if V_cache.dtype not in act:
        raise TypeError(f"V_cache dtype must be float16 or bfloat16, got {V_cache.dtype}")
    if k_new.dtype not in act or v_new.dtype not in act:
        raise TypeError(f"k_new/v_new dtype must be float16 or bfloat16, got {k_new.dtype}, {v_new.dtype}")
    pos = normalize_positions(positions, B, MAX_S, device=K_cache.device)
    return k_new, v_new, pos, B, MAX_S, H, D


def reference_kv_cache_update(K_cache, V_cache, k_new, v_new, positions):
    """ops/kv_cache_ops.py:93-107: a functional copy with row positions[b] of
    sequence b replaced by the new token."""
    k_new, v_new, pos, B, MAX_S, H, D = _validate_update_inputs(K_cache, V_cache, k_new, v_new, positions)
    idx = torch.arange(MAX_S, device=K_cache.device).reshape(1, MAX_S, 1, 1)
    mask = idx == pos.to(K_cache.device).long().reshape(B, 1, 1, 1)
    K_updated = torch.where(mask, k_new.to(K_cache.dtype).to(K_cache.device), K_cache)
    V_updated = torch.where(mask, v_new.to(V_cache.dtype).to(V_cache.device), V_cache)
    return K_updated, V_updated


def kv_cache_update(K_cache, V_cache, k_new, v_new, positions, *, backend: str = "auto", copy: bool = False):
    """ops/kv_cache_ops.py:110-150 over a contiguous cache [B, MAX_S, H, D].
    The HIP backend writes the B*H*D new elements in place through the paged
    update kernel over an identity-paged view of the cache and returns the
    same tensors (the reference returns new arrays that its callers rebind;
    ``copy=True`` updates fresh copies instead)."""
    from . import _contig, _lib
    from ._common import ci_safe_mode_enabled

    k_new, v_new, pos, B, MAX_S, H, D = _validate_update_inputs(K_cache, V_cache, k_new, v_new, positions)
    backend_name = backend.lower()
    if backend_name == "auto":
        backend_name = "metal"
    if ci_safe_mode_enabled() or backend_name == "reference":
        return reference_kv_cache_update(K_cache, V_cache, k_new, v_new, pos)
    if backend_name != "metal":
        raise ValueError("backend must be one of 'reference', 'metal', 'auto'")
    if K_cache.dtype != V_cache.dtype:
        raise TypeError(f"K_cache and V_cache must share a dtype, got {K_cache.dtype}, {V_cache.dtype}")
    dev = _lib.require_device(K_cache, V_cache)
    if copy:
        K_cache, V_cache = K_cache.clone(), V_cache.clone()
    P = _contig.page_size_for(MAX_S)
    Kp, Vp = _contig.as_pages(K_cache, P), _contig.as_pages(V_cache, P)
    bt = _contig.identity_table(B, MAX_S, P, dev)
    k = k_new.to(device=dev, dtype=K_cache.dtype).contiguous()
    v = v_new.to(device=dev, dtype=K_cache.dtype).contiguous()
    pos_d = pos.to(device=dev, dtype=torch.int32).contiguous()
    _lib.launch("mk_paged_kv_update", dev, _lib.ptr(Kp), _lib.ptr(Vp), _lib.ptr(k), _lib.ptr(v), _lib.ptr(bt),
                _lib.ptr(pos_d), B, H, D, P, MAX_S // P, Kp.shape[0], _lib.dtype_code(K_cache.dtype))
    return K_cache, V_cache
