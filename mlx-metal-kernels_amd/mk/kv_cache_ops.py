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
