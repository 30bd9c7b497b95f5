"""Contiguous KV caches as paged ones, without a copy.

A contiguous cache [B, MAX_S, H, X] (X = D for fp16/bf16 values, the code
bytes or scale groups for quantized ones) has exactly the memory layout of
B * MAX_S / P pages of P positions when P divides MAX_S: position j of
sequence b sits in page b * (MAX_S / P) + j // P, slot j % P.  The paged
kernels therefore serve the contiguous ops of the reference
(ops/decode_ops.py, ops/kv_cache_ops.py, ops/quantized_kv_cache_ops.py)
through a view and the identity block table of
ops/paged_kv_ops.py:99-105.
"""

from __future__ import annotations

import threading

import torch

_TABLES: dict = {}
_LOCK = threading.Lock()


def page_size_for(max_s: int) -> int:
    """The page size the view uses: 16 (the paged kernels' tile) when it
    divides MAX_S, else the largest power of two that does."""
    if max_s % 16 == 0:
        return 16
    p = 1
    while p < 16 and max_s % (2 * p) == 0:
        p *= 2
    return p


def as_pages(cache: torch.Tensor, page_size: int) -> torch.Tensor:
    """[B, MAX_S, H, X] -> [B * MAX_S / P, P, H, X] (a view of the same memory)."""
    if cache.ndim != 4:
        raise ValueError(f"cache must be 4-D [B,MAX_S,H,X], got {tuple(cache.shape)}")
    B, S, H, X = cache.shape
    if S % page_size:
        raise ValueError(f"page size {page_size} does not divide MAX_S={S}")
    if not cache.is_contiguous():
        raise ValueError("contiguous-cache kernels need a dense (contiguous) cache tensor")
    return cache.view(B * (S // page_size), page_size, H, X)


def identity_table(B: int, max_s: int, page_size: int, device) -> torch.Tensor:
    """The identity block table [B, MAX_S / P] (int32) on ``device``, built
    once per shape and device and reused: callers only read it."""
    key = (B, max_s, page_size, str(device))
    t = _TABLES.get(key)
    if t is None:
        with _LOCK:
            t = _TABLES.get(key)
            if t is None:
                mb = max_s // page_size
                t = (torch.arange(B, dtype=torch.int32, device=device).reshape(B, 1) * mb
                     + torch.arange(mb, dtype=torch.int32, device=device).reshape(1, mb))
                _TABLES[key] = t
    return t
