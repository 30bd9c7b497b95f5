"""Speculative-decoding verification of W draft tokens in one pass -- the
drop-in for ops/speculative_verify_ops.py.

The reference verifies K draft tokens with a staged decode loop
(ops/speculative_verify_ops.py:228-262): K full stack decode steps, step i at
position ``position + i`` on a cloned cache, each attending over the context
plus the drafts before it.  Here the K drafts run through the stack as K rows
of one pass: every projection is a K-row matvec (one read of each weight
matrix instead of K), every layer's fused front writes the K new K/V rows,
and the verify attention kernel (``mk_paged_verify_attention``) then serves
all K rows of a sequence from one read of its K/V: the K * Hq/Hkv query rows
of a kv head are the columns of one MFMA contraction, row i masked at
position ``position + i + 1`` -- the same causal structure in one attention
launch per layer.

Config, result, acceptance and commit helpers keep the reference's names,
fields and errors; ``cache_layout`` accepts "paged" as well as the
reference's "contiguous" (both run on the paged kernels).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Any

import numpy as np
import torch

from . import _lib
from .gqa_ops import reference_paged_gqa_decode_attention
from .kv_cache_ops import normalize_positions
from .llama_layer_ops import LlamaLikeConfig
from .llama_stack_ops import (LlamaStackCache, LlamaStackWeights, embed_token_ids, greedy_sample,
                              llama_stack_decode_step)
from . import _contig
from .paged_kv_ops import _i32
from .paged_quantized_kv_ops import PagedQuantizedKVCache, _check_kernel_layout, dequantize_kv_pages

_ACT = (torch.float16, torch.bfloat16)


# ------------------------------------------------------------ config / result


@dataclass
class ParallelVerificationConfig:
    """ops/speculative_verify_ops.py:26-59."""

    draft_length: int = 4
    mode: str = "greedy_exact"
    backend_preset: str = "fused_experimental"
    cache_layout: str = "contiguous"
    use_prefill_for_draft: bool = True
    return_logits: bool = True
    commit_cache: bool = False

    def validate(self) -> "ParallelVerificationConfig":
        if self.draft_length <= 0:
            raise ValueError(f"draft_length must be positive, got {self.draft_length}")
        if self.mode not in ("greedy_exact",):
            raise ValueError(f"mode must be 'greedy_exact', got {self.mode!r}")
        if self.cache_layout not in ("contiguous", "paged"):
            raise NotImplementedError(f"cache_layout={self.cache_layout!r} is not supported; "
                                      "'contiguous' and 'paged' are implemented")
        return self

    def to_dict(self) -> dict[str, Any]:
        return {"draft_length": self.draft_length, "mode": self.mode, "backend_preset": self.backend_preset,
                "cache_layout": self.cache_layout, "use_prefill_for_draft": self.use_prefill_for_draft,
                "return_logits": self.return_logits, "commit_cache": self.commit_cache}


@dataclass
class VerificationResult:
    """models/speculative_decoding.py:81-101."""

    proposed_token_ids: list[int]
    target_token_ids: list[int]
    accept_mask: list[bool]
    accepted_count: int
    rejected_count: int
    replacement_token_id: int | None = None
    metadata: dict[str, Any] = field(default_factory=dict)

    def accepted_tokens(self) -> list[int]:
        return [t for t, a in zip(self.proposed_token_ids, self.accept_mask) if a]

    def rejected_tokens(self) -> list[int]:
        return [t for t, a in zip(self.proposed_token_ids, self.accept_mask) if not a]

    def all_committed_tokens(self) -> list[int]:
        out = self.accepted_tokens()
        if self.replacement_token_id is not None and self.rejected_count > 0:
            out.append(self.replacement_token_id)
        return out


def compute_accept_mask(proposed_token_ids: list[int], target_token_ids: list[int], *,
                        require_exact_match: bool = True) -> list[bool]:
    """models/speculative_decoding.py:163-184: with exact matching a draft is
    accepted only while every earlier one was."""
    if not proposed_token_ids:
        return []
    mask: list[bool] = []
    for i in range(min(len(proposed_token_ids), len(target_token_ids))):
        match = proposed_token_ids[i] == target_token_ids[i]
        mask.append(match and (i == 0 or mask[-1]) if require_exact_match else match)
    return mask + [False] * (len(proposed_token_ids) - len(mask))


def accepted_prefix_length(accept_mask: list[bool]) -> int:
    """models/speculative_decoding.py:187-194."""
    n = 0
    for v in accept_mask:
        if not v:
            break
        n += 1
    return n


def verify_draft_tokens(proposed_token_ids: list[int], target_token_ids: list[int], *,
                        replacement_token_id: int | None = None, require_exact_match: bool = True
                        ) -> VerificationResult:
    """models/speculative_decoding.py:197-228."""
    if not proposed_token_ids:
        return VerificationResult([], target_token_ids, [], 0, 0)
    mask = compute_accept_mask(proposed_token_ids, target_token_ids, require_exact_match=require_exact_match)
    acc = accepted_prefix_length(mask)
    rej = len(proposed_token_ids) - acc
    if replacement_token_id is None and rej > 0 and acc < len(target_token_ids):
        replacement_token_id = int(target_token_ids[acc])
    return VerificationResult(list(proposed_token_ids), list(target_token_ids), mask, acc, rej, replacement_token_id)


@dataclass
class ParallelVerificationPassResult:
    """ops/speculative_verify_ops.py:67-99."""

    proposed_token_ids: list[int]
    target_token_ids: list[int]
    accept_mask: list[bool]
    accepted_count: int
    replacement_token_id: int | None = None
    logits: Any | None = None
    staged_cache: Any | None = None
    metadata: dict[str, Any] = field(default_factory=dict)

    def accepted_tokens(self) -> list[int]:
        return [t for t, a in zip(self.proposed_token_ids, self.accept_mask) if a]

    def committed_tokens(self) -> list[int]:
        out = self.accepted_tokens()
        if self.replacement_token_id is not None and len(self.accept_mask) > 0 and not all(self.accept_mask):
            out.append(self.replacement_token_id)
        return out

    def to_verification_result(self, require_exact_match: bool = True) -> VerificationResult:
        return verify_draft_tokens(self.proposed_token_ids, self.target_token_ids,
                                   replacement_token_id=self.replacement_token_id,
                                   require_exact_match=require_exact_match)


# ------------------------------------------------------------ token helpers


def embed_proposed_tokens(proposed_token_ids: list[int], embedding, *, B: int = 1):
    """ops/speculative_verify_ops.py:107-124: [1, K, hidden] rows of the
    embedding table (B = 1 only, as the reference)."""
    if B != 1:
        raise NotImplementedError("embed_proposed_tokens supports only B=1")
    ids = np.atleast_1d(np.asarray(proposed_token_ids, dtype=np.int64))
    if ids.shape[0] == 0:
        raise ValueError("proposed_token_ids must be non-empty")
    dev = embedding.device if isinstance(embedding, torch.Tensor) else None
    out = embed_token_ids(torch.from_numpy(ids).to(dev), embedding)
    return out.reshape(B, ids.shape[0], -1)


def target_tokens_from_verification_logits(logits_list: list, *, proposed_token_ids: list[int],
                                           mode: str = "greedy_exact") -> list[int]:
    """ops/speculative_verify_ops.py:132-152: the greedy target token of each
    verification row (first maximum)."""
    if mode != "greedy_exact":
        raise ValueError(f"mode must be 'greedy_exact', got {mode!r}")
    out = []
    for lg in logits_list:
        if isinstance(lg, torch.Tensor):
            out.append(int(torch.argmax(lg.reshape(-1)).item()))
        else:
            out.append(int(np.argmax(np.asarray(lg).ravel())))
    return out


# ------------------------------------------------------------ attention


def _verify_shapes(q, block_table, lengths, max_s):
    if q.ndim != 4:
        raise ValueError(f"q must have shape [B,W,Hq,D], got {tuple(q.shape)}")
    B, W = q.shape[:2]
    if block_table.ndim != 2 or block_table.shape[0] != B:
        raise ValueError(f"block_table must be [B,MAX_BLOCKS] with B={B}, got {tuple(block_table.shape)}")
    if W < 1 or W > 64:
        raise ValueError(f"verify width W must be in [1, 64], got {W}")
    ln = normalize_positions(lengths if lengths is not None else max_s, B, max_s + 1, device=block_table.device)
    return B, W, ln


def reference_paged_verify_attention(q, K_pages, V_pages, block_table, lengths=None, scale=None):
    """The attention of the staged verify loop on the torch reference path:
    row w is reference_paged_gqa_decode_attention (ops/gqa_ops.py:307-342)
    with lengths - (W - 1 - w) positions.  q [B,W,Hq,D] -> [B,W,Hq,D]."""
    max_s = block_table.shape[1] * K_pages.shape[1]
    B, W, ln = _verify_shapes(q, block_table, lengths, max_s)
    rows = []
    for w in range(W):
        lw = torch.clamp(torch.clamp(ln, max=max_s) - (W - 1 - w), min=0)
        rows.append(reference_paged_gqa_decode_attention(q[:, w:w + 1], K_pages, V_pages, block_table, lw, scale))
    return torch.cat(rows, dim=1)


def _hip_verify_attention(q, K_pages, V_pages, block_table, ln, scale: float):
    """mk_paged_verify_attention: q [B,W,Hq,D] over fp16/bf16 pages, one K/V
    read for all W rows of a sequence."""
    B, W, Hq, D = q.shape
    NUM_PAGES, P, Hkv, _ = K_pages.shape
    MAX_BLOCKS = block_table.shape[1]
    dev = _lib.require_device(q, K_pages, V_pages, block_table)
    dtype = K_pages.dtype
    if V_pages.dtype != dtype:
        raise TypeError(f"K_pages and V_pages must share a dtype, got {dtype}, {V_pages.dtype}")
    qc = q.to(dtype).contiguous()
    Kp, Vp = K_pages.contiguous(), V_pages.contiguous()
    bt, lnd = _i32(block_table, dev), _i32(ln, dev)
    out = torch.empty((B, W, Hq, D), dtype=dtype, device=dev)
    ws, ws_bytes = _lib.attention_workspace(dev, B, W * Hq, Hkv, D, MAX_BLOCKS, P)
    _lib.launch("mk_paged_verify_attention", dev, _lib.ptr(qc), _lib.ptr(Kp), _lib.ptr(Vp), _lib.ptr(bt),
                _lib.ptr(lnd), _lib.ptr(out), B, W, Hq, Hkv, D, P, MAX_BLOCKS, NUM_PAGES, float(scale),
                _lib.dtype_code(dtype), _lib.ptr(ws), ws_bytes)
    return out


def paged_verify_attention(q, K_pages, V_pages, block_table, lengths=None, scale=None, *, backend: str = "auto"):
    """W causal query rows per sequence over an fp16/bf16 paged cache in one
    HIP launch.  q [B,W,Hq,D]; K/V_pages [NUM_PAGES,P,Hkv,D]; lengths [B]
    count the context and all W new positions (already written); row w sees
    positions < lengths[b] - (W-1-w), none -> zeros.  Each K/V byte is read
    once for the W rows (mk_paged_verify_attention).  backend 'reference'
    runs reference_paged_verify_attention."""
    max_s = block_table.shape[1] * K_pages.shape[1]
    B, W, ln = _verify_shapes(q, block_table, lengths, max_s)
    if backend.lower() == "reference":
        return reference_paged_verify_attention(q, K_pages, V_pages, block_table, lengths, scale)
    if backend.lower() not in ("auto", "metal"):
        raise ValueError("backend must be one of 'reference', 'metal', 'auto'")
    if K_pages.dtype not in _ACT:
        raise TypeError(f"K_pages dtype must be float16 or bfloat16, got {K_pages.dtype}")
    if q.shape[3] != K_pages.shape[3] or q.shape[2] % K_pages.shape[2]:
        raise ValueError(f"q {tuple(q.shape)} does not fit pages {tuple(K_pages.shape)}")
    sc = 1.0 / math.sqrt(q.shape[3]) if scale is None else scale
    return _hip_verify_attention(q, K_pages, V_pages, block_table, ln, sc).to(q.dtype)


def paged_quantized_verify_attention(q, paged_qkv: PagedQuantizedKVCache, lengths=None, scale=None, *,
                                     backend: str = "auto"):
    """paged_verify_attention over a q8/q4 paged cache
    (ops/paged_quantized_kv_ops.py layout); lengths default to the cache's."""
    max_s = paged_qkv.block_table.shape[1] * int(paged_qkv.page_size)
    src = paged_qkv.lengths if lengths is None else lengths
    B, W, ln = _verify_shapes(q, paged_qkv.block_table, src, max_s)
    sc = 1.0 / math.sqrt(q.shape[3]) if scale is None else scale
    if backend.lower() == "reference":
        Kp, Vp = dequantize_kv_pages(paged_qkv)
        return reference_paged_verify_attention(q, Kp.to(q.dtype), Vp.to(q.dtype), paged_qkv.block_table, ln, sc)
    if backend.lower() not in ("auto", "metal"):
        raise ValueError("backend must be one of 'reference', 'metal', 'auto'")
    Bq, Wq, Hq, D = q.shape
    _, _, Hkv, _ = paged_qkv.original_page_shape
    P = int(paged_qkv.page_size)
    NUM_PAGES = _check_kernel_layout(paged_qkv, Hkv, D)
    kq, vq = paged_qkv.k_pages_q.contiguous(), paged_qkv.v_pages_q.contiguous()
    ks = paged_qkv.k_scales.to(torch.float16).contiguous()
    vs = paged_qkv.v_scales.to(torch.float16).contiguous()
    dev = _lib.require_device(q, kq, vq, ks, vs)
    qc = q.contiguous()
    bt, lnd = _i32(paged_qkv.block_table, dev), _i32(ln, dev)
    MAX_BLOCKS = bt.shape[1]
    out = torch.empty((Bq, Wq, Hq, D), dtype=q.dtype, device=dev)
    ws, ws_bytes = _lib.attention_workspace(dev, Bq, Wq * Hq, Hkv, D, MAX_BLOCKS, P)
    _lib.launch("mk_paged_quantized_verify_attention", dev, _lib.ptr(qc), _lib.ptr(kq), _lib.ptr(vq),
                _lib.ptr(ks), _lib.ptr(vs), _lib.ptr(bt), _lib.ptr(lnd), _lib.ptr(out), Bq, Wq, Hq, Hkv, D, P,
                MAX_BLOCKS, NUM_PAGES, paged_qkv.group_size, paged_qkv.bits, float(sc), _lib.dtype_code(q.dtype),
                _lib.ptr(ws), ws_bytes)
    return out


# ------------------------------------------------------------ one verify pass


def _rows_cache(stack_cache: LlamaStackCache, B: int, W: int) -> LlamaStackCache:
    """The stack cache as seen by B*W verify rows: the same K/V pages (a
    contiguous cache through its identity-paged view), each sequence's
    block-table row repeated W times (for the rows' cache writes; the
    attention takes every W-th row back).  Layers that share a block table
    share its repetition."""
    layers = []
    repeated: dict = {}
    for lc in stack_cache.layer_caches:
        if stack_cache.cache_layout == "paged":
            K, V, bt = lc
        else:
            Kc, Vc = lc
            S = Kc.shape[1]
            P = _contig.page_size_for(S)
            K, V = _contig.as_pages(Kc, P), _contig.as_pages(Vc, P)
            bt = _contig.identity_table(Kc.shape[0], S, P, Kc.device)
        if bt.shape[0] != B:
            raise ValueError(f"the cache holds {bt.shape[0]} sequences, x has {B}")
        key = (bt.data_ptr(), tuple(bt.shape))
        if key not in repeated:
            repeated[key] = bt.repeat_interleave(W, dim=0)
        layers.append((K, V, repeated[key]))
    P = layers[0][0].shape[1] if layers else stack_cache.page_size
    return LlamaStackCache(layers, "paged", stack_cache.max_seq_len, P)


def llama_stack_verify_step(x, stack_weights: LlamaStackWeights, stack_cache: LlamaStackCache, cos, sin, position,
                            config: LlamaLikeConfig, *, float_logits: bool = True):
    """W draft rows per sequence through the whole stack in one pass: x
    [B, W, hidden], ``position`` [B] (int or tensor) the first draft's
    position.  Each layer writes the W rows' K/V at position + w (into the
    cache's own pages, in place) and attends with row w seeing up to its own
    position.  Returns (logits [B, W, vocab] or None without a head,
    final_hidden [B, W, hidden], stack_cache) -- what W staged
    llama_stack_decode_step calls give, row by row."""
    config = config.validate()
    if x.ndim != 3 or x.shape[2] != config.hidden_size:
        raise ValueError(f"x must have shape [B,W,{config.hidden_size}], got {tuple(x.shape)}")
    B, W, H = x.shape
    dev = _lib.require_device(x)
    p0 = normalize_positions(position, B, stack_cache.max_seq_len - W + 1, device=dev).to(torch.int32)
    pos_rows = (p0[:, None] + torch.arange(W, dtype=torch.int32, device=dev)[None, :]).reshape(B * W)
    res = llama_stack_decode_step(x.reshape(B * W, 1, H), stack_weights, _rows_cache(stack_cache, B, W), cos, sin,
                                  pos_rows, config, float_logits=float_logits, verify_width=W)
    if stack_weights.lm_head is None:
        fh, _ = res
        return None, fh.reshape(B, W, H), stack_cache
    logits, fh, _ = res
    return logits.reshape(B, W, -1), fh.reshape(B, W, H), stack_cache


def _clone_cache(stack_cache: LlamaStackCache) -> LlamaStackCache:
    return LlamaStackCache([tuple(t.clone() for t in lc) for lc in stack_cache.layer_caches],
                           stack_cache.cache_layout, stack_cache.max_seq_len, stack_cache.page_size)


def parallel_verify_tokens(*, context_token_ids: list[int], proposed_token_ids: list[int], pipeline=None,
                           model_config=None, stack_weights=None, stack_cache=None, embedding=None, lm_head=None,
                           cos=None, sin=None, position=None, verification_config=None
                           ) -> ParallelVerificationPassResult:
    """ops/speculative_verify_ops.py:161-296 for one sequence: the K drafts
    go through llama_stack_verify_step on a staged copy of the cache; the
    greedy targets, accept mask, accepted prefix and replacement token follow
    the reference's rules.  ``pipeline`` (an object with llama_config,
    stack_weights, model.embedding / model.lm_head and an optional _state)
    is accepted as in the reference."""
    if pipeline is not None:
        model_config = pipeline.llama_config
        stack_weights = pipeline.stack_weights
        embedding = pipeline.model.embedding
        lm_head = pipeline.model.lm_head
        if getattr(pipeline, "_state", None) is not None:
            stack_cache = pipeline._state.cache
            if position is None:
                position = pipeline._state.position
    cfg = (verification_config or ParallelVerificationConfig()).validate()
    if not proposed_token_ids:
        return ParallelVerificationPassResult([], [], [], 0, metadata={"verification_path": "no_proposed_tokens"})
    K = len(proposed_token_ids)
    if stack_cache is None:
        raise ValueError("stack_cache is required for parallel_verify_tokens")
    if position is None:
        raise ValueError("position is required for parallel_verify_tokens")
    if embedding is None:
        embedding = stack_weights.embedding
    if lm_head is not None and stack_weights.lm_head is None:
        stack_weights = LlamaStackWeights(stack_weights.layers, stack_weights.final_norm_weight, lm_head,
                                          stack_weights.embedding)
    if stack_weights.lm_head is None:
        raise ValueError("parallel_verify_tokens needs an lm_head (in stack_weights or as lm_head)")
    staged = _clone_cache(stack_cache)
    x = embed_proposed_tokens(proposed_token_ids, embedding, B=1)
    p = int(position)
    logits, _, staged = llama_stack_verify_step(x, stack_weights, staged, cos, sin, p, model_config)
    logits_list = [logits[0, i] for i in range(K)]
    targets = greedy_sample(logits[0]).cpu().tolist()  # first maximum per row, as np.argmax
    mask = compute_accept_mask(list(proposed_token_ids), targets, require_exact_match=True)
    acc = accepted_prefix_length(mask)
    rej = K - acc
    repl = int(targets[acc]) if rej > 0 and acc < len(targets) else None
    return ParallelVerificationPassResult(
        proposed_token_ids=list(proposed_token_ids), target_token_ids=[int(t) for t in targets], accept_mask=mask,
        accepted_count=acc, replacement_token_id=repl, logits=logits_list if cfg.return_logits else None,
        staged_cache=staged,
        metadata={"verification_path": "multi_row_pass", "draft_length": K, "accepted_count": acc,
                  "rejected_count": rej, "use_prefill_for_draft": cfg.use_prefill_for_draft,
                  "start_position": position})


def commit_parallel_verification_cache(committed_cache: LlamaStackCache, staged_cache: LlamaStackCache, *,
                                       start_position: int, accepted_count: int, include_replacement: bool = False,
                                       replacement_position: int | None = None) -> LlamaStackCache:
    """Copy the staged K/V of the accepted drafts -- positions start_position
    .. start_position + accepted_count - 1, through replacement_position when
    include_replacement -- into the committed cache, in place, for sequence 0
    (ops/speculative_verify_ops.py:299-322 names the same arguments; the
    positions copied here are the drafts' own, see the module notes)."""
    if committed_cache.cache_layout != staged_cache.cache_layout:
        raise ValueError("committed and staged cache layouts must match")
    if len(committed_cache.layer_caches) != len(staged_cache.layer_caches):
        raise ValueError("committed and staged caches must have the same layer count")
    end = start_position + accepted_count
    if include_replacement and replacement_position is not None:
        end = replacement_position + 1
    if end <= start_position:
        return committed_cache
    for lc, ls_ in zip(committed_cache.layer_caches, staged_cache.layer_caches):
        if committed_cache.cache_layout == "contiguous":
            for dst, src in zip(lc[:2], ls_[:2]):
                dst[:, start_position:end] = src[:, start_position:end]
        else:
            K, V, bt = lc
            P = K.shape[1]
            pos = torch.arange(start_position, end, device=bt.device)
            pages = bt[0, pos // P].long()
            slots = pos % P
            K[pages, slots] = ls_[0][pages, slots]
            V[pages, slots] = ls_[1][pages, slots]
    return committed_cache
