"""Quantized Llama-like decode stack on paged KV caches -- what
``ops/llama_stack_ops.py`` runs for ``cache_layout="paged"`` (the reference
raises NotImplementedError there, ops/llama_stack_ops.py:129-130, 205-206),
built from the paged layer of ``mk.llama_layer_ops``.

A decode step (ops/llama_stack_ops.py:352-411): every layer in turn, the
final RMSNorm, then logits = final_hidden . lm_head^T (a q4/q8 matvec when
the head is quantized, a dense fp32-accumulated product otherwise) and greedy
sampling (models/sampling.py:120-124).  ``DecodeGraph`` captures one whole
step -- embedding gather, 32 layers, head, argmax -- in a HIP graph so a
token costs one graph launch; positions live in a device tensor the step
advances in place.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any

import torch

from . import _lib
from .llama_layer_ops import (
    LlamaLayerKernelWeights,
    LlamaLikeConfig,
    llama_layer_decode_step,
    reference_llama_layer_decode_step,
)
from .norm_ops import reference_rms_norm, rms_norm
from .quant_ops import q4_matvec_decode, q8_matvec_decode, q_rmsnorm_matvec
from .quantize_weights import QuantizationConfig, quantize_weight_groupwise


@dataclass
class QuantizedHead:
    """A q4/q8 [vocab, hidden] output projection (codes, scales, zeros)."""

    w: Any
    scales: Any
    zeros: Any | None
    bits: int = 4
    group_size: int = 32

    @property
    def shape(self):
        return (self.scales.shape[0], self.w.shape[1] * (2 if self.bits == 4 else 1))


@dataclass
class LlamaStackWeights:
    """ops/llama_stack_ops.py:134-169."""

    layers: list
    final_norm_weight: Any
    lm_head: Any | None = None
    embedding: Any | None = None

    def num_layers(self) -> int:
        return len(self.layers)

    def validate(self, config: LlamaLikeConfig) -> "LlamaStackWeights":
        config = config.validate()
        if len(self.layers) != config.num_hidden_layers:
            raise ValueError(f"layers must have length {config.num_hidden_layers}, got {len(self.layers)}")
        if tuple(self.final_norm_weight.shape) != (config.hidden_size,):
            raise ValueError(f"final_norm_weight must have shape {(config.hidden_size,)}, "
                             f"got {tuple(self.final_norm_weight.shape)}")
        if self.embedding is not None and self.embedding.shape[1] != config.hidden_size:
            raise ValueError(f"embedding must have shape [vocab_size,{config.hidden_size}], "
                             f"got {tuple(self.embedding.shape)}")
        if self.lm_head is not None and self.lm_head.shape[1] != config.hidden_size:
            raise ValueError("lm_head must use the documented [vocab_size, hidden_size] convention with hidden size "
                             f"{config.hidden_size}, got {tuple(self.lm_head.shape)}")
        for layer in self.layers:
            layer.validate(config)
        return self


@dataclass
class LlamaStackCache:
    """ops/llama_stack_ops.py:171-192 (paged: one (K_pages, V_pages,
    block_table) per layer)."""

    layer_caches: list
    cache_layout: str
    max_seq_len: int
    page_size: int | None = None

    def num_layers(self) -> int:
        return len(self.layer_caches)


def init_llama_stack_cache(config: LlamaLikeConfig, B: int, max_seq_len: int, *, cache_layout: str = "contiguous",
                           dtype=torch.float16, page_size: int = 16, device=None, block_table=None):
    """ops/llama_stack_ops.py:195-221.  "contiguous": per layer zero
    (K_cache, V_cache) [B, max_seq_len, Hkv, D].  "paged" (which the
    reference leaves unimplemented): per layer K/V pages
    [B * ceil(max_seq_len / P), P, Hkv, D] (zeros) sharing one block table
    [B, ceil(max_seq_len / P)] (identity unless given)."""
    config = config.validate()
    if cache_layout == "contiguous":
        shape = (B, max_seq_len, config.num_key_value_heads, config.head_dim)
        caches = [(torch.zeros(shape, dtype=dtype, device=device), torch.zeros(shape, dtype=dtype, device=device))
                  for _ in range(config.num_hidden_layers)]
        return LlamaStackCache(caches, "contiguous", max_seq_len, None)
    if cache_layout != "paged":
        raise ValueError(f"cache_layout must be one of ('contiguous', 'paged'), got {cache_layout!r}")
    mb = math.ceil(max_seq_len / page_size)
    if block_table is None:
        block_table = torch.arange(B * mb, dtype=torch.int32, device=device).reshape(B, mb)
    npg = int(block_table.max().item()) + 1 if block_table.numel() else 0
    shape = (max(npg, B * mb), page_size, config.num_key_value_heads, config.head_dim)
    caches = [(torch.zeros(shape, dtype=dtype, device=device), torch.zeros(shape, dtype=dtype, device=device),
               block_table) for _ in range(config.num_hidden_layers)]
    return LlamaStackCache(caches, "paged", max_seq_len, page_size)


def embed_token_ids(token_ids, embedding):
    """ops/llama_stack_ops.py:224-232: token ids [B] or [B,1] -> [B,1,hidden]."""
    ids = token_ids.reshape(-1, 1) if token_ids.ndim == 1 else token_ids
    if ids.ndim != 2:
        raise ValueError(f"token_ids must have shape [B] or [B,1], got {tuple(token_ids.shape)}")
    out = embedding.index_select(0, ids.reshape(-1).to(torch.int64))
    return out.reshape(ids.shape[0], ids.shape[1], -1)


def logits_from_hidden(hidden, lm_head):
    """ops/llama_stack_ops.py:235-240: hidden [B,T,H] . lm_head^T -> fp32
    logits [B,T,vocab].  A ``QuantizedHead`` runs the q4/q8 matvec (outputs
    in the activation dtype, then widened); a dense head accumulates in fp32."""
    if hidden.ndim != 3:
        raise ValueError(f"hidden must have shape [B,1,H] or [B,T,H], got {tuple(hidden.shape)}")
    B, T, H = hidden.shape
    if isinstance(lm_head, QuantizedHead):
        fn = q4_matvec_decode if lm_head.bits == 4 else q8_matvec_decode
        y = fn(hidden.reshape(B * T, H), lm_head.w, lm_head.scales, lm_head.zeros, group_size=lm_head.group_size)
        return y.float().reshape(B, T, -1)
    return (hidden.reshape(B * T, H).float() @ lm_head.float().t()).reshape(B, T, -1)


def greedy_sample(logits):
    """models/sampling.py:120-124: argmax over the vocabulary -> int64 [B],
    with np.argmax's rule (the first index on ties, a NaN wins).  Device
    logits (fp16/bf16/fp32) go to the HIP row argmax, host ones to torch."""
    rows = logits.reshape(logits.shape[0], -1)
    if not rows.is_cuda:
        return torch.argmax(rows, dim=-1)
    rows = rows.contiguous()
    dev = _lib.require_device(rows)
    out = torch.empty(rows.shape[0], dtype=torch.int64, device=rows.device)
    _lib.launch("mk_argmax_rows", dev, _lib.ptr(rows), _lib.ptr(out), rows.shape[0], rows.shape[1],
                _lib.dtype_code(rows.dtype))
    return out


def llama_stack_decode_step(x, stack_weights: LlamaStackWeights, stack_cache: LlamaStackCache, cos, sin, position,
                            config: LlamaLikeConfig, *, return_intermediates: bool = False, reference: bool = False,
                            float_logits: bool = True, verify_width: int = 1):
    """ops/llama_stack_ops.py:352-411 on paged caches.  Returns (logits,
    final_hidden, cache) when the weights carry an lm_head, else
    (final_hidden, cache); with return_intermediates the per-layer hidden
    states are appended as a dict.  Logits are fp32; ``float_logits=False``
    keeps a quantized head's logits in the activation dtype (the widening is
    exact, so an argmax over either agrees).  ``verify_width`` W > 1
    (extension): the rows are W draft rows per sequence (row b * W + w at
    position[b * W + w], consecutive positions, block tables repeated W
    times), whose attention runs as one verify launch per layer."""
    config = config.validate()
    hidden = x
    layers_out = []
    new_caches = []
    # every layer attends over positions 0..position: the lengths are shared
    lengths = position.to(torch.int32) + 1 if isinstance(position, torch.Tensor) and position.is_cuda else None
    if verify_width > 1:
        if lengths is None:
            raise ValueError("verify_width needs per-row positions as a device tensor")
        lengths = lengths[verify_width - 1::verify_width].contiguous()  # per sequence: the last row's + 1
    for li, lw in enumerate(stack_weights.layers):
        if reference:
            hidden, cache = reference_llama_layer_decode_step(hidden, lw, stack_cache.layer_caches[li], cos, sin,
                                                              position, config, cache_layout=stack_cache.cache_layout)
        else:
            hidden, cache = llama_layer_decode_step(hidden, lw, stack_cache.layer_caches[li], cos, sin, position,
                                                    config, cache_layout=stack_cache.cache_layout, lengths=lengths,
                                                    verify_width=verify_width)
        new_caches.append(cache)
        if return_intermediates:
            layers_out.append(hidden)
    cache = LlamaStackCache(new_caches, stack_cache.cache_layout, stack_cache.max_seq_len, stack_cache.page_size)
    head = stack_weights.lm_head
    logits = None
    if isinstance(head, QuantizedHead) and not reference:
        # final RMSNorm inside the head's matvec
        B, T, H = hidden.shape
        y, final_hidden = q_rmsnorm_matvec(hidden.reshape(B * T, H), stack_weights.final_norm_weight, head.w,
                                           head.scales, head.zeros, bits=head.bits, group_size=head.group_size,
                                           eps=config.rms_norm_eps, return_normed=True)
        final_hidden = final_hidden.reshape(B, T, H)
        logits = (y.float() if float_logits else y).reshape(B, T, -1)
    else:
        norm = reference_rms_norm if reference else rms_norm
        final_hidden = norm(hidden, stack_weights.final_norm_weight, eps=config.rms_norm_eps)
    inter = {"layers": layers_out, "final_hidden": final_hidden}
    if head is None:
        return (final_hidden, cache, inter) if return_intermediates else (final_hidden, cache)
    if logits is None:
        logits = logits_from_hidden(final_hidden, head)
    if return_intermediates:
        inter["logits"] = logits
        return logits, final_hidden, cache, inter
    return logits, final_hidden, cache


def llama_stack_decode_loop(inputs, stack_weights: LlamaStackWeights, stack_cache: LlamaStackCache, cos, sin,
                            config: LlamaLikeConfig, *, backend_preset: str = "fused_experimental",
                            cache_layout: str = "contiguous", T: int | None = None, return_logits: bool = True):
    """ops/llama_stack_ops.py:439-495: decode inputs [B, T, hidden] (or
    [B, T, 1, hidden]) one step at a time, step t at position t of every
    sequence.  Returns (logits [B, T, vocab] -- or the final hidden states
    when ``return_logits`` is False or there is no head -- and the final
    cache).  Preset "reference" runs the torch reference path."""
    if inputs.ndim == 4:
        if inputs.shape[2] != 1:
            raise ValueError(f"inputs with rank 4 must have shape [B,T,1,H], got {tuple(inputs.shape)}")
        inputs = inputs[:, :, 0, :]
    if inputs.ndim != 3:
        raise ValueError(f"inputs must have shape [B,T,H] or [B,T,1,H], got {tuple(inputs.shape)}")
    if backend_preset not in ("reference", "metal", "tiled", "fused_experimental"):
        raise ValueError("layer_backend_preset must be one of ('reference', 'metal', 'tiled', 'fused_experimental')")
    if cache_layout not in ("contiguous", "paged"):
        raise ValueError("cache_layout must be one of ('contiguous', 'paged')")
    if cache_layout != stack_cache.cache_layout:
        raise ValueError(f"cache_layout {cache_layout!r} does not match the stack cache's "
                         f"{stack_cache.cache_layout!r}")
    T = inputs.shape[1] if T is None else T
    outputs = []
    running = stack_cache
    for t in range(T):
        result = llama_stack_decode_step(inputs[:, t:t + 1, :], stack_weights, running, cos, sin, t, config,
                                         reference=backend_preset == "reference")
        if stack_weights.lm_head is None:
            out_t, running = result
        else:
            logits_t, final_hidden_t, running = result
            out_t = logits_t if return_logits else final_hidden_t
        outputs.append(out_t)
    out = torch.cat(outputs, dim=1) if len(outputs) > 1 else outputs[0]
    return out, running


def reference_llama_stack_decode_loop(inputs, stack_weights: LlamaStackWeights, stack_cache: LlamaStackCache, cos,
                                      sin, config: LlamaLikeConfig, *, cache_layout: str = "contiguous",
                                      T: int | None = None, return_logits: bool = True):
    """ops/llama_stack_ops.py:413-436."""
    return llama_stack_decode_loop(inputs, stack_weights, stack_cache, cos, sin, config, backend_preset="reference",
                                   cache_layout=cache_layout, T=T, return_logits=return_logits)


def _random_linear(out_dim, in_dim, bits, group_size, gen, device, dtype):
    w = torch.randn((out_dim, in_dim), generator=gen, device=device, dtype=torch.float32).mul_(0.02).to(dtype)
    qw = quantize_weight_groupwise(w, QuantizationConfig(bits=bits, group_size=group_size))
    zeros = torch.full(tuple(qw.scales.shape), 8.0 if bits == 4 else 128.0, dtype=qw.scales.dtype, device=device)
    return qw.packed_weight, qw.scales, zeros


def create_random_quantized_llama_stack_weights(config: LlamaLikeConfig, *, vocab_size=None, bits=4, group_size=32,
                                                dtype=torch.float16, seed=0, device=None, include_embedding=True,
                                                include_lm_head=True, quantized_lm_head=True):
    """ops/llama_stack_ops.py:498-555 on the device: every projection drawn
    N(0, 0.02) and quantized groupwise (symmetric, zero point 8 / 128),
    norm weights 1, embedding N(0, 1); the head quantized the same way, or
    dense N(0, 1) fp16 when ``quantized_lm_head`` is False."""
    config = config.validate()
    vocab = vocab_size or config.vocab_size or 128
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    H, I = config.hidden_size, config.intermediate_size
    layers = []
    for _ in range(config.num_hidden_layers):
        qkv = _random_linear(config.qkv_output_dim(), H, bits, group_size, gen, device, dtype)
        o = _random_linear(H, H, bits, group_size, gen, device, dtype)
        g = _random_linear(I, H, bits, group_size, gen, device, dtype)
        u = _random_linear(I, H, bits, group_size, gen, device, dtype)
        d = _random_linear(H, I, bits, group_size, gen, device, dtype)
        ones = torch.ones(H, dtype=dtype, device=device)
        layers.append(LlamaLayerKernelWeights(
            input_layernorm_weight=ones, post_attention_layernorm_weight=ones.clone(),
            qkv_w=qkv[0], qkv_scales=qkv[1], qkv_zeros=qkv[2], o_w=o[0], o_scales=o[1], o_zeros=o[2],
            gate_w=g[0], gate_scales=g[1], gate_zeros=g[2], up_w=u[0], up_scales=u[1], up_zeros=u[2],
            down_w=d[0], down_scales=d[1], down_zeros=d[2], bits=bits, group_size=group_size))
    final_norm = torch.ones(H, dtype=dtype, device=device)
    embedding = (torch.randn((vocab, H), generator=gen, device=device, dtype=torch.float32).to(dtype)
                 if include_embedding else None)
    lm_head = None
    if include_lm_head:
        if quantized_lm_head:
            w, s, z = _random_linear(vocab, H, bits, group_size, gen, device, dtype)
            lm_head = QuantizedHead(w, s, z, bits, group_size)
        else:
            lm_head = torch.randn((vocab, H), generator=gen, device=device, dtype=torch.float32).to(dtype)
    return LlamaStackWeights(layers=layers, final_norm_weight=final_norm, lm_head=lm_head,
                             embedding=embedding).validate(config)


class DecodeGraph:
    """One greedy decode step captured in a HIP graph: token ids [B] (int64,
    device) at per-sequence positions [B] (int32, device) -> next token ids,
    with every layer's cache written at those positions.  ``step()`` replays
    the graph and advances the positions by one in place.

    Construction already performs the first decode step, eagerly (it warms
    every buffer the capture reuses): the caches hold the given tokens at the
    given positions, ``first_tokens`` holds that step's output, ``tokens`` is
    the input of the first ``step()`` (equal to ``first_tokens``) and
    ``positions`` has advanced by one.  So the tokens of a greedy run are
    ``first_tokens`` followed by the output of each ``step()``."""

    def __init__(self, stack_weights: LlamaStackWeights, stack_cache: LlamaStackCache, cos, sin,
                 config: LlamaLikeConfig, token_ids, positions):
        if stack_weights.embedding is None or stack_weights.lm_head is None:
            raise ValueError("DecodeGraph needs an embedding and an lm_head")
        self.w, self.cache, self.cos, self.sin, self.config = stack_weights, stack_cache, cos, sin, config
        self.tokens = token_ids.clone()
        self.positions = positions.to(torch.int32).clone()
        self.stream = torch.cuda.Stream(device=self.tokens.device)
        self.stream.wait_stream(torch.cuda.current_stream(self.tokens.device))
        with torch.cuda.stream(self.stream):
            self.first_tokens = self._run().clone()  # the first step; warms every buffer outside the capture
        self.stream.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=self.stream):
            self.next_tokens = self._run()

    def _run(self):
        x = embed_token_ids(self.tokens, self.w.embedding)
        logits, _, _ = llama_stack_decode_step(x, self.w, self.cache, self.cos, self.sin, self.positions, self.config,
                                               float_logits=False)
        nxt = greedy_sample(logits)
        self.tokens.copy_(nxt)
        self.positions.add_(1)
        return nxt

    def step(self):
        """Replays one step on the current stream: returns the next tokens
        (the graph's output buffer, overwritten by the next step)."""
        self.graph.replay()
        return self.next_tokens
