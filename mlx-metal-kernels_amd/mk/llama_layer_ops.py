"""Quantized Llama-like decode layer on a paged KV cache -- the paged path of
``ops/llama_layer_ops.py`` over torch tensors.

One decode step of one layer (ops/llama_layer_ops.py:234-428):
    qkv = rms_norm(x, input_layernorm) . Wqkv^T                 mk_q{4,8}_rmsnorm_matvec
    h = x + o_proj(attn(rope(split(qkv))))                       paged_quantized_decode_block
                                                                 (the residual add in the o-proj
                                                                  matvec's epilogue)
    out = quantized_mlp_block(h, 0, post_attention_layernorm)    mk_q{4,8}_rmsnorm_gate_up + down
Every intermediate is rounded to the activation dtype at the reference's
points.  The reference raises for a paged multi-layer stack
(ops/llama_stack_ops.py:129-130); this module implements the layer the stack
composes.
"""

from __future__ import annotations

import math
from dataclasses import asdict, dataclass
from typing import Any

import torch

from . import _contig
from .mlp_block_ops import quantized_mlp_block, reference_quantized_mlp_block
from .norm_ops import reference_rms_norm, rms_norm
from .quantized_decode_block_ops import paged_quantized_decode_block, reference_paged_quantized_decode_block


@dataclass
class LlamaLikeConfig:
    """models/llama_config.py:11-104."""

    hidden_size: int
    intermediate_size: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    num_hidden_layers: int
    max_position_embeddings: int
    rope_theta: float = 10000.0
    rms_norm_eps: float = 1e-5
    vocab_size: int | None = None
    tie_word_embeddings: bool = False
    model_type: str = "llama_like"

    def validate(self) -> "LlamaLikeConfig":
        """models/llama_config.py:26-46."""
        if self.hidden_size != self.num_attention_heads * self.head_dim:
            raise ValueError(
                "hidden_size must equal num_attention_heads * head_dim, "
                f"got hidden_size={self.hidden_size}, num_attention_heads={self.num_attention_heads}, "
                f"head_dim={self.head_dim}")
        if self.num_attention_heads % self.num_key_value_heads != 0:
            raise ValueError("num_attention_heads must be divisible by num_key_value_heads, "
                             f"got {self.num_attention_heads}, {self.num_key_value_heads}")
        if self.intermediate_size <= self.hidden_size:
            raise ValueError(f"intermediate_size must be greater than hidden_size, got {self.intermediate_size}, "
                             f"{self.hidden_size}")
        if self.max_position_embeddings <= 0:
            raise ValueError("max_position_embeddings must be positive")
        if self.num_hidden_layers <= 0:
            raise ValueError("num_hidden_layers must be positive")
        return self

    def q_output_dim(self) -> int:
        return self.validate().num_attention_heads * self.head_dim

    def kv_output_dim(self) -> int:
        return self.validate().num_key_value_heads * self.head_dim

    def qkv_output_dim(self) -> int:
        return self.q_output_dim() + 2 * self.kv_output_dim()

    def to_dict(self) -> dict:
        """models/llama_config.py:98-100 (the dataclass fields)."""
        return asdict(self)

    @classmethod
    def from_dict(cls, data: dict) -> "LlamaLikeConfig":
        """models/llama_config.py:102-104."""
        return cls(**data).validate()


def llama3_8b_like() -> LlamaLikeConfig:
    """Llama-3-8B decode shape: 32 layers, hidden 4096,
    32 query / 8 key-value heads of 128, intermediate 14336, RoPE theta
    500000, vocabulary 128256."""
    return LlamaLikeConfig(hidden_size=4096, intermediate_size=14336, num_attention_heads=32, num_key_value_heads=8,
                           head_dim=128, num_hidden_layers=32, max_position_embeddings=8192, rope_theta=500000.0,
                           rms_norm_eps=1e-5, vocab_size=128256, model_type="llama3_8b_like").validate()


def tiny_gqa_debug_config() -> LlamaLikeConfig:
    """models/llama_config.py:141-152."""
    return LlamaLikeConfig(hidden_size=64, intermediate_size=128, num_attention_heads=4, num_key_value_heads=2,
                           head_dim=16, num_hidden_layers=2, max_position_embeddings=64, vocab_size=256,
                           model_type="llama_like_tiny_gqa_debug").validate()


def build_rope_tables(config: LlamaLikeConfig, seq_len: int | None = None, *, device=None):
    """models/llama_config.py:107-124: (cos, sin) fp32 [seq_len, head_dim / 2]."""
    config.validate()
    n = config.max_position_embeddings if seq_len is None else seq_len
    if n <= 0:
        raise ValueError(f"seq_len must be positive, got {n}")
    if config.head_dim % 2 != 0:
        raise ValueError(f"head_dim must be even for RoPE, got {config.head_dim}")
    pos = torch.arange(n, dtype=torch.float32, device=device)
    inv = 1.0 / (float(config.rope_theta) ** (torch.arange(0, config.head_dim, 2, dtype=torch.float32, device=device)
                                               / float(config.head_dim)))
    f = pos[:, None] * inv[None, :]
    return torch.cos(f), torch.sin(f)


@dataclass
class LlamaLayerKernelWeights:
    """ops/llama_layer_ops.py:88-145 (q4/q8 codes, scales, zeros per projection)."""

    input_layernorm_weight: Any
    post_attention_layernorm_weight: Any
    qkv_w: Any
    qkv_scales: Any | None = None
    qkv_zeros: Any | None = None
    o_w: Any | None = None
    o_scales: Any | None = None
    o_zeros: Any | None = None
    gate_w: Any | None = None
    gate_scales: Any | None = None
    gate_zeros: Any | None = None
    up_w: Any | None = None
    up_scales: Any | None = None
    up_zeros: Any | None = None
    down_w: Any | None = None
    down_scales: Any | None = None
    down_zeros: Any | None = None
    bits: int = 4
    group_size: int = 32

    def validate(self, config: LlamaLikeConfig) -> "LlamaLayerKernelWeights":
        """ops/llama_layer_ops.py:110-134."""
        if self.bits not in (4, 8):
            raise ValueError(f"bits must be 4 or 8, got {self.bits}")
        if self.group_size <= 0:
            raise ValueError(f"group_size must be positive, got {self.group_size}")
        H = config.hidden_size
        for name in ("input_layernorm_weight", "post_attention_layernorm_weight"):
            if tuple(getattr(getattr(self, name), "shape", ())) != (H,):
                raise ValueError(f"{name} must have shape {(H,)}, got {tuple(getattr(self, name).shape)}")

        def cols(k):
            return (k + 1) // 2 if self.bits == 4 else k

        expected = {"qkv_w": (config.qkv_output_dim(), cols(H)), "o_w": (H, cols(H)),
                    "gate_w": (config.intermediate_size, cols(H)), "up_w": (config.intermediate_size, cols(H)),
                    "down_w": (H, cols(config.intermediate_size))}
        for name, shp in expected.items():
            got = getattr(self, name)
            if got is None or tuple(got.shape) != shp:
                raise ValueError(f"{name} must have shape {shp}, got {None if got is None else tuple(got.shape)}")
        return self


_ZEROS: dict = {}


def _zero_residual(h):
    """A cached zero tensor shaped like h: the MLP block's residual (the
    layer feeds h as x and 0 as residual, ops/llama_layer_ops.py:360-395),
    allocated once rather than on every call (and every graph replay)."""
    key = (tuple(h.shape), h.dtype, h.device)
    z = _ZEROS.get(key)
    if z is None:
        z = torch.zeros(h.shape, dtype=h.dtype, device=h.device)
        _ZEROS[key] = z
    return z


def _check_decode(x, config: LlamaLikeConfig, cache, cache_layout: str):
    """(K_pages, V_pages, block_table, restore) for either cache layout.

    "paged": cache = (K_pages, V_pages, block_table).  "contiguous" (the
    reference's default, ops/llama_layer_ops.py:251-255): cache = (K_cache,
    V_cache) [B, MAX_S, Hkv, D], served as an identity-paged view of the same
    memory; ``restore`` turns the (possibly new) page tensors back into the
    caller's layout."""
    if x.ndim != 3 or x.shape[1] != 1 or x.shape[2] != config.hidden_size:
        raise ValueError(f"x must have shape [B,1,{config.hidden_size}], got {tuple(x.shape)}")
    if cache_layout == "paged":
        if not isinstance(cache, tuple) or len(cache) != 3:
            raise ValueError("paged cache must be a tuple (K_pages, V_pages, block_table)")
        return cache + ((lambda K, V, bt: (K, V, bt)),)
    if cache_layout != "contiguous":
        raise ValueError(f"cache_layout must be one of ('contiguous', 'paged'), got {cache_layout!r}")
    if not isinstance(cache, tuple) or len(cache) != 2:
        raise ValueError("contiguous cache must be a tuple (K_cache, V_cache)")
    K_cache, V_cache = cache
    want = (x.shape[0], K_cache.shape[1] if K_cache.ndim == 4 else -1, config.num_key_value_heads, config.head_dim)
    if K_cache.ndim != 4 or tuple(K_cache.shape) != want or K_cache.shape != V_cache.shape:
        raise ValueError(f"K_cache and V_cache must have shape [B,MAX_S,Hkv,D]={want}, got "
                         f"{tuple(K_cache.shape)}, {tuple(V_cache.shape)}")
    B, S = K_cache.shape[:2]
    P = _contig.page_size_for(S)
    bt = _contig.identity_table(B, S, P, K_cache.device)
    shape = tuple(K_cache.shape)
    return (_contig.as_pages(K_cache, P), _contig.as_pages(V_cache, P), bt,
            (lambda K, V, _bt: (K.reshape(shape), V.reshape(shape))))


def llama_layer_decode_step(x, weights: LlamaLayerKernelWeights, cache, cos, sin, position, config,
                            *, cache_layout: str = "contiguous", return_intermediates: bool = False, lengths=None,
                            verify_width: int = 1):
    """ops/llama_layer_ops.py:234-428, all stages on HIP.  x [B,1,hidden];
    cache (K_pages, V_pages, block_table) for cache_layout="paged" or
    (K_cache, V_cache) [B,MAX_S,Hkv,D] for "contiguous", updated in place;
    position int or per-sequence [B].  Returns (out, cache) or
    (out, cache, intermediates).  The input RMSNorm runs inside the qkv
    matvec and the residual add inside the o-proj matvec; ``lengths``
    (extension) = position + 1 as a device tensor shared by all layers;
    ``verify_width`` (extension): see paged_quantized_decode_block."""
    config = config.validate()
    weights.validate(config)
    K_pages, V_pages, block_table, restore = _check_decode(x, config, cache, cache_layout)
    # without intermediates the norm, qkv projection, RoPE and cache write are
    # one launch (the projection is then never materialised)
    blk = paged_quantized_decode_block(
        x, weights.qkv_w, weights.qkv_scales, weights.o_w, weights.o_scales, K_pages, V_pages, block_table, cos,
        sin, position, qkv_zeros=weights.qkv_zeros, out_zeros=weights.o_zeros, bits=weights.bits,
        group_size=weights.group_size, H=config.num_attention_heads, num_key_value_heads=config.num_key_value_heads,
        head_dim=config.head_dim, return_intermediates=return_intermediates, residual=x,
        norm_weight=weights.input_layernorm_weight, eps=config.rms_norm_eps, lengths=lengths,
        verify_width=verify_width)
    h, K_pages, V_pages = blk[:3]
    qkv, attn_out = (blk[3], blk[4]) if return_intermediates else (None, None)
    res = quantized_mlp_block(h, _zero_residual(h), weights.post_attention_layernorm_weight, weights.gate_w,
                              weights.gate_scales, weights.up_w, weights.up_scales, weights.down_w, weights.down_scales,
                              gate_zeros=weights.gate_zeros, up_zeros=weights.up_zeros, down_zeros=weights.down_zeros,
                              bits=weights.bits, group_size=weights.group_size, eps=config.rms_norm_eps,
                              backend_preset="fused_experimental", return_intermediates=return_intermediates)
    cache = restore(K_pages, V_pages, block_table)
    if not return_intermediates:
        return res, cache
    out, mi = res
    x_norm = rms_norm(x, weights.input_layernorm_weight, eps=config.rms_norm_eps)
    return out, cache, {"x_norm": x_norm, "qkv": qkv, "attn_out": attn_out, "h": h, "mlp_norm": mi["normed"],
                        "gate": mi["gate"], "up": mi["up"], "mlp": mi["mlp"], "down": mi["down"]}


def reference_llama_layer_decode_step(x, weights: LlamaLayerKernelWeights, cache, cos, sin, position, config,
                                      *, cache_layout: str = "contiguous", return_intermediates: bool = False):
    """ops/llama_layer_ops.py:214-231 (every stage on the torch reference
    path; the cache is updated functionally, the input cache untouched)."""
    config = config.validate()
    weights.validate(config)
    K_pages, V_pages, block_table, restore = _check_decode(x, config, cache, cache_layout)
    x_norm = reference_rms_norm(x, weights.input_layernorm_weight, eps=config.rms_norm_eps)
    attn_proj, K_pages, V_pages, qkv, attn_out = reference_paged_quantized_decode_block(
        x_norm, weights.qkv_w, weights.qkv_scales, weights.o_w, weights.o_scales, K_pages, V_pages, block_table, cos,
        sin, position, qkv_zeros=weights.qkv_zeros, out_zeros=weights.o_zeros, bits=weights.bits,
        group_size=weights.group_size, H=config.num_attention_heads, num_key_value_heads=config.num_key_value_heads,
        head_dim=config.head_dim, return_intermediates=True)
    h = (x.float() + attn_proj.float()).to(x.dtype)
    res = reference_quantized_mlp_block(h, torch.zeros_like(h), weights.post_attention_layernorm_weight, weights.gate_w,
                                        weights.gate_scales, weights.up_w, weights.up_scales, weights.down_w,
                                        weights.down_scales, gate_zeros=weights.gate_zeros, up_zeros=weights.up_zeros,
                                        down_zeros=weights.down_zeros, bits=weights.bits,
                                        group_size=weights.group_size, eps=config.rms_norm_eps,
                                        return_intermediates=return_intermediates)
    cache = restore(K_pages, V_pages, block_table)
    if not return_intermediates:
        return res, cache
    out, mi = res
    return out, cache, {"x_norm": x_norm, "qkv": qkv, "attn_out": attn_out, "h": h, "mlp_norm": mi["normed"],
                        "gate": mi["gate"], "up": mi["up"], "mlp": mi["mlp"], "down": mi["down"]}


_LOOP_PRESETS = ("reference", "metal", "tiled", "fused_experimental")


def llama_layer_decode_loop(inputs, weights: LlamaLayerKernelWeights, cache, cos, sin, config, *,
                            backend_preset: str = "fused_experimental", cache_layout: str = "contiguous",
                            T: int | None = None, return_final_cache: bool = True):
    """ops/llama_layer_ops.py:431-467: decode inputs [B, T, hidden] one step
    at a time, step t at position t of every sequence.  Preset "reference"
    runs every stage on the torch reference path (functional cache updates);
    the other presets run the HIP layer (caches updated in place).  Returns
    (out [B, T, hidden], final cache) or out alone."""
    if inputs.ndim != 3:
        raise ValueError(f"inputs must have shape [B,T,hidden_size], got {tuple(inputs.shape)}")
    if backend_preset not in _LOOP_PRESETS:
        raise ValueError(f"backend_preset must be one of {_LOOP_PRESETS}, got {backend_preset}")
    T = inputs.shape[1] if T is None else T
    step = reference_llama_layer_decode_step if backend_preset == "reference" else llama_layer_decode_step
    outputs = []
    running = cache
    for t in range(T):
        out_t, running = step(inputs[:, t:t + 1, :], weights, running, cos, sin, t, config, cache_layout=cache_layout)
        outputs.append(out_t)
    out = torch.cat(outputs, dim=1) if len(outputs) > 1 else outputs[0]
    return (out, running) if return_final_cache else out


def init_llama_layer_cache(config: LlamaLikeConfig, B: int, max_seq_len: int, *, cache_layout: str = "contiguous",
                           dtype=torch.float16, page_size: int = 16, device=None):
    """ops/llama_layer_ops.py:516-526: zero (K_cache, V_cache) [B, MAX_S, Hkv, D]
    or the paged (K_pages, V_pages, identity block table)."""
    from .paged_kv_ops import allocate_paged_kv_cache

    config = config.validate()
    if cache_layout == "contiguous":
        shape = (B, max_seq_len, config.num_key_value_heads, config.head_dim)
        return (torch.zeros(shape, dtype=dtype, device=device), torch.zeros(shape, dtype=dtype, device=device))
    if cache_layout == "paged":
        return allocate_paged_kv_cache(B, max_seq_len, config.num_key_value_heads, config.head_dim, page_size, dtype,
                                       device=device)
    raise ValueError(f"cache_layout must be 'contiguous' or 'paged', got {cache_layout}")


def kv_pages_for(config: LlamaLikeConfig, B: int, max_seq_len: int, page_size: int = 16):
    """Pages per layer cache for B sequences of max_seq_len positions."""
    return B * math.ceil(max_seq_len / page_size)
