"""mk -- MI355X (gfx950) quantized decode hot path, a drop-in for the
quant_ops / mlp_block_ops / paged_kv_ops / paged_quantized_kv_ops modules of
manishklach/mlx-metal-kernels over torch tensors.

Modules mirror the reference's ``ops/`` files one-to-one; the kernels live in
``libmk_hip.so`` (C ABI declared in include/mk_hip.h) and are loaded lazily
by ``mk._lib``.
"""

__all__ = [
    "activation_ops",
    "autotune_ops",
    "backend_registry",
    "decode_block_ops",
    "fused_ops",
    "gqa_ops",
    "kv_cache_ops",
    "llama_layer_ops",
    "llama_stack_ops",
    "mlp_block_ops",
    "norm_ops",
    "paged_kv_ops",
    "paged_quantized_kv_ops",
    "quantize_weights",
    "quant_ops",
    "quantized_decode_block_ops",
    "rope_ops",
]
