"""MI355X (gfx950) paged-KV decode path for InferKernelLab.

Hand-written HIP kernels (KV append, fused RoPE + append, paged decode
attention with split partitions, paged prefill attention) behind the C ABI
of include/ikl_paged.h, with the reference's operator surface (ops), paged
cache (cache), scheduler and runtime hooks, and the decode runners that
call them (decode: synthetic decoder; llama: Llama over the paged cache).
"""

from .cache import BlockAllocator, CacheLayout, PagedKVCache
from .ops import (
    append_kv_hip,
    append_kv_triton,
    hip_append_available,
    hip_available,
    paged_decode_attention_hip,
    paged_decode_attention_hip_grouped,
    paged_decode_attention_triton,
    paged_decode_attention_triton_grouped,
    paged_decode_autotune_config,
    paged_decode_grouped_autotune_config,
    paged_decode_grouped_dot_autotune_config,
    paged_decode_grouped_path,
    paged_decode_step_hip,
    paged_prefill_attention_hip,
    paged_prefill_path,
    PreparedAppend,
    PreparedDecodeStep,
    PreparedPagedAttention,
    PreparedPagedPrefill,
    rope_append_kv_hip,
    triton_append_available,
    triton_available,
)
from .runtime import InferenceRuntime, RuntimeStats
from .scheduler import InferenceRequest, ScheduleBatch, TokenBudgetScheduler

__all__ = [
    "BlockAllocator",
    "CacheLayout",
    "PagedKVCache",
    "InferenceRequest",
    "ScheduleBatch",
    "TokenBudgetScheduler",
    "InferenceRuntime",
    "RuntimeStats",
    "append_kv_hip",
    "append_kv_triton",
    "hip_available",
    "hip_append_available",
    "paged_decode_attention_hip",
    "paged_decode_attention_hip_grouped",
    "paged_decode_attention_triton",
    "paged_decode_attention_triton_grouped",
    "paged_decode_grouped_path",
    "paged_decode_step_hip",
    "PreparedAppend",
    "PreparedDecodeStep",
    "PreparedPagedAttention",
    "paged_prefill_attention_hip",
    "paged_prefill_path",
    "PreparedPagedPrefill",
    "rope_append_kv_hip",
    "paged_decode_autotune_config",
    "paged_decode_grouped_autotune_config",
    "paged_decode_grouped_dot_autotune_config",
    "triton_available",
    "triton_append_available",
]
