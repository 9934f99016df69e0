"""MI355X-native gated-delta verify hot path of DFlash speculative decoding.

Drop-in for the verify step of Aryagm/dflash-mlx's Qwen3.5 target: the
gated-delta scan with a per-token state tape, the fused greedy accept and the
tape-gather cache rollback, all on hand-written gfx950 kernels
(libdflash_gfx950.so, C ABI in include/dflash_gdn.h), behind the reference's
DFlashGenerator / dflash_generate decode API.  Names follow the reference
package (dflash_mlx/__init__.py:3-22) where the hot path has them; the
hybrid target model itself is dflash_mlx.target.HybridTargetModel.
"""
from .adapters import (
    LoadedTargetModel,
    Qwen35TargetAdapter,
    adapter_for_model_type,
    make_rollback_record,
    rewind_kv_caches,
    rollback_linear_caches,
)
from .cache import ArraysCache, KVCache
from .gated_delta import (
    advance_gated_delta_states,
    chunked_prefill_workspace_bytes,
    conv_rollback,
    gated_delta_kernel,
    gated_delta_prefill,
    gated_delta_verify,
    gated_delta_verify_rollback,
    tape_select,
)
from .runtime import (
    DFlashRuntimeEvent,
    dflash_generate,
    dflash_generate_stream,
    greedy_accept,
    lm_head_argmax,
    lm_head_greedy_accept,
    longest_prefix_match,
    sample_tokens,
    tile_weight,
    verify_block_chunked,
    verify_block_parallel_greedy_argmax,
    verify_block_parallel_lazy_logits,
    verify_block_parallel_replay,
    verify_block_stream,
)
from .api import DFlashGenerator, DFlashResult, DFlashStreamEvent

__all__ = [
    "ArraysCache",
    "DFlashGenerator",
    "DFlashResult",
    "DFlashRuntimeEvent",
    "DFlashStreamEvent",
    "LoadedTargetModel",
    "dflash_generate",
    "dflash_generate_stream",
    "verify_block_chunked",
    "verify_block_parallel_greedy_argmax",
    "verify_block_parallel_lazy_logits",
    "verify_block_stream",
    "KVCache",
    "Qwen35TargetAdapter",
    "adapter_for_model_type",
    "advance_gated_delta_states",
    "chunked_prefill_workspace_bytes",
    "conv_rollback",
    "gated_delta_kernel",
    "gated_delta_prefill",
    "gated_delta_verify",
    "gated_delta_verify_rollback",
    "greedy_accept",
    "lm_head_argmax",
    "lm_head_greedy_accept",
    "longest_prefix_match",
    "make_rollback_record",
    "rewind_kv_caches",
    "rollback_linear_caches",
    "sample_tokens",
    "tape_select",
    "tile_weight",
    "verify_block_parallel_replay",
]
