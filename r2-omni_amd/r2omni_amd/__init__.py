"""MI355X (gfx950) SSPA packed-KV decode path: a drop-in for R²-Omni's r2omni.sspa cache and
split-K attention call surface, backed by the hand-written HIP kernels of libr2o_sspa.so.

Import names mirror the reference modules the Qwen/MiniCPM SSPA manager imports
(r2omni/sspa/integration/qwen_sspa_attention.py:16-25, 50-59).
"""
from .batch import BatchedDecoder, DecodeStepGraph
from .cache import (
    BF16KeyArena,
    CacheVariant,
    CompactInt2KeyArena,
    CompactInt2ValueArena,
    CompactInt4KeyArena,
    CompactInt4ValueArena,
    CompactMetadataArena,
    DynamicCacheStats,
    PackedTensor,
    PhysicalPageIndex,
    PrecisionPool,
    ThreePrecisionCache,
    append_generated_token,
    build_compact_int2_key_arena,
    build_compact_int2_value_arena,
    build_compact_int4_key_arena,
    build_compact_int4_value_arena,
    build_three_precision_cache,
    flush_full_recent_pool,
    fused_gather_pack_int4_value,
    precision_cache_active_storage_breakdown,
    precision_cache_storage_breakdown,
)
from .policy import (
    LayerCompressionPlan,
    PageAssignment,
    PageClass,
    PageTable,
    build_layer_compression_plan,
    build_page_table,
    plan_from_pages,
    project_token_bits_to_pages,
)
from .reference import normalized_fwht, triton_mixed_reference
from .rope import FusedQwen3Rotary, FusedRotary, qwen3_qk_norm_rope, qwen_qk_mrope
from .splitk import (
    SplitKExecutor,
    SplitKWorkspace,
    allocate_splitk_workspace,
    allocated_workspace_bytes,
    append_recent_fp_triton,
    prepare_splitk_executor,
    required_splitk_blocks,
    stack_homogeneous_splitk_executors,
    triton_fwht_128,
)

__all__ = [name for name in dir() if not name.startswith("_")]
