"""Allocated vs. active cache storage on the GPU, mirroring the reference's
tests/test_active_cache_storage.py:15-112 on the same hand-built four-page plan (one FP, one INT4,
one INT2 and one evicted page of 32 tokens).

``precision_cache_storage_breakdown`` counts allocated capacity (reserved append space included);
``precision_cache_active_storage_breakdown`` counts populated payload and the metadata addressing it
(precision_pool.py:296-397).  Appends and flushes write into storage reserved at build time: the
allocated total stays fixed while the active total grows.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _plan(recent_capacity=128):
    from r2omni_amd.policy import LayerCompressionPlan, PageClass
    page_size = 32
    classes = torch.tensor([PageClass.FP_PAGE, PageClass.INT4_PAGE, PageClass.INT2_PAGE, PageClass.EVICTED_PAGE],
                           dtype=torch.long)
    positions = torch.arange(page_size * len(classes), dtype=torch.long)
    return LayerCompressionPlan(
        layer_id=0, fp_pages=torch.tensor([0]), int4_pages=torch.tensor([1]), int2_pages=torch.tensor([2]),
        evicted_pages=torch.tensor([3]), protected_pages=torch.empty(0, dtype=torch.long),
        recent_fp_capacity=recent_capacity, logical_positions=positions, global_token_indices=positions.clone(),
        page_offsets=torch.arange(len(classes), dtype=torch.long) * page_size,
        page_lengths=torch.full((len(classes),), page_size, dtype=torch.long), page_classes=classes)


def _cache(*, matched_fp=False, cache_variant="v_fourq_k_int4_compact", dtype=torch.float16):
    import r2omni_amd as ro
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    torch.manual_seed(0)
    key = torch.randn(2, 128, 128, dtype=dtype, device="cuda")
    value = torch.randn_like(key)
    return ro.build_three_precision_cache(key, value, _plan(), matched_fp=matched_fp, cache_variant=cache_variant,
                                          compact_key_append_capacity=1024)


@pytest.mark.parametrize("variant", ["v_fourq_k_int4_compact", "v_fourq_k_int2_compact"])
def test_active_storage_excludes_reserved_decode_capacity(variant):
    from r2omni_amd.cache import precision_cache_active_storage_breakdown, precision_cache_storage_breakdown
    cache = _cache(cache_variant=variant)
    active = precision_cache_active_storage_breakdown(cache)
    allocated = precision_cache_storage_breakdown(cache)
    assert active["persistent_cache_bytes"] < allocated["persistent_cache_bytes"]
    assert active["kv_payload_bytes"] < allocated["kv_payload_bytes"]
    assert cache.compact_key is not None
    assert cache.compact_key.bit_width == (4 if variant.endswith("int4_compact") else 2)
    assert cache.compact_key.active_nbytes < cache.compact_key.nbytes
    # every page and token index of the cache lives in the one metadata arena
    assert allocated["metadata_allocation_count"] == 1
    assert allocated["metadata_bytes"] == cache.metadata_arena.storage.untyped_storage().nbytes()


@pytest.mark.parametrize("variant", ["v_fourq_k_int4_compact", "v_fourq_k_int2_compact"])
def test_active_storage_tracks_append_and_flush_without_reallocation(variant):
    import r2omni_amd as ro
    from r2omni_amd.cache import precision_cache_active_storage_breakdown, precision_cache_storage_breakdown
    cache = _cache(cache_variant=variant)
    initial_active = precision_cache_active_storage_breakdown(cache)
    initial_allocated = precision_cache_storage_breakdown(cache)
    arena_ptr = cache.metadata_arena.storage.data_ptr()
    stats = ro.DynamicCacheStats()
    token = torch.randn(2, 1, 128, dtype=torch.float16, device="cuda")
    for index in range(129):
        ro.append_generated_token(cache, token, token, global_token_index=128 + index,
                                  logical_position=128 + index, stats=stats)
    torch.cuda.synchronize()
    final_active = precision_cache_active_storage_breakdown(cache)
    final_allocated = precision_cache_storage_breakdown(cache)
    assert stats.flushed_tokens == 128
    assert stats.recent_reallocation_count == 0
    assert cache.recent_fp_pool.active_length == 1
    assert final_active["persistent_cache_bytes"] > initial_active["persistent_cache_bytes"]
    assert final_allocated == initial_allocated
    assert cache.metadata_arena.storage.data_ptr() == arena_ptr
    # the flushed chunk's indices landed in the INT2 pool's reserved fields, in order
    int2 = cache.int2_pool.page_index
    assert int2.global_token_indices.tolist() == list(range(64, 96)) + list(range(128, 256))
    assert int2.logical_positions.tolist() == list(range(64, 96)) + list(range(128, 256))
    assert int2.physical_offsets.tolist() == [0, 32, 64, 96, 128]
    assert int2.lengths.tolist() == [32] * 5
    assert int2.original_page_ids.tolist() == [2, -1, -1, -1, -1]
    # and the ring holds the last token at slot 0
    ring = cache.recent_fp_pool
    assert int(ring.length_device) == 1
    assert ring.global_index_buffer[:1].tolist() == [256]
    assert ring.page_index.lengths.tolist() == [1, 0, 0, 0]


def test_matched_fp_recent_pool_counts_only_active_tokens():
    from r2omni_amd.cache import precision_cache_active_storage_breakdown, precision_cache_storage_breakdown
    cache = _cache(matched_fp=True, dtype=torch.bfloat16)
    active = precision_cache_active_storage_breakdown(cache)
    allocated = precision_cache_storage_breakdown(cache)
    assert cache.recent_fp_pool.active_length == 0
    assert cache.recent_fp_pool.active_payload_bytes == 0
    assert active["persistent_cache_bytes"] < allocated["persistent_cache_bytes"]


def test_bf16_key_variant_counts_its_shared_key_rows_once():
    from r2omni_amd.cache import precision_cache_active_storage_breakdown, precision_cache_storage_breakdown
    cache = _cache(cache_variant="v_fourq_k_bf16", dtype=torch.bfloat16)
    active = precision_cache_active_storage_breakdown(cache)
    allocated = precision_cache_storage_breakdown(cache)
    assert active["persistent_cache_bytes"] < allocated["persistent_cache_bytes"]
    # the three history pools' K rows are views of one arena: one allocation, counted once
    rows = cache.bf16_key.rows
    ptrs = {p.fp_k.untyped_storage().data_ptr() for p in cache.pools[:3] if p.fp_k is not None}
    assert ptrs == {rows.untyped_storage().data_ptr()}
    assert cache.metadata_arena is not None
    assert cache.metadata_arena.int2_lengths_buffer.numel() == cache.int2_pool.page_index.lengths.numel()
