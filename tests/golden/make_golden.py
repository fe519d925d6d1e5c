"""Write the golden fixtures for the SSPA packed-KV cache from the reference's own CPU path.

This script is run by hand, in the build container only, where the reference checkout is
mounted read-only at ``/root/reference``.  It imports the reference's torch-only runtime
(r2omni/sspa/runtime/*, r2omni/sspa/policy/page_assignment.py, cache_plan.py and
kernels/triton_fourq_attention.py) and records inputs and outputs as ``.npz`` fixtures next
to this file.  Nothing else in this repository imports the reference; the fixtures are data.

What the fixtures pin (functions with no closed form; every other function is also checked
against closed forms and invariants in tests/test_oracle_*.py):

* ``_compact_page_layouts`` stable FP -> INT4 -> INT2 token order and therefore the INT4-K
  superblock membership (precision_pool.py:611-669, compact_int4_key.py:223-281);
* ``append_superblock`` dequantise-then-requantise of a partial K tail on a flush
  (compact_int4_key.py:210-220) and the INT2-V flush append (fused_value_pack.py:474-516);
* the Recent-FP ring state after ``append_generated_token`` (dynamic_fourq_cache.py:172-267);
* ``triton_mixed_reference`` attention outputs on those caches (triton_fourq_attention.py:72-125);
* the matched-FP and K-BF16 caches (precision_pool.py:834-980): survivor order, pool K rows,
  the matched flush append (dynamic_fourq_cache.py:145-170) and the K-BF16 flush refusal (:226-230);
* generated INT4 values (``generated_value_precision="int4"``, precision_pool.py:935-956): the
  INT4-V arena with its static and flushed values (fused_value_pack.py:197-330), the INT4 pool's
  metadata after a flush (dynamic_fourq_cache.py:212-219, 236-243) and the attention over the INT4
  pool's two K runs (triton_fourq_attention.py:95-111).

Usage:  python tests/golden/make_golden.py [fixture names from _VARIANTS]
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REFERENCE = "/root/reference"


def _np(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().clone().contiguous()  # never a view of a tensor mutated later
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def _modality(total: int, gen: torch.Generator) -> torch.Tensor:
    """Runs of random length so that pages are ragged at modality boundaries."""
    out = []
    kind = 1
    while len(out) < total:
        run = int(torch.randint(5, 70, (1,), generator=gen))
        out.extend([kind] * run)
        kind = 1 + (kind % 2)
    return torch.tensor(out[:total], dtype=torch.long)


def _case(name, *, seq, hkv, dtype, page_size, sb, group, tier_probs, appends, seed):
    sys.path.insert(0, REFERENCE)
    from r2omni.sspa.policy.page_assignment import build_page_table, project_token_bits_to_pages
    from r2omni.sspa.runtime.cache_plan import build_layer_compression_plan
    from r2omni.sspa.runtime.precision_pool import build_three_precision_cache
    from r2omni.sspa.runtime.dynamic_fourq_cache import DynamicCacheStats, append_generated_token
    from r2omni.sspa.kernels.triton_fourq_attention import triton_mixed_reference

    gen = torch.Generator().manual_seed(seed)
    d = 128
    key = torch.randn(hkv, seq, d, generator=gen).to(dtype)
    outlier = torch.randperm(d, generator=gen)[:4]
    key[:, :, outlier] = (key[:, :, outlier].float() * 8.0).to(dtype)
    value = torch.randn(hkv, seq, d, generator=gen).to(dtype)
    modality = _modality(seq, gen)
    table = build_page_table(
        modality,
        page_size=page_size,
        protected_mask=torch.zeros(seq, dtype=torch.bool),
        recent_mask=torch.zeros(seq, dtype=torch.bool),
    )
    # one precision per page, drawn from a seeded categorical over (16, 4, 2) bits
    probs = torch.tensor(tier_probs, dtype=torch.float)
    page_tier = torch.multinomial(probs, table.num_pages, replacement=True, generator=gen)
    bits_per_tier = torch.tensor([16, 4, 2], dtype=torch.int8)
    bits = torch.empty(seq, dtype=torch.int8)
    for page, (off, ln) in enumerate(zip(table.offsets.tolist(), table.lengths.tolist())):
        bits[off : off + ln] = bits_per_tier[page_tier[page]]
    assignment = project_token_bits_to_pages(table, bits)
    plan = build_layer_compression_plan(0, assignment, recent_fp_capacity=128)
    cache = build_three_precision_cache(
        key,
        value,
        plan,
        page_size=page_size,
        key_quantization_superblock=sb,
        int2_group_size=group,
        compact_key_append_capacity=260,
        recent_flush_size=128,
    )
    hq = hkv * 8
    query = torch.randn(1, hq, d, generator=gen)
    record = {
        "key": _np(key),
        "value": _np(value),
        "dtype": np.array(str(dtype)),
        "page_offsets": _np(plan.page_offsets),
        "page_lengths": _np(plan.page_lengths),
        "page_classes": _np(plan.page_classes.to(torch.int64)),
        "page_size": np.array(page_size),
        "superblock": np.array(sb),
        "group": np.array(group),
        "query": _np(query),
    }

    def snapshot(prefix: str) -> None:
        ck = cache.compact_key
        record[prefix + "k_packed"] = _np(ck.packed[:, : ck.active_length])
        blocks = (ck.active_length + ck.superblock_size - 1) // ck.superblock_size
        record[prefix + "k_scale"] = _np(ck.scale[:, :blocks])
        record[prefix + "k_zero"] = _np(ck.zero_point[:, :blocks])
        record[prefix + "k_active"] = np.array(ck.active_length)
        record[prefix + "k_capacity"] = np.array(ck.capacity)
        record[prefix + "k_segments"] = np.array(ck.segment_offsets)
        cv = cache.compact_value
        record[prefix + "v2_packed"] = _np(cv.packed[:, : cv.active_length])
        record[prefix + "v2_scale"] = _np(cv.scale[:, : cv.active_length])
        record[prefix + "v2_zero"] = _np(cv.zero_point[:, : cv.active_length])
        record[prefix + "v2_active"] = np.array(cv.active_length)
        record[prefix + "v2_capacity"] = np.array(cv.capacity)
        i4 = cache.int4_pool
        if i4.token_count:
            record[prefix + "v4_packed"] = _np(i4.packed_v.packed)
            record[prefix + "v4_scale"] = _np(i4.packed_v.scale)
        else:
            record[prefix + "v4_packed"] = np.zeros(0, np.uint8)
            record[prefix + "v4_scale"] = np.zeros((hkv, 0, 1), np.float32)
        fp = cache.fp_pool
        record[prefix + "fp_v"] = (
            _np(fp.fp_v) if fp.token_count else np.zeros((hkv, 0, d), np.uint16 if dtype == torch.bfloat16 else np.float16)
        )
        rec = cache.recent_fp_pool
        record[prefix + "recent_k"] = _np(rec.fp_k[:, : rec.active_length])
        record[prefix + "recent_v"] = _np(rec.fp_v[:, : rec.active_length])
        record[prefix + "recent_active"] = np.array(rec.active_length)
        record[prefix + "recent_global"] = _np(rec.global_index_buffer[: rec.active_length])
        record[prefix + "recent_page_lengths"] = _np(rec.page_index.lengths)
        record[prefix + "pool_tokens"] = np.array(
            [fp.token_count, i4.token_count, cache.int2_pool.token_count, rec.token_count]
        )
        record[prefix + "int2_global"] = _np(cache.int2_pool.page_index.global_token_indices[: cache.int2_pool.token_count])
        record[prefix + "attn"] = _np(triton_mixed_reference(query, cache).float())

    stats_box = []
    snapshot("build_")
    stats = DynamicCacheStats()
    stats_box.append(stats)
    app_k = torch.randn(appends, hkv, 1, d, generator=gen).to(dtype)
    app_v = torch.randn(appends, hkv, 1, d, generator=gen).to(dtype)
    record["append_k"] = _np(app_k)
    record["append_v"] = _np(app_v)
    flushed_at = []
    for step in range(appends):
        flushed = append_generated_token(
            cache,
            app_k[step],
            app_v[step],
            global_token_index=seq + step,
            logical_position=seq + step,
            stats=stats,
        )
        if flushed:
            flushed_at.append(step)
    record["flushed_at"] = np.array(flushed_at, dtype=np.int64)
    record["tail_dequant_tokens"] = np.array(stats.local_tail_dequant_tokens)
    snapshot("after_")
    path = os.path.join(HERE, f"{name}.npz")
    np.savez_compressed(path, **record)
    print(f"wrote {path}: flushes at {flushed_at}, tail tokens {stats.local_tail_dequant_tokens}")


def _variant_case(name, *, variant, seq, hkv, dtype, page_size, sb, group, tier_probs, appends, seed):
    """Other K formats: ``matched`` (matched_fp=True), ``bf16k`` (cache_variant v_fourq_k_bf16) or
    ``int2k`` (cache_variant v_fourq_k_int2_compact)."""
    sys.path.insert(0, REFERENCE)
    from r2omni.sspa.policy.page_assignment import build_page_table, project_token_bits_to_pages
    from r2omni.sspa.runtime.cache_plan import build_layer_compression_plan
    from r2omni.sspa.runtime.precision_pool import build_three_precision_cache
    from r2omni.sspa.runtime.dynamic_fourq_cache import DynamicCacheStats, append_generated_token
    from r2omni.sspa.kernels.triton_fourq_attention import triton_mixed_reference

    gen = torch.Generator().manual_seed(seed)
    d = 128
    key = torch.randn(hkv, seq, d, generator=gen).to(dtype)
    value = torch.randn(hkv, seq, d, generator=gen).to(dtype)
    modality = _modality(seq, gen)
    table = build_page_table(modality, page_size=page_size, protected_mask=torch.zeros(seq, dtype=torch.bool),
                             recent_mask=torch.zeros(seq, dtype=torch.bool))
    probs = torch.tensor(tier_probs, dtype=torch.float)
    page_tier = torch.multinomial(probs, table.num_pages, replacement=True, generator=gen)
    bits_per_tier = torch.tensor([16, 4, 2, 0], dtype=torch.int8)  # 0 bits = evicted page
    bits = torch.empty(seq, dtype=torch.int8)
    for page, (off, ln) in enumerate(zip(table.offsets.tolist(), table.lengths.tolist())):
        bits[off : off + ln] = bits_per_tier[page_tier[page]]
    assignment = project_token_bits_to_pages(table, bits)
    plan = build_layer_compression_plan(0, assignment, recent_fp_capacity=128)
    kwargs = dict(page_size=page_size, key_quantization_superblock=sb, int2_group_size=group,
                  compact_key_append_capacity=260, recent_flush_size=128)
    if variant == "matched":
        cache = build_three_precision_cache(key, value, plan, matched_fp=True, **kwargs)
    elif variant == "int2k":
        cache = build_three_precision_cache(key, value, plan, cache_variant="v_fourq_k_int2_compact", **kwargs)
    else:
        cache = build_three_precision_cache(key, value, plan, cache_variant="v_fourq_k_bf16", **kwargs)
    query = torch.randn(1, hkv * 8, d, generator=gen)
    record = {"key": _np(key), "value": _np(value), "dtype": np.array(str(dtype)),
              "page_offsets": _np(plan.page_offsets), "page_lengths": _np(plan.page_lengths),
              "page_classes": _np(plan.page_classes.to(torch.int64)), "page_size": np.array(page_size),
              "superblock": np.array(sb), "group": np.array(group), "query": _np(query),
              "variant": np.array(variant)}

    def snapshot(prefix):
        pools = [cache.fp_pool, cache.int4_pool, cache.int2_pool]
        if variant == "int2k":
            ck = cache.compact_key
            blocks = -(-ck.active_length // ck.superblock_size)
            record[prefix + "k_packed"] = _np(ck.packed[:, : ck.active_length])
            record[prefix + "k_scale"] = _np(ck.scale[:, :blocks])
            record[prefix + "k_offset"] = _np(ck.zero_point[:, :blocks])
            record[prefix + "k_capacity"] = np.array(ck.capacity)
            record[prefix + "tail_dequant_tokens"] = np.array(stats_box[0].local_tail_dequant_tokens
                                                              if stats_box else 0)
        else:
            record[prefix + "k_rows"] = _np(torch.cat([p.fp_k for p in pools if p.token_count], dim=1))
        record[prefix + "pool_tokens"] = np.array([p.token_count for p in pools] + [cache.recent_fp_pool.token_count])
        fp = cache.fp_pool
        record[prefix + "fp_v"] = _np(fp.fp_v) if fp.token_count else np.zeros((hkv, 0, d), np.uint16)
        record[prefix + "fp_global"] = _np(fp.page_index.global_token_indices[: fp.token_count])
        if variant in ("bf16k", "int2k"):
            i4 = cache.int4_pool
            record[prefix + "v4_packed"] = _np(i4.packed_v.packed) if i4.token_count else np.zeros(0, np.uint8)
            record[prefix + "v4_scale"] = (_np(i4.packed_v.scale) if i4.token_count
                                           else np.zeros((hkv, 0, 1), np.float32))
            cv = cache.compact_value
            record[prefix + "v2_packed"] = _np(cv.packed[:, : cv.active_length])
            record[prefix + "v2_scale"] = _np(cv.scale[:, : cv.active_length])
            record[prefix + "v2_zero"] = _np(cv.zero_point[:, : cv.active_length])
        rec = cache.recent_fp_pool
        record[prefix + "recent_k"] = _np(rec.fp_k[:, : rec.active_length])
        record[prefix + "recent_v"] = _np(rec.fp_v[:, : rec.active_length])
        record[prefix + "attn"] = _np(triton_mixed_reference(query, cache).float())

    stats_box = []
    snapshot("build_")
    stats = DynamicCacheStats()
    stats_box.append(stats)
    app_k = torch.randn(appends, hkv, 1, d, generator=gen).to(dtype)
    app_v = torch.randn(appends, hkv, 1, d, generator=gen).to(dtype)
    record["append_k"] = _np(app_k)
    record["append_v"] = _np(app_v)
    flushed_at, refused_at = [], -1
    for step in range(appends):
        try:
            if append_generated_token(cache, app_k[step], app_v[step], global_token_index=seq + step,
                                      logical_position=seq + step, stats=stats):
                flushed_at.append(step)
        except RuntimeError:
            refused_at = step
            break
    record["flushed_at"] = np.array(flushed_at, dtype=np.int64)
    record["refused_at"] = np.array(refused_at)
    snapshot("after_")
    path = os.path.join(HERE, f"{name}.npz")
    np.savez_compressed(path, **record)
    print(f"wrote {path}: flushes at {flushed_at}, refused at {refused_at}")


def _gen_int4_case(name, *, seq, hkv, dtype, page_size, sb, group, tier_probs, appends, seed):
    """``generated_value_precision="int4"`` (precision_pool.py:935-956): the INT4 pool's values are a
    ``CompactInt4ValueArena`` with append room (fused_value_pack.py:197-330), a flush packs the 128
    oldest ring values into it (dynamic_fourq_cache.py:212-219), and ``triton_mixed_reference``
    reassembles the INT4 pool's keys from two K arena runs (triton_fourq_attention.py:95-111)."""
    sys.path.insert(0, REFERENCE)
    from r2omni.sspa.policy.page_assignment import build_page_table, project_token_bits_to_pages
    from r2omni.sspa.runtime.cache_plan import build_layer_compression_plan
    from r2omni.sspa.runtime.precision_pool import build_three_precision_cache
    from r2omni.sspa.runtime.dynamic_fourq_cache import DynamicCacheStats, append_generated_token
    from r2omni.sspa.kernels.triton_fourq_attention import triton_mixed_reference

    gen = torch.Generator().manual_seed(seed)
    d = 128
    key = torch.randn(hkv, seq, d, generator=gen).to(dtype)
    outlier = torch.randperm(d, generator=gen)[:4]
    key[:, :, outlier] = (key[:, :, outlier].float() * 8.0).to(dtype)
    value = torch.randn(hkv, seq, d, generator=gen).to(dtype)
    modality = _modality(seq, gen)
    table = build_page_table(modality, page_size=page_size, protected_mask=torch.zeros(seq, dtype=torch.bool),
                             recent_mask=torch.zeros(seq, dtype=torch.bool))
    probs = torch.tensor(tier_probs, dtype=torch.float)
    page_tier = torch.multinomial(probs, table.num_pages, replacement=True, generator=gen)
    bits_per_tier = torch.tensor([16, 4, 2], dtype=torch.int8)
    bits = torch.empty(seq, dtype=torch.int8)
    for page, (off, ln) in enumerate(zip(table.offsets.tolist(), table.lengths.tolist())):
        bits[off : off + ln] = bits_per_tier[page_tier[page]]
    assignment = project_token_bits_to_pages(table, bits)
    plan = build_layer_compression_plan(0, assignment, recent_fp_capacity=128)
    cache = build_three_precision_cache(key, value, plan, page_size=page_size, key_quantization_superblock=sb,
                                        int2_group_size=group, compact_key_append_capacity=260,
                                        recent_flush_size=128, generated_value_precision="int4")
    query = torch.randn(1, hkv * 8, d, generator=gen)
    record = {"key": _np(key), "value": _np(value), "dtype": np.array(str(dtype)),
              "page_offsets": _np(plan.page_offsets), "page_lengths": _np(plan.page_lengths),
              "page_classes": _np(plan.page_classes.to(torch.int64)), "page_size": np.array(page_size),
              "superblock": np.array(sb), "group": np.array(group), "query": _np(query),
              "gen_values": np.array("int4")}

    def snapshot(prefix):
        ck = cache.compact_key
        blocks = -(-ck.active_length // ck.superblock_size)
        record[prefix + "k_packed"] = _np(ck.packed[:, : ck.active_length])
        record[prefix + "k_scale"] = _np(ck.scale[:, :blocks])
        record[prefix + "k_zero"] = _np(ck.zero_point[:, :blocks])
        record[prefix + "k_active"] = np.array(ck.active_length)
        record[prefix + "k_capacity"] = np.array(ck.capacity)
        record[prefix + "k_segments"] = np.array(ck.segment_offsets)
        record[prefix + "generated_k_offset"] = np.array(cache.generated_k_offset)
        record[prefix + "static_int4_tokens"] = np.array(cache.static_int4_tokens)
        v4 = cache.compact_int4_value
        record[prefix + "v4_packed"] = _np(v4.packed[:, : v4.active_length])
        record[prefix + "v4_scale"] = _np(v4.scale[:, : v4.active_length])
        record[prefix + "v4_active"] = np.array(v4.active_length)
        record[prefix + "v4_capacity"] = np.array(v4.capacity)
        cv = cache.compact_value
        record[prefix + "v2_packed"] = _np(cv.packed[:, : cv.active_length])
        record[prefix + "v2_scale"] = _np(cv.scale[:, : cv.active_length])
        record[prefix + "v2_zero"] = _np(cv.zero_point[:, : cv.active_length])
        record[prefix + "v2_active"] = np.array(cv.active_length)
        record[prefix + "v2_capacity"] = np.array(cv.capacity)
        fp = cache.fp_pool
        record[prefix + "fp_v"] = (_np(fp.fp_v) if fp.token_count
                                   else np.zeros((hkv, 0, d), np.uint16 if dtype == torch.bfloat16 else np.float16))
        rec = cache.recent_fp_pool
        record[prefix + "recent_k"] = _np(rec.fp_k[:, : rec.active_length])
        record[prefix + "recent_v"] = _np(rec.fp_v[:, : rec.active_length])
        record[prefix + "recent_active"] = np.array(rec.active_length)
        record[prefix + "recent_global"] = _np(rec.global_index_buffer[: rec.active_length])
        record[prefix + "pool_tokens"] = np.array([fp.token_count, cache.int4_pool.token_count,
                                                   cache.int2_pool.token_count, rec.token_count])
        i4, i2 = cache.int4_pool, cache.int2_pool
        record[prefix + "int4_global"] = _np(i4.page_index.global_token_indices[: i4.token_count])
        record[prefix + "int4_logical"] = _np(i4.page_index.logical_positions[: i4.token_count])
        record[prefix + "int2_global"] = _np(i2.page_index.global_token_indices[: i2.token_count])
        record[prefix + "attn"] = _np(triton_mixed_reference(query, cache).float())

    snapshot("build_")
    stats = DynamicCacheStats()
    app_k = torch.randn(appends, hkv, 1, d, generator=gen).to(dtype)
    app_v = torch.randn(appends, hkv, 1, d, generator=gen).to(dtype)
    record["append_k"] = _np(app_k)
    record["append_v"] = _np(app_v)
    flushed_at = []
    for step in range(appends):
        if append_generated_token(cache, app_k[step], app_v[step], global_token_index=seq + step,
                                  logical_position=seq + step, stats=stats):
            flushed_at.append(step)
    record["flushed_at"] = np.array(flushed_at, dtype=np.int64)
    record["tail_dequant_tokens"] = np.array(stats.local_tail_dequant_tokens)
    record["flushed_int4_value_tokens"] = np.array(stats.flushed_int4_value_tokens)
    snapshot("after_")
    path = os.path.join(HERE, f"{name}.npz")
    np.savez_compressed(path, **record)
    print(f"wrote {path}: flushes at {flushed_at}, tail tokens {stats.local_tail_dequant_tokens}, "
          f"INT4 value tokens flushed {stats.flushed_int4_value_tokens}")


def main() -> None:
    only = set(sys.argv[1:])
    if only:
        for name, fn in _VARIANTS.items():
            if name in only:
                fn()
        return
    # Qwen profile: 32-token pages (ragged at modality boundaries), K superblock 32, INT2 group 32.
    _case("qwen_ragged_bf16", seq=333, hkv=2, dtype=torch.bfloat16, page_size=32, sb=32,
          group=32, tier_probs=(0.2, 0.5, 0.3), appends=140, seed=11)
    # fp16 inputs, as in the reference's own cache test, with 64-token pages.
    _case("qwen_pages64_fp16", seq=420, hkv=2, dtype=torch.float16, page_size=64, sb=32,
          group=32, tier_probs=(0.15, 0.45, 0.4), appends=130, seed=12)
    # MiniCPM all-lowbit profile: K superblock 128, INT2 group 128, all INT2 values.
    _case("minicpm_lowbit_bf16", seq=300, hkv=2, dtype=torch.bfloat16, page_size=32, sb=128,
          group=128, tier_probs=(0.0, 0.0, 1.0), appends=129, seed=13)
    # matched BF16 cache (the 7B profile's first layers): survivors in page order, flush appends.
    _variant_case("matched_fp_bf16", variant="matched", seq=300, hkv=2, dtype=torch.bfloat16, page_size=32,
                  sb=32, group=32, tier_probs=(0.3, 0.3, 0.3, 0.1), appends=131, seed=14)
    # K-BF16 / V-FourQ cache: tiered values, bf16 keys; a flush is refused by the reference.
    _variant_case("kbf16_tiered_bf16", variant="bf16k", seq=330, hkv=2, dtype=torch.bfloat16, page_size=32,
                  sb=32, group=32, tier_probs=(0.2, 0.4, 0.4, 0.0), appends=130, seed=15)
    # compact INT2-K caches: Qwen-style 32-token K blocks, and MiniCPM-style 128-token blocks in fp16
    _VARIANTS["k_int2_tiered_bf16"]()
    _VARIANTS["k_int2_sb128_fp16"]()
    # generated INT4 values (generated_value_precision="int4")
    _VARIANTS["gen_int4_bf16"]()
    _VARIANTS["gen_int4_sb128_fp16"]()


_VARIANTS = {
    "k_int2_tiered_bf16": lambda: _variant_case("k_int2_tiered_bf16", variant="int2k", seq=333, hkv=2,
                                                dtype=torch.bfloat16, page_size=32, sb=32, group=32,
                                                tier_probs=(0.2, 0.4, 0.3, 0.1), appends=140, seed=16),
    # generated INT4 values: Qwen-style geometry (K superblock 32, INT2 group 32), two flushes, the
    # second after a ring that refilled across the first flush's K tail
    "gen_int4_bf16": lambda: _gen_int4_case("gen_int4_bf16", seq=333, hkv=2, dtype=torch.bfloat16, page_size=32,
                                            sb=32, group=32, tier_probs=(0.2, 0.5, 0.3), appends=260, seed=18),
    # fp16 with 64-token pages, K superblock 128, INT2 group 64
    "gen_int4_sb128_fp16": lambda: _gen_int4_case("gen_int4_sb128_fp16", seq=420, hkv=2, dtype=torch.float16,
                                                  page_size=64, sb=128, group=64, tier_probs=(0.15, 0.45, 0.4),
                                                  appends=131, seed=19),
    "k_int2_sb128_fp16": lambda: _variant_case("k_int2_sb128_fp16", variant="int2k", seq=300, hkv=2,
                                               dtype=torch.float16, page_size=64, sb=128, group=128,
                                               tier_probs=(0.1, 0.2, 0.7, 0.0), appends=131, seed=17),
    "matched_fp_bf16": lambda: _variant_case("matched_fp_bf16", variant="matched", seq=300, hkv=2,
                                             dtype=torch.bfloat16, page_size=32, sb=32, group=32,
                                             tier_probs=(0.3, 0.3, 0.3, 0.1), appends=131, seed=14),
    "kbf16_tiered_bf16": lambda: _variant_case("kbf16_tiered_bf16", variant="bf16k", seq=330, hkv=2,
                                               dtype=torch.bfloat16, page_size=32, sb=32, group=32,
                                               tier_probs=(0.2, 0.4, 0.4, 0.0), appends=130, seed=15),
}

if __name__ == "__main__":
    main()
