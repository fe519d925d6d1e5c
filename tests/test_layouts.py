"""CPU checks of the cache build's host logic against plain per-page restatements.

* Tier order (precision_pool.py:611-669): pages stably sorted FP (+protected, recent) < INT4 < INT2 <
  evicted, each pool's tokens in page order, offsets restarting per pool.
* The metadata arena (precision_pool.py:400-585): one int64 allocation whose views are every pool's
  page index, the evicted global indices and the Recent-FP ring's buffers; the INT2 fields reserve
  whole pages whose page fields are written ahead, and an INT2 flush fills them in place
  (precision_pool.py:66-118).
"""
import dataclasses
import random

import pytest
import torch

from r2omni_amd.cache import (PrecisionPool, _build_metadata_arena, _expand_tier_tokens, _tier_page_table)
from r2omni_amd.policy import PageClass, plan_from_pages

TIER = {int(PageClass.FP_PAGE): 0, int(PageClass.PROTECTED_FP_PAGE): 0, int(PageClass.RECENT_FP_PAGE): 0,
        int(PageClass.INT4_PAGE): 1, int(PageClass.INT2_PAGE): 2, int(PageClass.EVICTED_PAGE): 3}


def _per_page(offs, lens, cls):
    out = []
    for tier in range(4):
        pages = [p for p in range(len(cls)) if TIER[cls[p]] == tier]
        tokens, offsets, pos = [], [], 0
        for p in pages:
            offsets.append(pos)
            tokens.extend(range(offs[p], offs[p] + lens[p]))
            pos += lens[p]
        out.append((tokens, offsets, [lens[p] for p in pages], pages))
    return out


def _random_plan(seed, page_sizes=(16, 32, 64), recent=128):
    rnd = random.Random(seed)
    n = rnd.randint(1, 80)
    lens = [rnd.choice(page_sizes) for _ in range(n)]
    offs = [sum(lens[:i]) for i in range(n)]
    cls = [rnd.choice(list(TIER)) for _ in range(n)]
    return plan_from_pages(offs, lens, cls, recent_fp_capacity=recent), offs, lens, cls


@pytest.mark.parametrize("seed", range(30))
def test_tier_tokens_match_a_per_page_loop(seed):
    plan, offs, lens, cls = _random_plan(seed)
    assert plan.host_page_table is not None
    want = _per_page(offs, lens, cls)
    # with the host copy of the page table, and without it (a plan made on the device has none)
    for p in (plan, dataclasses.replace(plan, host_page_table=None)):
        tab = _tier_page_table(p)
        tokens = _expand_tier_tokens(tab, "cpu").tolist()
        t0 = 0
        for t, (w_tok, w_off, w_len, w_pages) in enumerate(want):
            sl = slice(int(tab.first_page[t]), int(tab.first_page[t + 1]))
            assert tab.pages[sl].tolist() == w_pages
            assert tab.offsets[sl].tolist() == w_off
            assert tab.lengths[sl].tolist() == w_len
            assert tokens[t0:t0 + len(w_tok)] == w_tok
            t0 += len(w_tok)
        assert t0 == len(tokens) == sum(lens)


def _arena(plan, reserve, recent, reserve4=0):
    tab = _tier_page_table(plan)
    tokens = _expand_tier_tokens(tab, "cpu")
    gi = torch.arange(plan.global_token_indices.numel()) * 7 + 3   # distinct from token ids
    lp = torch.arange(plan.logical_positions.numel()) * 5 + 1
    return tab, gi, lp, _build_metadata_arena(tab, tokens, gi, lp, page_size=32, recent_capacity=recent,
                                              int2_reserve=reserve, int4_reserve=reserve4)


@pytest.mark.parametrize("seed", range(20))
@pytest.mark.parametrize("reserve,reserve4", [(0, 0), (128, 0), (256, 0), (0, 256), (128, 96)])
def test_metadata_arena_views_match_a_per_page_loop(seed, reserve, reserve4):
    plan, offs, lens, cls = _random_plan(seed, page_sizes=(32,))
    want = _per_page(offs, lens, cls)
    tab, gi, lp, (arena, indexes, evicted, (ring_g, ring_l, ring_len)) = _arena(plan, reserve, 128, reserve4)
    storage = arena.storage
    views = [evicted, ring_g, ring_l, ring_len] + [getattr(pi, f.name) for pi in indexes
                                                   for f in dataclasses.fields(pi)]
    for v in views:  # one allocation backs every field
        assert v.untyped_storage().data_ptr() == storage.untyped_storage().data_ptr()
    for t in range(3):
        w_tok, w_off, w_len, w_pages = want[t]
        pi = indexes[t]
        assert pi.original_page_ids.tolist() == w_pages
        assert pi.physical_offsets.tolist() == w_off
        assert pi.lengths.tolist() == w_len
        assert pi.global_token_indices.tolist() == gi[w_tok].tolist()
        assert pi.logical_positions.tolist() == lp[w_tok].tolist()
    assert evicted.tolist() == gi[want[3][0]].tolist()
    ring = indexes[3]
    assert ring.original_page_ids.tolist() == [-1] * 4
    assert ring.physical_offsets.tolist() == [0, 32, 64, 96]
    assert ring.lengths.tolist() == [0] * 4
    assert ring_g.tolist() == ring_l.tolist() == [-1] * 128
    assert ring.global_token_indices is ring_g and ring.logical_positions is ring_l
    assert ring_len.dtype == torch.int32 and ring_len.dim() == 0 and int(ring_len) == 0
    # the INT4 and INT2 reserves: page fields written ahead, token fields -1
    for tier, t, r in (("int4", 1, reserve4), ("int2", 2, reserve)):
        n_t, p_t = len(want[t][0]), len(want[t][3])
        assert getattr(arena, f"{tier}_page_count") == p_t and getattr(arena, f"{tier}_token_count") == n_t
        buf = lambda name: getattr(arena, f"{tier}_{name}_buffer")  # noqa: E731
        assert buf("lengths").numel() == p_t + r // 32
        assert buf("original_page_ids")[p_t:].tolist() == [-1] * (r // 32)
        assert buf("physical_offsets")[p_t:].tolist() == [n_t + 32 * k for k in range(r // 32)]
        assert buf("lengths")[p_t:].tolist() == [32] * (r // 32)
        assert buf("global_index")[n_t:].tolist() == [-1] * r
        assert buf("logical_position")[n_t:].tolist() == [-1] * r
        assert buf("global_index")[:n_t].tolist() == gi[want[t][0]].tolist()
    # one allocation of exactly the fields' sizes
    pages = len(lens) - len(want[3][3]) + (reserve + reserve4) // 32 + 4
    assert storage.numel() == 3 * pages + 1 + 2 * (sum(lens) - len(want[3][0]) + reserve + reserve4) \
        + len(want[3][0]) + 256


def test_int2_flush_metadata_is_written_in_place():
    plan, offs, lens, cls = _random_plan(3, page_sizes=(32,))
    want = _per_page(offs, lens, cls)
    tab, gi, lp, (arena, indexes, evicted, _) = _arena(plan, 256, 128)
    pool = PrecisionPool(name="int2", page_index=indexes[2])
    before = arena.storage.clone()
    fp_pi, i4_pi = indexes[0], indexes[1]
    n_i2, p_i2 = len(want[2][0]), len(want[2][3])
    for k in range(2):
        g = torch.arange(128) + 1000 * (k + 1)
        arena.append_int2_pages(pool, g, -g, 32)
        pi = pool.page_index
        assert pi.lengths.numel() == p_i2 + 4 * (k + 1)
        assert pi.global_token_indices.tolist()[n_i2 + 128 * k:] == g.tolist()
        assert pi.logical_positions.tolist()[n_i2 + 128 * k:] == (-g).tolist()
        assert pi.physical_offsets.tolist()[p_i2:] == [n_i2 + 32 * j for j in range(4 * (k + 1))]
        assert pi.global_token_indices.data_ptr() == arena.int2_global_index_buffer.data_ptr()
    # nothing outside the INT2 token fields changed, and the reserve is now exhausted
    changed = (arena.storage != before).nonzero().flatten()
    g0 = arena.int2_global_index_buffer.data_ptr() // 8 - arena.storage.data_ptr() // 8
    l0 = arena.int2_logical_position_buffer.data_ptr() // 8 - arena.storage.data_ptr() // 8
    allowed = set(range(g0 + n_i2, g0 + n_i2 + 256)) | set(range(l0 + n_i2, l0 + n_i2 + 256))
    assert set(changed.tolist()) <= allowed
    assert fp_pi.global_token_indices.tolist() == gi[want[0][0]].tolist()
    with pytest.raises(RuntimeError, match="capacity exhausted"):
        arena.append_int2_pages(pool, torch.arange(32), torch.arange(32), 32)
    with pytest.raises(ValueError, match="complete pages"):
        arena.append_int2_pages(pool, torch.arange(31), torch.arange(31), 32)


def test_int4_flush_metadata_is_written_in_place():
    """Generated INT4 values: flushed pages continue the INT4 pool in its reserve, and neither the
    INT2 pool's fields nor anything else in the arena changes (precision_pool.py:136-149)."""
    plan, offs, lens, cls = _random_plan(5, page_sizes=(32,))
    want = _per_page(offs, lens, cls)
    tab, gi, lp, (arena, indexes, evicted, _) = _arena(plan, 64, 128, reserve4=256)
    pool = PrecisionPool(name="int4", page_index=indexes[1])
    before = arena.storage.clone()
    n_i4, p_i4 = len(want[1][0]), len(want[1][3])
    for k in range(2):
        g = torch.arange(128) + 1000 * (k + 1)
        arena.append_int4_pages(pool, g, -g, 32)
        pi = pool.page_index
        assert pool.token_count == n_i4 + 128 * (k + 1)
        assert pi.lengths.numel() == p_i4 + 4 * (k + 1)
        assert pi.global_token_indices.tolist()[:n_i4] == gi[want[1][0]].tolist()
        assert pi.global_token_indices.tolist()[n_i4 + 128 * k:] == g.tolist()
        assert pi.logical_positions.tolist()[n_i4 + 128 * k:] == (-g).tolist()
        assert pi.physical_offsets.tolist()[p_i4:] == [n_i4 + 32 * j for j in range(4 * (k + 1))]
        assert pi.global_token_indices.data_ptr() == arena.int4_global_index_buffer.data_ptr()
    changed = (arena.storage != before).nonzero().flatten()
    g0 = arena.int4_global_index_buffer.data_ptr() // 8 - arena.storage.data_ptr() // 8
    l0 = arena.int4_logical_position_buffer.data_ptr() // 8 - arena.storage.data_ptr() // 8
    allowed = set(range(g0 + n_i4, g0 + n_i4 + 256)) | set(range(l0 + n_i4, l0 + n_i4 + 256))
    assert set(changed.tolist()) <= allowed
    assert arena.int2_token_count == len(want[2][0])
    assert indexes[2].global_token_indices.tolist() == gi[want[2][0]].tolist()
    with pytest.raises(RuntimeError, match="INT4 page metadata capacity exhausted"):
        arena.append_int4_pages(pool, torch.arange(32), torch.arange(32), 32)
    with pytest.raises(ValueError, match="complete pages"):
        arena.append_int4_pages(pool, torch.arange(31), torch.arange(31), 32)
