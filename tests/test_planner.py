"""CPU checks of the split-K work-item planner (host logic only, fake cache geometry).  The planner runs
in native code (r2o_plan_work_items, callable without a GPU); tests/planner_reference.py restates it in
Python, and the native plans must equal that restatement item for item."""
import random
from types import SimpleNamespace

import pytest

from r2omni_amd import _lib
from r2omni_amd.splitk import _TILE_COST, TILE, _segments, max_work_items, plan_work_items


def _fake_cache(s_fp, s_i4, s_i2, recent_cap=128, gen_i4=None):
    """Pool geometry of a cache; ``gen_i4`` (not None) makes its generated values INT4, with that
    many tokens flushed into the INT4 pool after the static ones."""
    n = SimpleNamespace
    i4_arena = None if gen_i4 is None else n(capacity=s_i4 + gen_i4 + 256)
    return n(compact_key=n(segment_offsets=(0, s_fp, s_fp + s_i4)), bf16_key=None, matched_fp=False,
             fp_pool=n(token_count=s_fp), int4_pool=n(token_count=s_i4 + (gen_i4 or 0)),
             compact_value=n(active_length=s_i2), recent_fp_pool=n(capacity=recent_cap),
             compact_int4_value=i4_arena, static_int4_tokens=s_i4, generated_k_offset=s_fp + s_i4 + s_i2)


def _random_cache(rnd, max_i2=60000, recent_caps=(128,)):
    sizes = (rnd.choice([0, rnd.randint(1, 20000)]), rnd.choice([0, rnd.randint(1, 40000)]),
             rnd.choice([0, rnd.randint(1, max_i2)]))
    gen = rnd.choice([None, None, 0, 128 * rnd.randint(1, 40)])
    return _fake_cache(*sizes, rnd.choice(recent_caps), gen_i4=gen)


@pytest.mark.parametrize("seed", range(40))
def test_items_cover_every_tile_once_and_respect_the_bound(seed):
    rnd = random.Random(seed)
    b = rnd.randint(1, 6)
    hkv = rnd.choice([1, 2, 4, 8])
    cus = rnd.choice([8, 64, 256])
    caches = [_random_cache(rnd) for _ in range(b)]
    extra = rnd.choice([0, 128, 256])
    items, begins = plan_work_items(caches, hkv, cus, extra_int2=extra)
    items = items.tolist()
    begins = begins.tolist()
    assert len(items) <= max_work_items(b, hkv, cus)
    # slots are 0..n-1, contiguous per (request, kv head) group, in group order
    assert sorted(it[8] for it in items) == list(range(len(items)))
    assert len(begins) == b * hkv + 1 and begins[0] == 0 and begins[-1] == len(items)
    by_slot = sorted(items, key=lambda it: it[8])
    for gi in range(b * hkv):
        for it in by_slot[begins[gi] : begins[gi + 1]]:
            assert (it[0], it[1]) == divmod(gi, hkv)
    # every tile of every segment (and of the Recent-FP ring) is covered exactly once
    for r, c in enumerate(caches):
        segs = _segments(c, extra) + [(_lib.KIND_RECENT, 0, c.recent_fp_pool.capacity, 0)]
        for h in range(hkv):
            for kind, lo, hi, vd in segs:
                mine = sorted((it[3], it[4]) for it in items
                              if it[0] == r and it[1] == h and it[2] == kind and it[5] == lo)
                t0 = lo // TILE * TILE
                pos = t0
                for tile0, ntiles in mine:
                    assert tile0 == pos and ntiles >= 1
                    pos += TILE * ntiles
                assert pos >= hi and pos - TILE < hi
                assert all(it[6] == hi and it[7] == vd
                           for it in items if it[0] == r and it[1] == h and it[2] == kind and it[5] == lo)
    # launch order: largest (cost-weighted) first
    costs = [it[4] * _TILE_COST[it[2]] for it in items]
    assert all(a >= b for a, b in zip(costs, costs[1:]))


@pytest.mark.parametrize("nt,n_items,share", [(4096, 64, 0.7), (4097, 63, 0.7), (100, 3, 0.7), (37, 2, 0.7),
                                              (8, 2, 0.7), (5, 2, 0.7), (4096, 64, 1.0), (130, 7, 0.5)])
def test_split_run_covers_the_run_with_wave_shares(nt, n_items, share):
    from planner_reference import split_run
    from r2omni_amd.splitk import _WAVES_PER_ITEM
    items = split_run(nt, n_items, share)
    assert 1 <= len(items) <= n_items
    assert items[0][0] == 0 and sum(s for _, s in items) == nt
    assert all(f2 == f1 + s1 for (f1, s1), (f2, _) in zip(items, items[1:]))
    assert all(s > 0 and s % _WAVES_PER_ITEM == 0 for _, s in items[:-1])
    if share < 1.0 and nt >= 64 * n_items:  # the later half gets about `share` of the earlier half's work
        big = items[: -(-n_items // 2)]
        small = items[-(-n_items // 2):-1]
        ratio = (sum(s for _, s in small) / len(small)) / (sum(s for _, s in big) / len(big))
        assert abs(ratio - share) < 0.1


def test_single_kind_plans_give_the_later_launched_half_less_work():
    """Two workgroups share a CU (launch slots j and j + CUs) and the earlier one runs ahead: an
    all-INT2 plan that fills both slots gives the later-launched half about the late share of the
    work, a mixed plan keeps equal items per run, and a plan within one slot per CU is even."""
    from r2omni_amd.splitk import _LATE_SHARE, _LATE_SHARE_BY_K
    share = _LATE_SHARE_BY_K.get(_lib.K_INT4, _LATE_SHARE)  # plan_work_items plans INT4-K caches
    cus = 256
    uniform = [_fake_cache(0, 0, 131072)]
    items = plan_work_items(uniform, 8, cus)[0].tolist()
    seg = [it for it in items if it[2] == _lib.KIND_INT2]
    assert len(items) > cus
    early = [it[4] for it in seg if items.index(it) < cus]
    late = [it[4] for it in seg if items.index(it) >= cus]
    ratio = (sum(late) / len(late)) / (sum(early) / len(early))
    assert abs(ratio - share) < 0.06
    mixed = [_fake_cache(8192, 24576, 32768), _fake_cache(2048, 6144, 8192)]
    items = plan_work_items(mixed, 4, cus)[0].tolist()
    for r in range(2):
        for h in range(4):
            for kind in (_lib.KIND_FP, _lib.KIND_INT4, _lib.KIND_INT2):
                sizes = [it[4] for it in items if (it[0], it[1], it[2]) == (r, h, kind)]
                assert max(sizes[:-1] or [0]) - min(sizes[:-1] or [0]) <= 0  # equal but the last
    small = plan_work_items([_fake_cache(0, 0, 4096)], 2, cus)[0].tolist()
    assert len(small) <= cus
    sizes = sorted(it[4] for it in small if it[2] == _lib.KIND_INT2)
    assert sizes[-1] - sizes[1] <= 4  # even (one wave share of rounding), the remainder aside


@pytest.mark.parametrize("seed", range(60))
def test_native_plan_equals_the_python_restatement(seed):
    from planner_reference import python_plan_work_items

    import torch

    rnd = random.Random(1000 + seed)
    b = rnd.randint(1, 8)
    hkv = rnd.choice([1, 2, 4, 8])
    cus = rnd.choice([8, 64, 80, 256])
    caches = [_random_cache(rnd, 131072, (32, 128, 256)) for _ in range(b)]
    extra = rnd.choice([0, 128, 256])
    got = plan_work_items(caches, hkv, cus, extra_int2=extra)
    want = python_plan_work_items(caches, hkv, cus, extra_int2=extra)
    assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])


@pytest.mark.parametrize("k_format,group", [(_lib.K_INT4, 32), (_lib.K_INT2, 128), (_lib.K_BF16, 64)])
def test_native_plan_fills_each_items_base_pointers(k_format, group):
    """With the host request descriptors the planner writes each item's base pointers: the per-head
    offsets into the request's K arena, K operand blocks, V pool, V scales and zeros, or its ring; and
    INT2-V items carry the V group size."""
    from planner_reference import item_pointers

    import torch

    from r2omni_amd.splitk import _plan

    rnd = random.Random(7)
    sizes = [(4096, 8192, 16384), (0, 3072, 640)]
    caches = [_fake_cache(*s) for s in sizes]
    hkv = 4
    words = []
    for r, (s_fp, s_i4, s_i2) in enumerate(sizes):
        w = {f: (r + 1) * (1 << 40) + (i + 1) * (1 << 32) for i, f in enumerate(_lib.REQUEST_FIELDS)}
        # random sizes that still hold every run (the planner rejects runs outside them)
        need = {"k_capacity": -(-(s_fp + s_i4 + s_i2) // 128) * 128, "k_superblocks": 1, "fp_stride": s_fp,
                "i4_stride": s_i4, "i2_stride": s_i2, "recent_capacity": 128}
        for f, lo in need.items():
            w[f] = rnd.randint(lo, lo + (1 << 14))
        if k_format == _lib.K_BF16:
            w["k_operands"] = 0
        words.append(w)
    reqs = torch.tensor([[w[f] for f in _lib.REQUEST_FIELDS] for w in words], dtype=torch.int64)
    items, _ = _plan(caches, hkv, 64, reqs=reqs, k_format=k_format, int2_group=group)
    for it in items.tolist():
        assert it[9:15] == item_pointers(words[it[0]], k_format, it[2], it[1], 128 // group)
        assert it[15] == (group if it[2] == _lib.KIND_INT2 else 0)  # v_group: INT2-V items carry the group size


@pytest.mark.parametrize("s_fp,s_i4,s_i2,gen,extra", [(640, 1000, 3000, 0, 0), (0, 0, 500, 256, 0),
                                                      (64, 4096, 0, 384, 128), (100, 37, 2000, 128, 256),
                                                      (0, 96, 64, 0, 128)])
def test_generated_int4_runs_map_every_int4_row_once(s_fp, s_i4, s_i2, gen, extra):
    """With INT4 generated values the INT4 pool is two K runs: its static segment, and the generated
    keys after the static INT2 segment.  Together their V rows (K position - v_delta) are the INT4-V
    arena's rows 0..n-1, each once, in that order; no run's K range overlaps another's; ``extra``
    tokens go to the generated run."""
    c = _fake_cache(s_fp, s_i4, s_i2, gen_i4=gen)
    segs = _segments(c, extra)
    runs4 = [(lo, hi, vd) for kind, lo, hi, vd in segs if kind == _lib.KIND_INT4]
    rows = [k - vd for lo, hi, vd in runs4 for k in range(lo, hi)]
    assert rows == list(range(s_i4 + gen + extra))
    spans = sorted((lo, hi) for _, lo, hi, _ in segs)
    assert all(a[1] <= b[0] for a, b in zip(spans, spans[1:]))
    i2 = [(lo, hi) for kind, lo, hi, _ in segs if kind == _lib.KIND_INT2]
    assert i2 == ([(s_fp + s_i4, s_fp + s_i4 + s_i2)] if s_i2 else [])
    if gen + extra:
        assert runs4[-1][:2] == (s_fp + s_i4 + s_i2, s_fp + s_i4 + s_i2 + gen + extra)


def _plan_raw(runs, reqs=None, n_reqs=1, n_groups=1, k_format=_lib.K_INT4, int2_group=32):
    """r2o_plan_work_items on explicit runs: (status, items as int64 rows)."""
    import ctypes

    import torch

    arr = (_lib.PlanRun * len(runs))(*[_lib.PlanRun(*r) for r in runs])
    cfg = _lib.PlanConfig(num_cus=8, blocks_per_cu=2, tiles_per_item=8, waves_per_item=4, min_tiles_per_item=4,
                          late_share=1.0)
    items = torch.zeros(64, 16, dtype=torch.int64)
    begins = torch.zeros(n_groups + 1, dtype=torch.int32)
    n = ctypes.c_int64(0)
    rc = _lib.load().r2o_plan_work_items(arr, len(runs), ctypes.byref(cfg), None if reqs is None else reqs.data_ptr(),
                                         n_reqs, k_format, int2_group, items.data_ptr(), 64, begins.data_ptr(),
                                         n_groups, ctypes.byref(n))
    return rc, items[: n.value].tolist()


def _reqs(k_capacity=1024, strides=(256, 256, 256), recent=128):
    import torch

    w = {f: (i + 1) << 32 for i, f in enumerate(_lib.REQUEST_FIELDS)}
    w.update(k_capacity=k_capacity, k_superblocks=k_capacity // 32, fp_stride=strides[0], i4_stride=strides[1],
             i2_stride=strides[2], recent_capacity=recent)
    return torch.tensor([[w[f] for f in _lib.REQUEST_FIELDS]], dtype=torch.int64)


@pytest.mark.parametrize("group", [32, 64, 128])
def test_int2_items_carry_their_group_without_descriptors(group):
    """The partial kernel takes the INT2-V group size from the item alone, so the planner writes it
    whether or not the request descriptors are given."""
    runs = [(0, 0, _lib.KIND_INT2, 0, 8, 0, 256, 0), (0, 0, _lib.KIND_RECENT, 0, 4, 0, 128, 0)]
    rc, items = _plan_raw(runs, int2_group=group)
    assert rc == 0 and items
    assert all(it[15] == (group if it[2] == _lib.KIND_INT2 else 0) for it in items)
    assert _plan_raw(runs, int2_group=48)[0] == 1            # an INT2 run needs a valid group
    assert _plan_raw(runs[1:], int2_group=0)[0] == 0         # a plan without INT2 runs does not


def test_planner_rejects_runs_outside_their_arena():
    """Runs whose tiles, valid range, KV head or V rows would make the partial kernel read outside the
    request's arenas are refused before any item is written."""
    ok = (0, 1, _lib.KIND_INT4, 64, 4, 70, 180, 0)
    reqs = _reqs()
    good = [ok[:1] + (0,) + ok[2:], ok]
    assert _plan_raw(good, reqs, n_groups=2)[0] == 0
    # every group (request g / hkv, KV head g % hkv) has runs, in group order
    assert _plan_raw([ok], reqs, n_groups=2)[0] == 1
    assert _plan_raw(good[::-1], reqs, n_groups=2)[0] == 1
    assert _plan_raw(good, reqs, n_groups=3)[0] == 1
    bad = {
        "kvh past the request's heads": (0, 2, _lib.KIND_INT4, 64, 4, 70, 180, 0),
        "request past the batch": (1, 1, _lib.KIND_INT4, 64, 4, 70, 180, 0),
        "negative kvh": (0, -1, _lib.KIND_INT4, 64, 4, 70, 180, 0),
        "lo > hi": (0, 1, _lib.KIND_INT4, 64, 4, 180, 70, 0),
        "empty range": (0, 1, _lib.KIND_INT4, 64, 4, 100, 100, 0),
        "tile0 > lo": (0, 1, _lib.KIND_INT4, 96, 4, 70, 180, 0),
        "unaligned tile0": (0, 1, _lib.KIND_INT4, 48, 4, 70, 180, 0),
        "hi past the tiles": (0, 1, _lib.KIND_INT4, 64, 2, 70, 180, 0),
        "tiles past the K arena": (0, 1, _lib.KIND_INT4, 960, 4, 960, 1000, 0),
        "V rows past the pool": (0, 1, _lib.KIND_INT2, 64, 8, 70, 300, 0),
        "V rows before the pool": (0, 1, _lib.KIND_FP, 64, 4, 70, 180, 100),
        "ring tiles past the ring": (0, 1, _lib.KIND_RECENT, 0, 8, 0, 256, 0),
    }
    for what, run in bad.items():
        assert _plan_raw([good[0], run], reqs, n_groups=2)[0] == 1, what
        if what in ("kvh past the request's heads", "negative kvh", "request past the batch", "lo > hi",
                    "empty range", "tile0 > lo", "unaligned tile0", "hi past the tiles"):
            assert _plan_raw([good[0], run], None, n_groups=2)[0] == 1, what  # checked without descriptors too


@pytest.mark.parametrize("value,b,want", [
    (7, 3, [7, 7, 7]), (True, 2, [1, 1]), ([5], 3, [5, 5, 5]), ((4, 5), 2, [4, 5]), ([4, 5, 6], 3, [4, 5, 6]),
    ([True, 2], 2, [1, 2]), ("tensor", 2, [8, 9]), ("tensor1", 3, [8, 8, 8]),
])
def test_per_request_positions_take_every_form_of_the_reference(value, b, want):
    """The append's (global, logical) positions: an int, one value per request, or a single value
    broadcast, as ints, lists, tuples or tensors (triton_fourq_splitk.py:1336-1354); the fast path for
    plain ints and lists of ints gives what the general path gives."""
    import torch

    from r2omni_amd.splitk import _per_request

    if value == "tensor":
        value = torch.tensor([8, 9])
    elif value == "tensor1":
        value = torch.tensor([8])
    got = _per_request(value, b)
    assert got == want and all(type(v) is int for v in got)
    if isinstance(value, list):  # a fresh list: the caller's is never handed on
        assert got is not value


def test_per_request_positions_reject_a_wrong_count():
    from r2omni_amd.splitk import _per_request

    with pytest.raises(ValueError, match="one value per request"):
        _per_request([1, 2, 3], 2)
    with pytest.raises(ValueError, match="one value per request"):
        _per_request((1, 2), 3)
