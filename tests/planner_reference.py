"""Python restatement of the split-K work-item planner (test infrastructure).

The product plans in native code (r2o_plan_work_items, r2-omni_amd/csrc/r2o_plan.cpp); this module
states the same algorithm in Python so that tests/test_planner.py can check the native plans item for
item on random cache geometries.  Nothing in the package imports it.
"""
from __future__ import annotations

import heapq

import torch

from r2omni_amd import _lib
from r2omni_amd.splitk import (TILE, _BLOCKS_PER_CU, _LATE_SHARE, _LATE_SHARE_BY_K, _MIN_TILES_PER_ITEM, _TILE_COST,
                               _TILES_PER_ITEM_TARGET, _WAVES_PER_ITEM, _plan_runs)


def split_run(nt: int, n_items: int, late_share: float = 1.0):
    """(first tile, tiles) of the items of one run: multiples of a wave share each, all but the
    last; with late_share < 1 the second half of the items gets that share of the first half's."""
    w = _WAVES_PER_ITEM
    if late_share >= 1.0 or n_items < 2:
        n = -(-(-(-nt // n_items)) // w) * w  # even split, a share per wave
        return [(f, min(n, nt - f)) for f in range(0, nt, n)]
    big = -(-n_items // 2)
    small = n_items - big
    x = nt / (big + late_share * small)
    bsize = -(-int(round(x)) // w) * w
    out, f = [], 0
    for k in range(n_items):
        if f >= nt:
            break
        if k < big:
            size = bsize
        else:
            left = n_items - k
            size = -(-(-(-(nt - f) // left)) // w) * w
        size = min(size, nt - f)
        out.append((f, size))
        f += size
    if f < nt:  # rounding left a remainder: extend the last item
        last_f, last_s = out[-1]
        out[-1] = (last_f, last_s + nt - f)
    return out


def python_plan_work_items(caches, hkv: int, num_cus: int, extra_int2: int = 0, k_format: int = _lib.K_INT4):
    """Water-filling of the runs (the most expensive run's items split once more, ties to the earlier
    run, until 2 x CUs items, or about _TILES_PER_ITEM_TARGET tiles per item but at least CUs items),
    partial slots in (request, kv head) order, launch order largest first.  Returns
    (items [n, 9] int64, group_begin [B*hkv + 1] int32)."""
    runs = _plan_runs(caches, hkv, extra_int2)
    cus = max(1, num_cus)
    total_tiles = sum(r[4] for r in runs)
    target = min(_BLOCKS_PER_CU * cus, max(cus, total_tiles // _TILES_PER_ITEM_TARGET))
    counts = [1] * len(runs)

    def item_cost(i: int) -> float:
        nt = runs[i][4]
        per = -(-nt // counts[i])
        return (-(-per // _WAVES_PER_ITEM) * _WAVES_PER_ITEM) * _TILE_COST[runs[i][2]]

    heap = [(-item_cost(i), i) for i in range(len(runs))]
    heapq.heapify(heap)
    total = sum(counts)
    while total < target and heap:
        _, i = heapq.heappop(heap)
        if -(-runs[i][4] // (counts[i] + 1)) < _MIN_TILES_PER_ITEM:
            continue  # already at the smallest useful item size
        counts[i] += 1
        total += 1
        heapq.heappush(heap, (-item_cost(i), i))
    uniform = len({r[2] for r in runs if r[2] != _lib.KIND_RECENT}) == 1
    late_share = _LATE_SHARE_BY_K.get(k_format, _LATE_SHARE) if uniform and total > cus else 1.0
    items = []
    begins = [0]
    group = (0, 0)
    for (r, h, kind, t0, nt, lo, hi, vd), n_items in zip(runs, counts):
        if (r, h) != group:
            begins.append(len(items))
            group = (r, h)
        for first, size in split_run(nt, n_items, late_share):
            items.append([r, h, kind, t0 + TILE * first, size, lo, hi, vd, len(items)])
    begins.append(len(items))
    items.sort(key=lambda it: -it[4] * _TILE_COST[it[2]])  # stable: largest first, ties keep slot order
    return torch.tensor(items, dtype=torch.int64), torch.tensor(begins, dtype=torch.int32)


_K_ROW_BYTES = {_lib.K_INT4: 64, _lib.K_INT2: 32, _lib.K_BF16: 256}


def item_pointers(words: dict, k_format: int, kind: int, h: int, groups: int) -> list:
    """Base pointers (k_base, k_ops, v_base, v_scale, v_zero, ring_length) of KV head ``h`` for an
    item of ``kind``, from one request's descriptor words (byte addresses)."""
    if kind == _lib.KIND_RECENT:
        row = h * words["recent_capacity"] * 256
        return [words["recent_k"] + row, 0, words["recent_v"] + row, 0, 0, words["recent_length"]]
    k_base = words["k_packed"] + h * words["k_capacity"] * _K_ROW_BYTES[k_format]
    k_ops = words["k_operands"] + h * words["k_superblocks"] * 128 * 4 if words["k_operands"] else 0
    if kind == _lib.KIND_FP:
        return [k_base, k_ops, words["fp_v"] + h * words["fp_stride"] * 256, 0, 0, 0]
    if kind == _lib.KIND_INT4:
        st = words["i4_stride"]
        return [k_base, k_ops, words["i4_v"] + h * st * 64, words["i4_scale"] + h * st * 4, 0, 0]
    st = words["i2_stride"]
    return [k_base, k_ops, words["i2_v"] + h * st * 32, words["i2_scale"] + h * st * groups * 2,
            words["i2_zero"] + h * st * groups, 0]
