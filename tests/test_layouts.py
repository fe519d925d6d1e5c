"""CPU checks of the tier-ordered page layout (host logic of build_three_precision_cache) against a
plain per-page restatement of precision_pool.py:611-669: pages stably sorted FP (+protected,
recent) < INT4 < INT2 < evicted, each pool's tokens in page order, offsets restarting per pool."""
import dataclasses
import random

import pytest
import torch

from r2omni_amd.cache import _compact_page_layouts
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


@pytest.mark.parametrize("seed", range(30))
def test_layouts_match_a_per_page_loop(seed):
    rnd = random.Random(seed)
    n = rnd.randint(1, 80)
    lens = [rnd.choice([16, 32, 64]) for _ in range(n)]
    offs = [sum(lens[:i]) for i in range(n)]
    cls = [rnd.choice(list(TIER)) for _ in range(n)]
    plan = plan_from_pages(offs, lens, cls, recent_fp_capacity=128)
    assert plan.host_page_table is not None
    want = _per_page(offs, lens, cls)
    # with the host copy of the page table, and without it (a plan made on the device has none)
    for p in (plan, dataclasses.replace(plan, host_page_table=None)):
        got = _compact_page_layouts(p, "cpu")
        for g, w in zip((got[0], got[1], got[2], got[4]), want):
            for gx, wx in zip(g, w):
                assert gx.tolist() == list(wx)
        assert all(t.numel() == 0 for t in got[3])  # the Recent-FP pool starts empty
