"""Page-table boundary types of the SSPA cache (host-side index bookkeeping).

Same names, fields and error behaviour as the reference's policy/runtime types that feed
``build_three_precision_cache``:
  PageClass                  r2omni/sspa/policy/four_quadrant.py:6-12
  PageTable, PageAssignment  r2omni/sspa/policy/page_assignment.py:11-33
  build_page_table           page_assignment.py:63-137  (pages never cross a modality change)
  project_token_bits_to_pages page_assignment.py:36-60   (16 > 4 > 2 > 0 bits per page)
  LayerCompressionPlan, build_layer_compression_plan  r2omni/sspa/runtime/cache_plan.py:11-52
The precision policy that decides the bits (scoring, allocation) is not part of the decode path.
"""
from __future__ import annotations

from dataclasses import dataclass
from enum import IntEnum

import torch

TEXT, VIDEO, AUDIO, OTHER = 0, 1, 2, 3


class PageClass(IntEnum):
    EVICTED_PAGE = 0
    FP_PAGE = 1
    INT4_PAGE = 2
    RECENT_FP_PAGE = 3
    PROTECTED_FP_PAGE = 4
    INT2_PAGE = 5


@dataclass(frozen=True)
class PageTable:
    offsets: torch.Tensor
    lengths: torch.Tensor
    modality: torch.Tensor
    token_indices: torch.Tensor
    logical_positions: torch.Tensor
    global_token_indices: torch.Tensor
    protected: torch.Tensor
    recent: torch.Tensor

    @property
    def num_pages(self) -> int:
        return int(self.offsets.numel())


@dataclass(frozen=True)
class PageAssignment:
    page_table: PageTable
    page_classes: torch.Tensor
    attention_scores: torch.Tensor
    alignment_scores: torch.Tensor
    fused_scores: torch.Tensor


def build_page_table(modality: torch.Tensor, *, page_size: int = 32, logical_positions=None,
                     global_token_indices=None, protected_mask=None, recent_mask=None) -> PageTable:
    """Split the token sequence into runs of one modality, at most ``page_size`` long."""
    if page_size not in (16, 32, 64):
        raise ValueError("page_size must be one of 16, 32, or 64")
    mod = modality.flatten().to(torch.long)
    n = int(mod.numel())
    dev = mod.device

    def per_token(value, default, dtype):
        out = default if value is None else value.flatten().to(device=dev, dtype=dtype)
        return out

    logical = per_token(logical_positions, torch.arange(n, device=dev), torch.long)
    global_idx = per_token(global_token_indices, torch.arange(n, device=dev), torch.long)
    protected = per_token(protected_mask, (mod == TEXT) | (mod == OTHER), torch.bool)
    recent = per_token(recent_mask, torch.zeros(n, dtype=torch.bool, device=dev), torch.bool)
    for name, v in (("logical_positions", logical), ("global_token_indices", global_idx),
                    ("protected_mask", protected), ("recent_mask", recent)):
        if v.numel() != n:
            raise ValueError(f"{name} must have one value per token")
    mods, prot, rec = mod.tolist(), protected.tolist(), recent.tolist()
    offsets, lengths, pmod, pprot, prec = [], [], [], [], []
    start = 0
    while start < n:
        end = start + 1
        while end < n and end - start < page_size and mods[end] == mods[start]:
            end += 1
        offsets.append(start)
        lengths.append(end - start)
        pmod.append(mods[start])
        pprot.append(any(prot[start:end]))
        prec.append(any(rec[start:end]))
        start = end
    as_long = lambda xs: torch.tensor(xs, dtype=torch.long, device=dev)  # noqa: E731
    return PageTable(
        offsets=as_long(offsets), lengths=as_long(lengths), modality=as_long(pmod),
        token_indices=torch.arange(n, dtype=torch.long, device=dev),
        logical_positions=logical.clone(), global_token_indices=global_idx.clone(),
        protected=torch.tensor(pprot, dtype=torch.bool, device=dev),
        recent=torch.tensor(prec, dtype=torch.bool, device=dev),
    )


def project_token_bits_to_pages(page_table: PageTable, token_bits: torch.Tensor) -> PageAssignment:
    """Page class = the widest precision any of its tokens asks for (protected/recent win)."""
    bits = token_bits.flatten().to(device=page_table.offsets.device, dtype=torch.int8)
    if bits.numel() != page_table.token_indices.numel():
        raise ValueError("token_bits must have one value per page-table token")
    if not bool(torch.all((bits == 0) | (bits == 2) | (bits == 4) | (bits == 16))):
        raise ValueError("token_bits may contain only 0, 2, 4, or 16")
    classes = []
    bits_l = bits.tolist()
    for page, (off, ln) in enumerate(zip(page_table.offsets.tolist(), page_table.lengths.tolist())):
        present = set(bits_l[off : off + ln])
        if bool(page_table.protected[page]):
            cls = PageClass.PROTECTED_FP_PAGE
        elif bool(page_table.recent[page]):
            cls = PageClass.RECENT_FP_PAGE
        elif 16 in present:
            cls = PageClass.FP_PAGE
        elif 4 in present:
            cls = PageClass.INT4_PAGE
        elif 2 in present:
            cls = PageClass.INT2_PAGE
        else:
            cls = PageClass.EVICTED_PAGE
        classes.append(int(cls))
    dev = bits.device
    zeros = torch.zeros(page_table.num_pages, device=dev, dtype=torch.float32)
    return PageAssignment(page_table, torch.tensor(classes, dtype=torch.int8, device=dev), zeros, zeros, zeros)


@dataclass(frozen=True)
class LayerCompressionPlan:
    layer_id: int
    fp_pages: torch.Tensor
    int4_pages: torch.Tensor
    int2_pages: torch.Tensor
    evicted_pages: torch.Tensor
    protected_pages: torch.Tensor
    recent_fp_capacity: int
    logical_positions: torch.Tensor
    global_token_indices: torch.Tensor
    page_offsets: torch.Tensor
    page_lengths: torch.Tensor
    page_classes: torch.Tensor
    # Host copy of (page_classes, page_offsets, page_lengths) as int64 [3, pages] when the plan was
    # made from host data: the cache build then sorts the page table without a device round trip.
    host_page_table: torch.Tensor | None = None


def build_layer_compression_plan(layer_id: int, assignment: PageAssignment, *,
                                 recent_fp_capacity: int = 256) -> LayerCompressionPlan:
    if layer_id < 0:
        raise ValueError("layer_id must be non-negative")
    if recent_fp_capacity <= 0:
        raise ValueError("recent_fp_capacity must be positive")
    cls = assignment.page_classes
    pages = lambda mask: mask.nonzero(as_tuple=False).flatten()  # noqa: E731
    fp = (cls == PageClass.FP_PAGE) | (cls == PageClass.RECENT_FP_PAGE) | (cls == PageClass.PROTECTED_FP_PAGE)
    table = assignment.page_table
    return LayerCompressionPlan(
        layer_id=int(layer_id), fp_pages=pages(fp), int4_pages=pages(cls == PageClass.INT4_PAGE),
        int2_pages=pages(cls == PageClass.INT2_PAGE), evicted_pages=pages(cls == PageClass.EVICTED_PAGE),
        protected_pages=pages(cls == PageClass.PROTECTED_FP_PAGE), recent_fp_capacity=int(recent_fp_capacity),
        logical_positions=table.logical_positions.clone(), global_token_indices=table.global_token_indices.clone(),
        page_offsets=table.offsets.clone(), page_lengths=table.lengths.clone(), page_classes=cls.clone(),
    )


def plan_from_pages(page_offsets, page_lengths, page_classes, *, recent_fp_capacity: int = 128,
                    device=None) -> LayerCompressionPlan:
    """Plan from explicit page geometry (synthetic workloads and tests)."""
    dev = torch.device(device) if device is not None else torch.device("cpu")
    host = None
    if all(not (isinstance(v, torch.Tensor) and v.device.type != "cpu")
           for v in (page_offsets, page_lengths, page_classes)):
        host = torch.stack([torch.as_tensor(v, dtype=torch.long) for v in (page_classes, page_offsets, page_lengths)])
    offs = torch.as_tensor(page_offsets, dtype=torch.long, device=dev)
    lens = torch.as_tensor(page_lengths, dtype=torch.long, device=dev)
    cls = torch.as_tensor(page_classes, dtype=torch.long, device=dev)
    total = int(lens.sum())
    positions = torch.arange(total, dtype=torch.long, device=dev)
    pages = lambda mask: mask.nonzero(as_tuple=False).flatten()  # noqa: E731
    fp = (cls == PageClass.FP_PAGE) | (cls == PageClass.RECENT_FP_PAGE) | (cls == PageClass.PROTECTED_FP_PAGE)
    return LayerCompressionPlan(
        layer_id=0, fp_pages=pages(fp), int4_pages=pages(cls == PageClass.INT4_PAGE),
        int2_pages=pages(cls == PageClass.INT2_PAGE), evicted_pages=pages(cls == PageClass.EVICTED_PAGE),
        protected_pages=pages(cls == PageClass.PROTECTED_FP_PAGE), recent_fp_capacity=int(recent_fp_capacity),
        logical_positions=positions, global_token_indices=positions.clone(), page_offsets=offs,
        page_lengths=lens, page_classes=cls, host_page_table=host,
    )
