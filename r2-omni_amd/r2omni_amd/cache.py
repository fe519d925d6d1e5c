"""Three-pool SSPA packed-KV cache on the GPU: arenas, builder, append and flush.

Drop-in for the reference runtime (same names, fields, layouts and error messages):
  CompactInt4KeyArena        r2omni/sspa/runtime/compact_int4_key.py:113-220
  build (INT4-K gather-pack) compact_int4_key.py:223-281
  PackedTensor (INT4-V pool) packed_kv_layout.py:11-32, fused_value_pack.py:152-193
  CompactInt4ValueArena      fused_value_pack.py:196-299, build :302-330 (generated INT4 values)
  CompactInt2ValueArena      fused_value_pack.py:401-516, build :519-575
  PrecisionPool, ThreePrecisionCache, build_three_precision_cache  precision_pool.py:152-274, 787-984
  CompactMetadataArena       precision_pool.py:45-145, 400-585
  append_generated_token, DynamicCacheStats  dynamic_fourq_cache.py:16-24, 172-267
All payload bytes are produced by the gfx950 kernels of libr2o_sspa.so (r2o_pack_int4_k,
r2o_pack_int4_v, r2o_pack_int2_v, r2o_gather_rows, r2o_recent_append, r2o_recent_shift);
torch only allocates the tensors and keeps small index vectors.  Variants: the released
``v_fourq_k_int4_compact`` cache, ``v_fourq_k_int2_compact``, ``v_fourq_k_bf16`` and the matched-FP
cache; generated (flushed) values INT2 (released) or INT4 (``generated_value_precision="int4"``).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Literal, NamedTuple

import numpy as np
import torch

from . import _lib
from .policy import LayerCompressionPlan, PageClass

CacheVariant = Literal["v_fourq_k_int2_compact", "v_fourq_k_int4_compact", "v_fourq_k_bf16"]


def _round_up(value: int, multiple: int) -> int:
    return -(-int(value) // int(multiple)) * int(multiple)


def _nbytes(t: torch.Tensor | None) -> int:
    return 0 if t is None else int(t.numel() * t.element_size())


# ----------------------------------------------------------------------------- page index
@dataclass(frozen=True)
class PhysicalPageIndex:
    original_page_ids: torch.Tensor
    physical_offsets: torch.Tensor
    lengths: torch.Tensor
    global_token_indices: torch.Tensor
    logical_positions: torch.Tensor


@dataclass
class CompactMetadataArena:
    """Every page and token index of a compact cache in one int64 allocation
    (precision_pool.py:45-145, 400-585).

    The INT4 and INT2 pools' five fields are each reserved up to what their packed V arena and the
    compact K arena can still take (INT4 only when generated values are INT4), and the page fields
    of the reserved pages (id -1, offsets continuing the pool, full length) are written at build
    time, so a flush copies its token indices in place and allocates nothing.  The flushed pool's
    ``page_index`` is re-pointed at longer views of the same buffers.
    """

    storage: torch.Tensor
    int2_original_page_ids_buffer: torch.Tensor
    int2_physical_offsets_buffer: torch.Tensor
    int2_lengths_buffer: torch.Tensor
    int2_global_index_buffer: torch.Tensor
    int2_logical_position_buffer: torch.Tensor
    int2_page_count: int
    int2_token_count: int
    int4_original_page_ids_buffer: torch.Tensor
    int4_physical_offsets_buffer: torch.Tensor
    int4_lengths_buffer: torch.Tensor
    int4_global_index_buffer: torch.Tensor
    int4_logical_position_buffer: torch.Tensor
    int4_page_count: int
    int4_token_count: int

    def _append_pages(self, pool: "PrecisionPool", global_indices: torch.Tensor, logical_positions: torch.Tensor,
                      page_size: int, tier: str) -> None:
        n = int(global_indices.numel())
        if n <= 0 or n != int(logical_positions.numel()) or n % int(page_size):
            raise ValueError(f"compact {tier.upper()} metadata append requires matching complete pages")
        if global_indices.dtype != torch.long or logical_positions.dtype != torch.long \
                or global_indices.device != self.storage.device or logical_positions.device != self.storage.device:
            raise ValueError(f"compact {tier.upper()} metadata append requires same-device int64 indices")
        ids, offs, lens, g, l = (getattr(self, f"{tier}_{name}_buffer") for name in
                                 ("original_page_ids", "physical_offsets", "lengths", "global_index",
                                  "logical_position"))
        pages, tokens = getattr(self, f"{tier}_page_count"), getattr(self, f"{tier}_token_count")
        page_end = pages + n // int(page_size)
        token_end = tokens + n
        if page_end > lens.numel():
            raise RuntimeError(f"compact {tier.upper()} page metadata capacity exhausted")
        if token_end > g.numel():
            raise RuntimeError(f"compact {tier.upper()} token metadata capacity exhausted")
        g[tokens:token_end].copy_(global_indices)
        l[tokens:token_end].copy_(logical_positions)
        setattr(self, f"{tier}_page_count", page_end)
        setattr(self, f"{tier}_token_count", token_end)
        pool.page_index = PhysicalPageIndex(original_page_ids=ids[:page_end], physical_offsets=offs[:page_end],
                                            lengths=lens[:page_end], global_token_indices=g[:token_end],
                                            logical_positions=l[:token_end])

    def append_int2_pages(self, pool: "PrecisionPool", global_indices: torch.Tensor,
                          logical_positions: torch.Tensor, page_size: int) -> None:
        self._append_pages(pool, global_indices, logical_positions, page_size, "int2")

    def append_int4_pages(self, pool: "PrecisionPool", global_indices: torch.Tensor,
                          logical_positions: torch.Tensor, page_size: int) -> None:
        self._append_pages(pool, global_indices, logical_positions, page_size, "int4")


# ------------------------------------------------------------------------ BF16 K rows
@dataclass
class BF16KeyArena:
    """Key rows kept in the model dtype (bf16 or fp16) in physical pool order (FP, INT4, INT2) with
    append capacity.

    Backs the matched-FP cache and the v_fourq_k_bf16 variant: the pools' ``fp_k`` are views of
    ``rows`` (precision_pool.py:834-906 keeps one bf16 K tensor per pool; one arena serves the
    decode kernel, which reads K rows by physical position).
    """
    rows: torch.Tensor              # bf16 / fp16 [H, capacity, D]
    active_length: int
    capacity: int
    segment_offsets: tuple[int, int, int]

    def view(self, start: int, length: int) -> torch.Tensor:
        return self.rows[:, start : start + length]

    def append_block(self, key_block: torch.Tensor) -> None:
        n = int(key_block.shape[1])
        if self.active_length + n > self.capacity:
            grown = torch.zeros((self.rows.shape[0], _round_up(self.active_length + n + 128, 128), self.rows.shape[2]),
                                device=self.rows.device, dtype=self.rows.dtype)
            grown[:, : self.active_length].copy_(self.rows[:, : self.active_length])
            self.rows, self.capacity = grown, int(grown.shape[1])
        self.rows[:, self.active_length : self.active_length + n].copy_(key_block)
        self.active_length += n


# ------------------------------------------------------------------------ compact INT4 K
@dataclass
class CompactInt4KeyArena:
    """Per-channel affine INT4 K for all FP/INT4/INT2 tokens in physical order."""

    packed: torch.Tensor          # u8  [H, capacity, D/2]
    scale: torch.Tensor           # f16 [H, capacity/SB, D]
    zero_point: torch.Tensor      # u8  [H, capacity/SB, D]
    active_length: int
    capacity: int
    segment_offsets: tuple[int, int, int]
    original_dtype: torch.dtype
    superblock_size: int = 128
    bit_width: int = 4
    # u32 [H, capacity/SB, 128]: per superblock, the fp16 scale pairs and -(1024 + zero) pairs in
    # the channel order of the decode kernel's QK MFMA (derived from scale/zero by the packer)
    kernel_operands: torch.Tensor | None = None

    def __post_init__(self) -> None:
        if self.packed.ndim != 3 or self.packed.dtype != torch.uint8:
            raise ValueError("compact INT4 K storage must be uint8 [H,capacity,D/2]")
        h, capacity, d2 = map(int, self.packed.shape)
        if self.superblock_size not in (32, 64, 128):
            raise ValueError("compact INT4 K superblock must be 32, 64, or 128 tokens")
        blocks = -(-capacity // self.superblock_size)
        if capacity != self.capacity or not 0 <= self.active_length <= capacity:
            raise ValueError("compact INT4 K active length/capacity is invalid")
        if tuple(self.scale.shape) != (h, blocks, d2 * 2):
            raise ValueError("compact INT4 K scale shape is invalid")
        if self.zero_point.shape != self.scale.shape:
            raise ValueError("compact INT4 K zero-point shape is invalid")
        if self.scale.dtype != torch.float16 or self.zero_point.dtype != torch.uint8:
            raise ValueError("compact INT4 K metadata dtypes are invalid")
        if tuple(sorted(self.segment_offsets)) != tuple(self.segment_offsets):
            raise ValueError("compact INT4 K segment offsets must be monotonic")
        if self.kernel_operands is not None and (tuple(self.kernel_operands.shape) != (h, blocks, 128)
                                                 or self.kernel_operands.dtype != torch.int32):
            raise ValueError("compact INT4 K kernel operands must be int32 [H,blocks,128]")

    @property
    def head_count(self) -> int:
        return int(self.packed.shape[0])

    @property
    def head_dim(self) -> int:
        return int(self.packed.shape[2]) * 2

    @property
    def superblock_count(self) -> int:
        return int(self.scale.shape[1])

    @property
    def nbytes(self) -> int:
        return sum(_nbytes(t) for t in self.allocation_tensors())

    @property
    def active_nbytes(self) -> int:
        if self.active_length <= 0:
            return 0
        blocks = -(-self.active_length // self.superblock_size)
        per_block = self.head_count * blocks * self.head_dim
        return int(self.head_count * self.active_length * self.head_dim // 2
                   + per_block * self.scale.element_size() + per_block * self.zero_point.element_size())

    def allocation_tensors(self):
        if self.kernel_operands is None:
            return self.packed, self.scale, self.zero_point
        return self.packed, self.scale, self.zero_point, self.kernel_operands

    def dequantize_range(self, start: int, length: int) -> torch.Tensor:
        """fp32 (code - z) * s of arena positions [start, start+length) (inspection only)."""
        start, length = int(start), int(length)
        if start < 0 or length < 0 or start + length > self.active_length:
            raise ValueError("compact INT4 K range is outside the active payload")
        payload = self.packed[:, start : start + length]
        codes = torch.stack((payload & 15, payload >> 4), dim=-1).reshape(self.head_count, length, self.head_dim)
        blocks = torch.arange(start, start + length, device=payload.device) // self.superblock_size
        s = self.scale.index_select(1, blocks).float()
        z = self.zero_point.index_select(1, blocks).float()
        return (codes.float() - z) * s

    def dequantize(self) -> torch.Tensor:
        return self.dequantize_range(0, self.active_length)

    def append_superblock(self, key_block: torch.Tensor, *, source_tokens: int | None = None) -> int:
        """Flush 128 tokens: re-quantise the partial tail superblock together with them.

        ``key_block`` may be a [H, 128, D] view whose rows are strided by ``source_tokens``
        (the Recent-FP ring passes its first 128 slots without a copy).
        """
        if tuple(key_block.shape) != (self.head_count, 128, self.head_dim):
            raise ValueError("compact INT4 K flush requires 128 matching tokens")
        if self.active_length + 128 > self.capacity:
            raise RuntimeError("compact INT4 K capacity exhausted")
        _lib.require_device(key_block, "compact INT4 K flush block")
        rows = int(source_tokens) if source_tokens is not None else 128
        if key_block.stride() != (rows * self.head_dim, self.head_dim, 1):
            raise ValueError("compact INT4 K flush block must have contiguous rows")
        prefix = self.active_length // self.superblock_size * self.superblock_size
        tail = self.active_length - prefix
        _lib.call("r2o_pack_int4_k", _lib.ptr(key_block), _lib.dtype_code(key_block.dtype), self.head_count, rows,
                  None, 128, tail, prefix, _lib.ptr(self.packed), _lib.ptr(self.scale), _lib.ptr(self.zero_point),
                  _lib.ptr(self.kernel_operands), self.capacity, self.superblock_count, self.superblock_size,
                  _lib.stream_of(key_block.device))
        self.active_length += 128
        return tail


def build_compact_int4_key_arena(key: torch.Tensor, segment_token_indices, *, append_capacity: int = 0,
                                 superblock_size: int = 128) -> CompactInt4KeyArena:
    if key.ndim != 3 or not torch.is_floating_point(key) or int(key.shape[2]) % 2:
        raise ValueError("key must be floating [H,S,D] with even D")
    if superblock_size not in (32, 64, 128):
        raise ValueError("compact per-channel INT4 K superblock must be 32, 64, or 128 tokens")
    _lib.require_device(key, "key")
    lengths = tuple(int(ix.numel()) for ix in segment_token_indices)
    offsets = (0, lengths[0], lengths[0] + lengths[1])
    active = sum(lengths)
    capacity = max(128, _round_up(active + int(append_capacity), 128))
    h, s, d = map(int, key.shape)
    blocks = capacity // superblock_size
    dev = key.device
    arena = CompactInt4KeyArena(
        packed=torch.zeros((h, capacity, d // 2), device=dev, dtype=torch.uint8),
        scale=torch.zeros((h, blocks, d), device=dev, dtype=torch.float16),
        zero_point=torch.zeros((h, blocks, d), device=dev, dtype=torch.uint8),
        active_length=active, capacity=capacity, segment_offsets=offsets,
        original_dtype=key.dtype, superblock_size=superblock_size,
        kernel_operands=torch.zeros((h, blocks, 128), device=dev, dtype=torch.int32),
    )
    if active:
        key = key.contiguous()
        ordered = torch.cat([ix.to(device=dev, dtype=torch.long) for ix in segment_token_indices]).contiguous()
        _lib.call("r2o_pack_int4_k", _lib.ptr(key), _lib.dtype_code(key.dtype), h, s, _lib.ptr(ordered), active,
                  0, 0, _lib.ptr(arena.packed), _lib.ptr(arena.scale), _lib.ptr(arena.zero_point),
                  _lib.ptr(arena.kernel_operands), capacity, blocks, superblock_size, _lib.stream_of(dev))
    return arena


@dataclass
class CompactInt2KeyArena:
    """Per-channel affine INT2 K (OScaR form) for all FP/INT4/INT2 tokens in physical order
    (compact_int2_key.py:14-122): dequant = code * scale + offset, the offset kept in the
    ``zero_point`` field as fp16 like the reference's."""

    packed: torch.Tensor          # u8  [H, capacity, D/4]
    scale: torch.Tensor           # f16 [H, capacity/SB, D]
    zero_point: torch.Tensor      # f16 [H, capacity/SB, D] (the offset)
    active_length: int
    capacity: int
    segment_offsets: tuple[int, int, int]
    original_dtype: torch.dtype
    superblock_size: int = 128
    bit_width: int = 2
    # u32 [H, capacity/SB, 128]: per superblock, the (scale / 4^u) pairs and offset pairs in the
    # channel order of the decode kernel's INT2-K QK MFMA (derived by the packer)
    kernel_operands: torch.Tensor | None = None

    def __post_init__(self) -> None:
        if self.packed.ndim != 3 or self.packed.dtype != torch.uint8:
            raise ValueError("compact INT2 K storage must be uint8 [H,capacity,D/4]")
        h, capacity, d4 = map(int, self.packed.shape)
        if self.superblock_size not in (32, 64, 128):
            raise ValueError("per-channel INT2 K block size must be 32, 64, or 128")
        blocks = -(-capacity // self.superblock_size)
        if capacity != self.capacity or not 0 <= self.active_length <= capacity:
            raise ValueError("compact INT2 K active length/capacity is invalid")
        if tuple(self.scale.shape) != (h, blocks, d4 * 4) or self.zero_point.shape != self.scale.shape:
            raise ValueError("compact INT2 K metadata shape is invalid")
        if self.scale.dtype != torch.float16 or self.zero_point.dtype != torch.float16:
            raise ValueError("compact INT2 K metadata dtypes are invalid")
        if tuple(sorted(self.segment_offsets)) != tuple(self.segment_offsets):
            raise ValueError("compact INT2 K segment offsets must be monotonic")
        if self.kernel_operands is not None and (tuple(self.kernel_operands.shape) != (h, blocks, 128)
                                                 or self.kernel_operands.dtype != torch.int32):
            raise ValueError("compact INT2 K kernel operands must be int32 [H,blocks,128]")

    @property
    def head_count(self) -> int:
        return int(self.packed.shape[0])

    @property
    def head_dim(self) -> int:
        return int(self.packed.shape[2]) * 4

    @property
    def superblock_count(self) -> int:
        return int(self.scale.shape[1])

    @property
    def nbytes(self) -> int:
        return sum(_nbytes(t) for t in self.allocation_tensors())

    @property
    def active_nbytes(self) -> int:
        if self.active_length <= 0:
            return 0
        blocks = -(-self.active_length // self.superblock_size)
        per_block = self.head_count * blocks * self.head_dim
        return int(self.head_count * self.active_length * (self.head_dim // 4)
                   + per_block * self.scale.element_size() + per_block * self.zero_point.element_size())

    def allocation_tensors(self):
        if self.kernel_operands is None:
            return self.packed, self.scale, self.zero_point
        return self.packed, self.scale, self.zero_point, self.kernel_operands

    def dequantize_range(self, start: int, length: int) -> torch.Tensor:
        """fp32 code * s + o of arena positions [start, start+length) (inspection only)."""
        start, length = int(start), int(length)
        if start < 0 or length < 0 or start + length > self.active_length:
            raise ValueError("compact INT2 K range is outside the active payload")
        payload = self.packed[:, start : start + length]
        codes = torch.stack([(payload >> (2 * i)) & 3 for i in range(4)], dim=-1)
        codes = codes.reshape(self.head_count, length, self.head_dim)
        blocks = torch.arange(start, start + length, device=payload.device) // self.superblock_size
        return codes.float() * self.scale.index_select(1, blocks).float() \
            + self.zero_point.index_select(1, blocks).float()

    def dequantize(self) -> torch.Tensor:
        return self.dequantize_range(0, self.active_length)

    def append_superblock(self, key_block: torch.Tensor, *, source_tokens: int | None = None) -> int:
        """Flush 128 tokens: re-quantise the partial tail superblock together with them
        (compact_int2_key.py:110-122).  ``key_block`` as in ``CompactInt4KeyArena.append_superblock``."""
        if tuple(key_block.shape) != (self.head_count, 128, self.head_dim):
            raise ValueError("compact INT2 K flush requires 128 matching tokens")
        if self.active_length + 128 > self.capacity:
            raise RuntimeError("compact INT2 K capacity exhausted")
        _lib.require_device(key_block, "compact INT2 K flush block")
        rows = int(source_tokens) if source_tokens is not None else 128
        if key_block.stride() != (rows * self.head_dim, self.head_dim, 1):
            raise ValueError("compact INT2 K flush block must have contiguous rows")
        prefix = self.active_length // self.superblock_size * self.superblock_size
        tail = self.active_length - prefix
        _lib.call("r2o_pack_int2_k", _lib.ptr(key_block), _lib.dtype_code(key_block.dtype), self.head_count, rows,
                  None, 128, tail, prefix, _lib.ptr(self.packed), _lib.ptr(self.scale), _lib.ptr(self.zero_point),
                  _lib.ptr(self.kernel_operands), self.capacity, self.superblock_count, self.superblock_size,
                  _lib.stream_of(key_block.device))
        self.active_length += 128
        return tail


def build_compact_int2_key_arena(key: torch.Tensor, segment_token_indices, *, append_capacity: int = 0,
                                 superblock_size: int = 128) -> CompactInt2KeyArena:
    """``build_compact_int2_key_arena`` (compact_int2_key.py:125-153), packed on the GPU."""
    if key.ndim != 3 or not torch.is_floating_point(key) or int(key.shape[2]) % 4:
        raise ValueError("key must be floating [H,S,D] with D divisible by four")
    if superblock_size not in (32, 64, 128):
        raise ValueError("per-channel INT2 K block size must be 32, 64, or 128")
    _lib.require_device(key, "key")
    lengths = tuple(int(ix.numel()) for ix in segment_token_indices)
    offsets = (0, lengths[0], lengths[0] + lengths[1])
    active = sum(lengths)
    capacity = max(128, _round_up(active + int(append_capacity), 128))
    h, s, d = map(int, key.shape)
    blocks = capacity // superblock_size
    dev = key.device
    arena = CompactInt2KeyArena(
        packed=torch.zeros((h, capacity, d // 4), device=dev, dtype=torch.uint8),
        scale=torch.zeros((h, blocks, d), device=dev, dtype=torch.float16),
        zero_point=torch.zeros((h, blocks, d), device=dev, dtype=torch.float16),
        active_length=active, capacity=capacity, segment_offsets=offsets,
        original_dtype=key.dtype, superblock_size=superblock_size,
        kernel_operands=torch.zeros((h, blocks, 128), device=dev, dtype=torch.int32),
    )
    if active:
        key = key.contiguous()
        ordered = torch.cat([ix.to(device=dev, dtype=torch.long) for ix in segment_token_indices]).contiguous()
        _lib.call("r2o_pack_int2_k", _lib.ptr(key), _lib.dtype_code(key.dtype), h, s, _lib.ptr(ordered), active,
                  0, 0, _lib.ptr(arena.packed), _lib.ptr(arena.scale), _lib.ptr(arena.zero_point),
                  _lib.ptr(arena.kernel_operands), capacity, blocks, superblock_size, _lib.stream_of(dev))
    return arena


# ---------------------------------------------------------------------- INT4-V pool payload
@dataclass
class PackedTensor:
    packed: torch.Tensor
    scale: torch.Tensor
    zero_point: torch.Tensor | None
    num_bits: int
    original_shape: tuple[int, ...]
    dtype: torch.dtype
    quant_scheme: str
    pack_metadata: dict[str, Any]
    quant_metadata: dict[str, Any] = field(default_factory=dict)

    @property
    def nbytes(self) -> int:
        return _nbytes(self.packed) + _nbytes(self.scale) + _nbytes(self.zero_point)

    def dequantize(self) -> torch.Tensor:
        """Per-token INT4 dequantised and rounded to the input dtype (packed_kv_layout.py:30-32)."""
        h, s, d = self.original_shape
        p = self.packed.reshape(h, s, d // 2)
        lo = (p & 15).to(torch.int16)
        hi = (p >> 4).to(torch.int16)
        codes = torch.stack((torch.where(lo >= 8, lo - 16, lo), torch.where(hi >= 8, hi - 16, hi)), -1)
        return (codes.reshape(h, s, d).float() * self.scale.float()).to(self.dtype)


def fused_gather_pack_int4_value(value: torch.Tensor, token_indices: torch.Tensor) -> PackedTensor:
    if value.ndim != 3 or int(value.shape[2]) != 128:
        raise ValueError("INT4 V source must be [Hkv,S,128]")
    if token_indices.ndim != 1 or token_indices.device != value.device:
        raise ValueError("INT4 V token indices must be rank-1 on the V device")
    _lib.require_device(value, "value")
    h, s, d = map(int, value.shape)
    n = int(token_indices.numel())
    packed = torch.empty((h, n, d // 2), device=value.device, dtype=torch.uint8)
    scale = torch.empty((h, n, 1), device=value.device, dtype=torch.float32)
    if n:
        value = value.contiguous()
        idx = token_indices.to(torch.long).contiguous()
        _lib.call("r2o_pack_int4_v", _lib.ptr(value), _lib.dtype_code(value.dtype), h, s, _lib.ptr(idx), n, 0,
                  _lib.ptr(packed), _lib.ptr(scale), n, _lib.stream_of(value.device))
    return PackedTensor(packed=packed.flatten(), scale=scale, zero_point=None, num_bits=4, original_shape=(h, n, d),
                        dtype=value.dtype, quant_scheme="per_token",
                        pack_metadata={"pack_axis": "flatten_c_order", "fused_gather": True},
                        quant_metadata={"dim": 2, "fused_gather": True})


# ------------------------------------------------------------------------ compact INT4 V
@dataclass
class CompactInt4ValueArena:
    """Per-token symmetric INT4 V with room for generated flushes (fused_value_pack.py:196-299): the
    static INT4 pool's tokens first, then each flushed block, packed in place by r2o_pack_int4_v."""

    packed: torch.Tensor          # u8  [H, capacity, D/2]
    scale: torch.Tensor           # f32 [H, capacity, 1]
    active_length: int
    capacity: int
    original_dtype: torch.dtype
    num_bits: int = 4
    quant_scheme: str = "per_token"
    zero_point: None = None

    def __post_init__(self) -> None:
        if self.packed.ndim != 3 or self.packed.dtype != torch.uint8:
            raise ValueError("compact INT4 V packed storage must be uint8 [H,capacity,D/2]")
        h, capacity, _ = map(int, self.packed.shape)
        if capacity != self.capacity or not 0 <= self.active_length <= capacity:
            raise ValueError("compact INT4 V active length/capacity is invalid")
        if tuple(self.scale.shape) != (h, capacity, 1) or self.scale.dtype != torch.float32:
            raise ValueError("compact INT4 V scale storage must be float32 [H,capacity,1]")

    @property
    def original_shape(self) -> tuple[int, int, int]:
        return int(self.packed.shape[0]), int(self.active_length), int(self.packed.shape[2]) * 2

    @property
    def nbytes(self) -> int:
        return sum(_nbytes(t) for t in self.allocation_tensors())

    @property
    def active_nbytes(self) -> int:
        h, _, d2 = map(int, self.packed.shape)
        return int(h * self.active_length * (d2 + self.scale.element_size()))

    def allocation_tensors(self):
        return self.packed, self.scale

    def dequantize_range(self, start: int, length: int) -> torch.Tensor:
        """fp32 code * scale (not rounded to the input dtype, unlike ``PackedTensor.dequantize``)."""
        start, length = int(start), int(length)
        if start < 0 or length < 0 or start + length > self.active_length:
            raise ValueError("compact INT4 V dequantization range is outside active storage")
        h, _, d2 = map(int, self.packed.shape)
        p = self.packed[:, start:start + length]
        lo = (p & 15).to(torch.int16)
        hi = (p >> 4).to(torch.int16)
        codes = torch.stack((torch.where(lo >= 8, lo - 16, lo), torch.where(hi >= 8, hi - 16, hi)), -1)
        return codes.reshape(h, length, d2 * 2).float() * self.scale[:, start:start + length]

    def dequantize(self) -> torch.Tensor:
        return self.dequantize_range(0, self.active_length)

    def append_block(self, value_block: torch.Tensor, *, source_tokens: int | None = None) -> None:
        """Pack ``value_block`` [H, n, D] (rows of ``source_tokens`` per head, default n) after the
        active tokens."""
        h, _, d = self.original_shape
        if value_block.ndim != 3 or int(value_block.shape[0]) != h or int(value_block.shape[2]) != d \
                or int(value_block.shape[1]) <= 0:
            raise ValueError("compact INT4 V append must contain matching tokens")
        n = int(value_block.shape[1])
        dst = self.active_length
        if dst + n > self.capacity:
            raise RuntimeError(f"compact INT4 V capacity exhausted: need {dst + n}, have {self.capacity}")
        _lib.require_device(value_block, "compact INT4 V append block")
        rows = int(source_tokens) if source_tokens is not None else n
        if value_block.stride() != (rows * d, d, 1):
            raise ValueError("compact INT4 V append block must have contiguous rows")
        _lib.call("r2o_pack_int4_v", _lib.ptr(value_block), _lib.dtype_code(value_block.dtype), h, rows, None, n, dst,
                  _lib.ptr(self.packed), _lib.ptr(self.scale), self.capacity, _lib.stream_of(value_block.device))
        self.active_length += n


def build_compact_int4_value_arena(value: torch.Tensor, token_indices: torch.Tensor, *,
                                   append_capacity: int = 0) -> CompactInt4ValueArena:
    """INT4 V of ``value[:, token_indices]`` with ``append_capacity`` more tokens of room
    (fused_value_pack.py:302-330: capacity = max(1, tokens + append_capacity))."""
    if value.ndim != 3 or int(value.shape[2]) != 128:
        raise ValueError("compact INT4 V source must be [Hkv,S,128]")
    if append_capacity < 0:
        raise ValueError("append_capacity must be non-negative")
    _lib.require_device(value, "value")
    n = int(token_indices.numel())
    capacity = max(1, n + int(append_capacity))
    h, s, d = map(int, value.shape)
    dev = value.device
    arena = CompactInt4ValueArena(packed=torch.zeros((h, capacity, d // 2), device=dev, dtype=torch.uint8),
                                  scale=torch.zeros((h, capacity, 1), device=dev, dtype=torch.float32),
                                  active_length=n, capacity=capacity, original_dtype=value.dtype)
    if n:
        value = value.contiguous()
        idx = token_indices.to(device=dev, dtype=torch.long).contiguous()
        _lib.call("r2o_pack_int4_v", _lib.ptr(value), _lib.dtype_code(value.dtype), h, s, _lib.ptr(idx), n, 0,
                  _lib.ptr(arena.packed), _lib.ptr(arena.scale), capacity, _lib.stream_of(dev))
    return arena


# ------------------------------------------------------------------------ compact INT2 V
@dataclass
class CompactInt2ValueArena:
    """Per-token-group affine INT2 V with in-place generated flushes."""

    packed: torch.Tensor          # u8  [H, capacity, D/4]
    scale: torch.Tensor           # f16 [H, capacity, D/G, 1]
    zero_point: torch.Tensor      # u8  [H, capacity, D/G, 1]
    active_length: int
    capacity: int
    original_dtype: torch.dtype
    group_size: int = 32
    axis: str = "per_token_group"
    superblock_size: int = 128

    def __post_init__(self) -> None:
        if self.packed.ndim != 3 or self.packed.dtype != torch.uint8:
            raise ValueError("compact INT2 V packed storage must be uint8 [H,capacity,D/4]")
        h, capacity, d4 = map(int, self.packed.shape)
        groups = d4 * 4 // self.group_size
        if capacity != self.capacity or not 0 <= self.active_length <= capacity:
            raise ValueError("compact INT2 V active length/capacity is invalid")
        if tuple(self.scale.shape) != (h, capacity, groups, 1):
            raise ValueError("compact INT2 V scale shape is invalid")
        if self.zero_point.shape != self.scale.shape:
            raise ValueError("compact INT2 V zero-point shape is invalid")
        if self.scale.dtype != torch.float16 or self.zero_point.dtype != torch.uint8:
            raise ValueError("compact INT2 V metadata dtypes are invalid")

    @property
    def original_shape(self) -> tuple[int, int, int]:
        return int(self.packed.shape[0]), int(self.active_length), int(self.packed.shape[2]) * 4

    @property
    def nbytes(self) -> int:
        return sum(_nbytes(t) for t in self.allocation_tensors())

    @property
    def active_nbytes(self) -> int:
        h, _, d4 = map(int, self.packed.shape)
        groups = d4 * 4 // self.group_size
        return int(h * self.active_length * (d4 + groups * (self.scale.element_size() + self.zero_point.element_size())))

    def allocation_tensors(self):
        return self.packed, self.scale, self.zero_point

    def dequantize_range(self, start: int, length: int) -> torch.Tensor:
        start, length = int(start), int(length)
        if start < 0 or length < 0 or start + length > self.active_length:
            raise ValueError("compact INT2 V dequantization range is outside active storage")
        h, _, d4 = map(int, self.packed.shape)
        d = d4 * 4
        p = self.packed[:, start : start + length]
        codes = torch.stack([(p >> (2 * k)) & 3 for k in range(4)], dim=-1).reshape(h, length, d)
        grouped = codes.reshape(h, length, d // self.group_size, self.group_size).float()
        s = self.scale[:, start : start + length].float()
        z = self.zero_point[:, start : start + length].float()
        return ((grouped - z) * s).reshape(h, length, d)

    def dequantize(self) -> torch.Tensor:
        return self.dequantize_range(0, self.active_length)

    def append_superblock(self, value_block: torch.Tensor, *, source_tokens: int | None = None) -> None:
        h, _, d = self.original_shape
        if value_block.ndim != 3 or int(value_block.shape[0]) != h or int(value_block.shape[2]) != d \
                or int(value_block.shape[1]) <= 0:
            raise ValueError("compact INT2 V flush must contain matching tokens")
        n = int(value_block.shape[1])
        dst = self.active_length
        if dst + n > self.capacity:
            raise RuntimeError(f"compact INT2 V capacity exhausted: need {dst + n}, have {self.capacity}")
        _lib.require_device(value_block, "compact INT2 V flush block")
        rows = int(source_tokens) if source_tokens is not None else n
        if value_block.stride() != (rows * d, d, 1):
            raise ValueError("compact INT2 V flush block must have contiguous rows")
        _lib.call("r2o_pack_int2_v", _lib.ptr(value_block), _lib.dtype_code(value_block.dtype), h, rows, None, n,
                  dst, self.group_size, _lib.ptr(self.packed), _lib.ptr(self.scale), _lib.ptr(self.zero_point),
                  self.capacity, _lib.stream_of(value_block.device))
        self.active_length += n


def build_compact_int2_value_arena(value: torch.Tensor, token_indices: torch.Tensor, *, append_capacity: int = 0,
                                   group_size: int = 32) -> CompactInt2ValueArena:
    if value.ndim != 3 or int(value.shape[2]) != 128:
        raise ValueError("compact INT2 V source must be [Hkv,S,128]")
    if group_size not in (32, 64, 128):
        raise ValueError("compact INT2 V requires group_size 32, 64, or 128")
    if append_capacity < 0:
        raise ValueError("append_capacity must be non-negative")
    _lib.require_device(value, "value")
    n = int(token_indices.numel())
    capacity = max(128, _round_up(n + int(append_capacity), 128))
    h, s, d = map(int, value.shape)
    groups = d // group_size
    dev = value.device
    arena = CompactInt2ValueArena(
        packed=torch.zeros((h, capacity, d // 4), device=dev, dtype=torch.uint8),
        scale=torch.zeros((h, capacity, groups, 1), device=dev, dtype=torch.float16),
        zero_point=torch.zeros((h, capacity, groups, 1), device=dev, dtype=torch.uint8),
        active_length=n, capacity=capacity, original_dtype=value.dtype, group_size=group_size,
    )
    if n:
        value = value.contiguous()
        idx = token_indices.to(device=dev, dtype=torch.long).contiguous()
        _lib.call("r2o_pack_int2_v", _lib.ptr(value), _lib.dtype_code(value.dtype), h, s, _lib.ptr(idx), n, 0,
                  group_size, _lib.ptr(arena.packed), _lib.ptr(arena.scale), _lib.ptr(arena.zero_point), capacity,
                  _lib.stream_of(dev))
    return arena


# ----------------------------------------------------------------------------- pools/cache
@dataclass
class PrecisionPool:
    name: str
    page_index: PhysicalPageIndex
    fp_k: torch.Tensor | None = None
    fp_v: torch.Tensor | None = None
    packed_k: Any = None
    packed_v: Any = None
    active_length: int | None = None
    capacity: int = 0
    length_device: torch.Tensor | None = None
    global_index_buffer: torch.Tensor | None = None
    logical_position_buffer: torch.Tensor | None = None

    @property
    def token_count(self) -> int:
        if self.active_length is not None:
            return int(self.active_length)
        return int(self.page_index.global_token_indices.numel())

    @property
    def payload_bytes(self) -> int:
        return int(_nbytes(self.fp_k) + _nbytes(self.fp_v)
                   + (0 if self.packed_k is None else self.packed_k.nbytes)
                   + (0 if self.packed_v is None else self.packed_v.nbytes))

    @property
    def active_payload_bytes(self) -> int:
        n = self.token_count

        def fp(t):
            if t is None:
                return 0
            if self.active_length is None:
                return _nbytes(t)
            return int(t.shape[0]) * int(t.shape[2]) * n * t.element_size()

        def packed(x):
            return 0 if x is None else int(getattr(x, "active_nbytes", x.nbytes))

        return int(fp(self.fp_k) + fp(self.fp_v) + packed(self.packed_k) + packed(self.packed_v))


@dataclass
class ThreePrecisionCache:
    fp_pool: PrecisionPool
    int4_pool: PrecisionPool
    int2_pool: PrecisionPool
    recent_fp_pool: PrecisionPool
    evicted_global_indices: torch.Tensor
    page_size: int
    quantization_superblock: int
    matched_fp: bool
    cache_variant: str
    compact_key: CompactInt4KeyArena | CompactInt2KeyArena | None = None
    compact_value: CompactInt2ValueArena | None = None
    compact_int4_value: CompactInt4ValueArena | None = None  # INT4 pool's V when generated values are INT4
    metadata_arena: CompactMetadataArena | None = None
    recent_flush_size: int = 128
    generated_value_precision: str = "int2"
    static_int4_tokens: int = 0
    generated_k_offset: int = 0
    bf16_key: BF16KeyArena | None = None   # K rows of the matched-FP / v_fourq_k_bf16 caches

    @property
    def pools(self):
        return (self.fp_pool, self.int4_pool, self.int2_pool, self.recent_fp_pool)

    @property
    def payload_bytes(self) -> int:
        total = sum(p.payload_bytes for p in self.pools) + (0 if self.compact_key is None else self.compact_key.nbytes)
        if self.bf16_key is not None:  # the history pools' fp_k are views of one arena: count it once
            total += _nbytes(self.bf16_key.rows) - sum(_nbytes(p.fp_k) for p in self.pools[:3])
        return total

    @property
    def survivor_count(self) -> int:
        return sum(p.token_count for p in self.pools)

    @property
    def uniform_int4_key(self) -> bool:
        return self.cache_variant == "v_fourq_k_int4_compact" and not self.matched_fp

    @property
    def uniform_int2_key(self) -> bool:
        return self.cache_variant == "v_fourq_k_int2_compact" and not self.matched_fp

    @property
    def full_precision_key(self) -> bool:
        return self.cache_variant == "v_fourq_k_bf16" or self.matched_fp

    @property
    def compact_int4_key(self) -> bool:
        return self.compact_key is not None and self.compact_key.bit_width == 4

    @property
    def compact_int2_key(self) -> bool:
        return self.compact_key is not None and self.compact_key.bit_width == 2

    @property
    def compact_int2_value(self) -> bool:
        return self.compact_value is not None

    @property
    def storage_bytes(self) -> int:
        return precision_cache_storage_breakdown(self)["persistent_cache_bytes"]


def _pool_metadata(pool: PrecisionPool):
    pi = pool.page_index
    return (pi.original_page_ids, pi.physical_offsets, pi.lengths, pi.global_token_indices, pi.logical_positions,
            pool.length_device, pool.global_index_buffer, pool.logical_position_buffer)


def precision_cache_storage_breakdown(cache: ThreePrecisionCache) -> dict[str, int]:
    """Allocated bytes, counting each storage once (precision_pool.py:296-344)."""
    payload: list[torch.Tensor] = []
    if cache.compact_key is not None:
        payload.extend(cache.compact_key.allocation_tensors())
    for pool in cache.pools:
        payload.extend(t for t in (pool.fp_k, pool.fp_v) if t is not None)
        for pk in (pool.packed_k, pool.packed_v):
            if pk is not None:
                payload.extend(t for t in (pk.packed, pk.scale, pk.zero_point) if t is not None)
    seen: set[int] = set()
    pay = 0
    for t in payload:
        key = t.untyped_storage().data_ptr()
        if key not in seen:
            seen.add(key)
            pay += int(t.untyped_storage().nbytes())
    meta_seen: set[int] = set()
    meta = 0
    arena = [] if cache.metadata_arena is None else [cache.metadata_arena.storage]
    for t in [cache.evicted_global_indices] + arena + [m for p in cache.pools for m in _pool_metadata(p)]:
        if t is None:
            continue
        key = t.untyped_storage().data_ptr()
        if key in seen or key in meta_seen:
            continue
        meta_seen.add(key)
        meta += int(t.untyped_storage().nbytes())
    return {"kv_payload_bytes": pay, "kv_payload_allocation_count": len(seen), "metadata_bytes": meta,
            "metadata_allocation_count": len(meta_seen), "persistent_cache_bytes": pay + meta,
            "persistent_allocation_count": len(seen) + len(meta_seen)}


def precision_cache_active_storage_breakdown(cache: ThreePrecisionCache) -> dict[str, int]:
    """Populated payload and the metadata that addresses it (precision_pool.py:347-397)."""
    payload = sum(p.active_payload_bytes for p in cache.pools)
    if cache.compact_key is not None:
        payload += cache.compact_key.active_nbytes
    meta = _nbytes(cache.evicted_global_indices)
    fields = 0
    for pool in cache.pools:
        n = pool.token_count
        pages = int(pool.page_index.lengths.numel()) if pool.active_length is None else -(-n // cache.page_size)
        pi = pool.page_index
        meta += sum(pages * t.element_size() for t in (pi.original_page_ids, pi.physical_offsets, pi.lengths))
        meta += sum(n * t.element_size() for t in (pi.global_token_indices, pi.logical_positions))
        fields += 3 * (pages > 0) + 2 * (n > 0)
        if pool.length_device is not None:
            meta += pool.length_device.element_size()
            fields += 1
    return {"kv_payload_bytes": int(payload), "kv_payload_allocation_count": 0, "metadata_bytes": int(meta),
            "metadata_allocation_count": int(fields), "persistent_cache_bytes": int(payload + meta),
            "persistent_allocation_count": int(fields)}


class _TierTable(NamedTuple):
    """Host page table in tier order FP(+protected, recent) < INT4 < INT2 < evicted."""
    pages: np.ndarray        # plan page ids, tier order
    offsets: np.ndarray      # offset of each page inside its tier's pool
    lengths: np.ndarray      # tokens per page
    shift: np.ndarray        # plan token index minus position in the tier-ordered concatenation
    first_page: np.ndarray   # [5] index of each tier's first page (and the end)
    tier_tokens: np.ndarray  # [4] tokens per tier


# tier of each PageClass value: FP (+protected, recent) 0, INT4 1, INT2 2, evicted 3
_TIER_OF_CLASS = np.zeros(max(int(c) for c in PageClass) + 1, dtype=np.int64)
for _c, _t in ((PageClass.EVICTED_PAGE, 3), (PageClass.FP_PAGE, 0), (PageClass.PROTECTED_FP_PAGE, 0),
               (PageClass.RECENT_FP_PAGE, 0), (PageClass.INT4_PAGE, 1), (PageClass.INT2_PAGE, 2)):
    _TIER_OF_CLASS[int(_c)] = _t


def _tier_page_table(plan: LayerCompressionPlan) -> _TierTable:
    """Pages stably sorted by tier, each keeping its token order (precision_pool.py:611-669).

    The page table is small: it is sorted on the host, from the plan's host copy or one copy from
    the device when the plan lives there.
    """
    table = plan.host_page_table
    if table is None:
        table = torch.stack((plan.page_classes.detach().to(torch.long), plan.page_offsets.detach().to(torch.long),
                             plan.page_lengths.detach().to(torch.long))).to("cpu")
    classes, starts, lens = table.numpy()
    if classes.size and (int(classes.min()) < 0 or int(classes.max()) >= _TIER_OF_CLASS.size):
        raise ValueError("page_classes holds a value that is not a PageClass")
    cat = _TIER_OF_CLASS[classes]
    groups = [np.flatnonzero(cat == t) for t in range(4)]
    counts = np.array([g.size for g in groups], dtype=np.int64)
    pages = np.concatenate(groups)
    first_page = np.concatenate(([0], np.cumsum(counts)))
    pl = lens[pages]
    end = np.cumsum(pl)
    glob_off = end - pl  # offset of each page in the tier-ordered concatenation
    bounds = np.concatenate(([0], end))[first_page]
    return _TierTable(pages=pages, offsets=glob_off - np.repeat(bounds[:-1], counts), lengths=pl,
                      shift=starts[pages] - glob_off, first_page=first_page, tier_tokens=np.diff(bounds))


def _expand_tier_tokens(tab: _TierTable, device) -> torch.Tensor:
    """Plan token indices of every tier, concatenated in tier order, on ``device``: token j of the
    concatenation is start(page) + (j - offset of the page in it), one expansion for all tiers."""
    dev = torch.device(device)
    n_tok = int(tab.tier_tokens.sum())
    if not n_tok:
        return torch.zeros(0, dtype=torch.long, device=dev)
    d = torch.from_numpy(np.stack((tab.shift, tab.lengths)))
    if dev.type != "cpu":  # pinned staging: a copy from pageable memory would wait for the stream's earlier work
        d = d.pin_memory().to(dev, non_blocking=True)
    return torch.repeat_interleave(d[0], d[1], output_size=n_tok) + torch.arange(n_tok, device=dev,
                                                                                  dtype=torch.long)


def _build_metadata_arena(tab: _TierTable, tokens: torch.Tensor, gi: torch.Tensor, lp: torch.Tensor, *,
                          page_size: int, recent_capacity: int, int2_reserve: int, int4_reserve: int = 0):
    """One int64 allocation holding the page index of every pool, the evicted global indices, the
    Recent-FP ring's index buffers and its device length (precision_pool.py:400-585).

    ``tokens`` are the tier-ordered token indices of ``_expand_tier_tokens``; ``gi`` / ``lp`` the
    plan's global / logical token indices on the same device.  ``int4_reserve`` / ``int2_reserve``
    tokens (whole pages) are reserved after the INT4 / INT2 pool's fields.  Layout: the page fields
    of every pool and the length slot (built on the host, one copy), then the token fields: global
    [FP INT4 INT4-reserve INT2 INT2-reserve], logical [the same], evicted, ring global, ring logical.
    Returns the arena, the four pools' page indexes, the evicted indices and the ring's (global,
    logical, length) buffers.
    """
    ps = int(page_size)
    cap = int(recent_capacity)
    if int2_reserve % ps or int4_reserve % ps or cap % ps:
        raise ValueError("metadata reserves must be whole pages")
    dev = tokens.device
    tiers = [slice(int(tab.first_page[t]), int(tab.first_page[t + 1])) for t in range(3)]
    reserve_pages = (0, int(int4_reserve) // ps, int(int2_reserve) // ps)
    ring_pages = cap // ps

    page_parts = []
    for t, extra in zip(tiers, reserve_pages):
        n_tok = int(tab.tier_tokens[len(page_parts)])
        page_parts.append(np.concatenate((tab.pages[t], np.full(extra, -1), tab.offsets[t],
                                          n_tok + ps * np.arange(extra), tab.lengths[t], np.full(extra, ps))))
    page_parts.append(np.concatenate((np.full(ring_pages, -1), ps * np.arange(ring_pages),
                                      np.zeros(ring_pages, np.int64))))
    page_parts.append(np.zeros(1, np.int64))  # the ring's device length (int32 in the low half)
    page_block = torch.from_numpy(np.concatenate(page_parts).astype(np.int64))
    n_pages_total = int(page_block.numel())
    n_surv = int(tab.tier_tokens[:3].sum())
    n_ev = int(tab.tier_tokens[3])
    n_head = int(tab.tier_tokens[:2].sum())  # FP + INT4 tokens, before the INT4 reserve
    surv_span = n_surv + int(int4_reserve) + int(int2_reserve)
    storage = torch.empty(n_pages_total + 2 * surv_span + n_ev + 2 * cap, device=dev, dtype=torch.long)
    if dev.type != "cpu":
        page_block = page_block.pin_memory()
    storage[:n_pages_total].copy_(page_block, non_blocking=True)
    tok = storage[n_pages_total:]
    tok.fill_(-1)
    g_all, l_all = tok[:surv_span], tok[surv_span:2 * surv_span]
    evicted = tok[2 * surv_span:2 * surv_span + n_ev]
    ring_g = tok[2 * surv_span + n_ev:2 * surv_span + n_ev + cap]
    ring_l = tok[2 * surv_span + n_ev + cap:]
    i2_at = n_head + int(int4_reserve)
    for dst, lo, hi in ((0, 0, n_head), (i2_at, n_head, n_surv)):
        if hi > lo:
            torch.index_select(gi, 0, tokens[lo:hi], out=g_all[dst:dst + hi - lo])
            torch.index_select(lp, 0, tokens[lo:hi], out=l_all[dst:dst + hi - lo])
    if n_ev:
        torch.index_select(gi, 0, tokens[n_surv:], out=evicted)

    cursor = 0

    def take(n):
        nonlocal cursor
        v = storage[cursor:cursor + n]
        cursor += n
        return v

    indexes = []
    tok_start = 0
    for t, extra in zip(tiers, reserve_pages):
        npg = t.stop - t.start + extra
        ids, offs, lens = take(npg), take(npg), take(npg)
        nt = int(tab.tier_tokens[len(indexes)])
        span = nt + extra * ps
        g, l = g_all[tok_start:tok_start + span], l_all[tok_start:tok_start + span]
        tok_start += span
        indexes.append((ids, offs, lens, g, l, npg - extra, nt))
    ring_ids, ring_offs, ring_lens = take(ring_pages), take(ring_pages), take(ring_pages)
    length = take(1).view(torch.int32)[0]
    pools = [PhysicalPageIndex(original_page_ids=ids[:np_], physical_offsets=offs[:np_], lengths=lens[:np_],
                               global_token_indices=g[:nt], logical_positions=l[:nt])
             for ids, offs, lens, g, l, np_, nt in indexes]
    pools.append(PhysicalPageIndex(original_page_ids=ring_ids, physical_offsets=ring_offs, lengths=ring_lens,
                                   global_token_indices=ring_g, logical_positions=ring_l))
    tier_fields = {}
    for name, (ids, offs, lens, g, l, np_, nt) in (("int4", indexes[1]), ("int2", indexes[2])):
        tier_fields.update({f"{name}_original_page_ids_buffer": ids, f"{name}_physical_offsets_buffer": offs,
                            f"{name}_lengths_buffer": lens, f"{name}_global_index_buffer": g,
                            f"{name}_logical_position_buffer": l, f"{name}_page_count": np_,
                            f"{name}_token_count": nt})
    arena = CompactMetadataArena(storage=storage, **tier_fields)
    return arena, pools, evicted, (ring_g, ring_l, length)


def _survivor_layout(plan: LayerCompressionPlan, device):
    """Every non-evicted page in page order: the single pool of a matched-FP cache (precision_pool.py:834-846)."""
    classes = plan.page_classes.detach().to("cpu", torch.long)
    starts = plan.page_offsets.detach().to("cpu", torch.long)
    lens = plan.page_lengths.detach().to("cpu", torch.long)
    pages = torch.nonzero(classes != PageClass.EVICTED_PAGE, as_tuple=False).flatten()
    pl = lens[pages]
    offsets = pl.cumsum(0) - pl
    n_tok = int(pl.sum())
    dev = torch.device(device)
    if n_tok:
        shift = torch.repeat_interleave((starts[pages] - offsets).to(dev), pl.to(dev), output_size=n_tok)
        tokens = shift + torch.arange(n_tok, device=dev, dtype=torch.long)
    else:
        tokens = torch.zeros(0, dtype=torch.long, device=dev)
    return tokens, offsets, pl, pages


def _gather_key_rows(key: torch.Tensor, tokens: torch.Tensor, append_capacity: int, segments) -> BF16KeyArena:
    h, s, d = map(int, key.shape)
    n = int(tokens.numel())
    cap = max(128, _round_up(n + int(append_capacity), 128))
    rows = torch.zeros((h, cap, d), device=key.device, dtype=key.dtype)
    if n:
        _lib.call("r2o_gather_rows", _lib.ptr(key), h, s, _lib.ptr(tokens), n, _lib.ptr(rows), cap,
                  _lib.stream_of(key.device))
    return BF16KeyArena(rows=rows, active_length=n, capacity=cap, segment_offsets=tuple(segments))


def _make_page_index(layout, gi: torch.Tensor, lp: torch.Tensor) -> PhysicalPageIndex:
    """Page index of one pool; ``gi`` / ``lp`` are the plan's global / logical token indices on the
    pool's device."""
    tokens, offsets, lengths, pages = layout
    dev = gi.device
    tokens = tokens.to(dev)
    return PhysicalPageIndex(original_page_ids=pages.to(dev), physical_offsets=offsets.to(dev),
                             lengths=lengths.to(dev), global_token_indices=gi[tokens], logical_positions=lp[tokens])


def _preallocate_recent_pool(name: str, key: torch.Tensor, *, page_size: int, capacity: int,
                             metadata=None) -> PrecisionPool:
    """The Recent-FP ring: bf16/fp16 K and V rows of ``capacity`` tokens and its index buffers.
    ``metadata`` = (page index, global buffer, logical buffer, int32 length) views of a metadata arena;
    without it they are allocated here (the matched-FP cache has no arena)."""
    if capacity < page_size or capacity % page_size:
        raise ValueError("Recent-FP capacity must be positive and page aligned")
    h, _, d = map(int, key.shape)
    dev = key.device
    if metadata is None:
        gbuf = torch.full((capacity,), -1, device=dev, dtype=torch.long)
        lbuf = torch.full((capacity,), -1, device=dev, dtype=torch.long)
        pages = capacity // page_size
        index = PhysicalPageIndex(
            original_page_ids=torch.full((pages,), -1, device=dev, dtype=torch.long),
            physical_offsets=torch.arange(pages, device=dev, dtype=torch.long) * page_size,
            lengths=torch.zeros(pages, device=dev, dtype=torch.long),
            global_token_indices=gbuf, logical_positions=lbuf)
        length = torch.zeros((), device=dev, dtype=torch.int32)
    else:
        index, gbuf, lbuf, length = metadata
    return PrecisionPool(
        name=name, page_index=index,
        fp_k=torch.zeros((h, capacity, d), device=dev, dtype=key.dtype),
        fp_v=torch.zeros((h, capacity, d), device=dev, dtype=key.dtype),
        active_length=0, capacity=capacity, length_device=length,
        global_index_buffer=gbuf, logical_position_buffer=lbuf,
    )


def build_three_precision_cache(
    key: torch.Tensor,
    value: torch.Tensor,
    plan: LayerCompressionPlan,
    *,
    page_size: int = 32,
    quantization_superblock: int = 128,
    key_quantization_superblock: int = 32,
    int2_group_size: int = 32,
    generated_value_precision: str = "int2",
    matched_fp: bool = False,
    preallocate_recent: bool = True,
    cache_variant: str = "v_fourq_k_int4_compact",
    compact_key_append_capacity: int | None = None,
    recent_flush_size: int = 128,
) -> ThreePrecisionCache:
    """Stable page reorder into contiguous FP/INT4/INT2/Recent-FP pools, packed on the GPU."""
    if key.shape != value.shape or key.ndim != 3:
        raise ValueError("key/value must be logical [Hkv,S,D]")
    if int(key.shape[1]) != int(plan.logical_positions.numel()):
        raise ValueError("K/V sequence length must match the static plan")
    if page_size not in (16, 32, 64):
        raise ValueError("page_size must be 16, 32, or 64")
    if quantization_superblock != 128:
        raise ValueError("formal precision pools use 128-token quantization superblocks")
    if key_quantization_superblock not in (32, 64, 128):
        raise ValueError("K quantization superblock must be 32, 64, or 128")
    if recent_flush_size not in (32, 64, 128) or recent_flush_size % page_size \
            or recent_flush_size % key_quantization_superblock:
        raise ValueError("recent_flush_size must be 32/64/128 and align to page/K blocks")
    if preallocate_recent and plan.recent_fp_capacity < recent_flush_size:
        raise ValueError("Recent-FP capacity must cover one configured flush")
    if cache_variant not in ("v_fourq_k_int2_compact", "v_fourq_k_int4_compact", "v_fourq_k_bf16"):
        raise ValueError(f"unsupported cache_variant: {cache_variant}")
    if generated_value_precision not in ("int2", "int4"):
        raise ValueError("generated_value_precision must be int2 or int4")
    if not preallocate_recent:
        raise NotImplementedError("the gfx950 path implements the caches with a preallocated Recent-FP ring")
    if int(key.shape[2]) != 128:
        raise ValueError("the SSPA decode path requires head_dim 128")
    _lib.require_device(key, "key")
    _lib.dtype_code(key.dtype)
    bf16_keys = matched_fp or cache_variant == "v_fourq_k_bf16"  # key rows in the model dtype (bf16 or fp16)
    key = key.contiguous()
    value = value.contiguous()
    dev = key.device
    tab = _tier_page_table(plan)
    if int(tab.tier_tokens.sum()) != int(key.shape[1]):
        raise ValueError("compact physical pools must cover every logical token")
    if plan.recent_fp_capacity < page_size or plan.recent_fp_capacity % page_size:
        raise ValueError("Recent-FP capacity must be positive and page aligned")
    h = int(key.shape[0])
    stream = _lib.stream_of(dev)
    append_capacity = plan.recent_fp_capacity if compact_key_append_capacity is None \
        else int(compact_key_append_capacity)
    gi = plan.global_token_indices.detach().to(dev, torch.long)
    lp = plan.logical_positions.detach().to(dev, torch.long)
    tokens = _expand_tier_tokens(tab, dev)
    s_fp, s_i4, s_i2 = (int(n) for n in tab.tier_tokens[:3])
    n_surv = s_fp + s_i4 + s_i2
    common = dict(page_size=int(page_size), quantization_superblock=int(quantization_superblock),
                  cache_variant=cache_variant, recent_flush_size=int(recent_flush_size),
                  generated_value_precision=str(generated_value_precision))
    if matched_fp:  # every surviving page, K and V in bf16, in one FP pool (precision_pool.py:834-876)
        surv = _survivor_layout(plan, dev)
        n = int(surv[0].numel())
        arena = _gather_key_rows(key, surv[0], append_capacity, (0, n, n))
        fp_pool = PrecisionPool(name="fp", page_index=_make_page_index(surv, gi, lp), fp_k=arena.view(0, n))
        fp_pool.fp_v = torch.empty((h, n, 128), device=dev, dtype=value.dtype)
        if n:
            _lib.call("r2o_gather_rows", _lib.ptr(value), h, int(value.shape[1]), _lib.ptr(surv[0]), n,
                      _lib.ptr(fp_pool.fp_v), n, stream)
        empty = (surv[0][:0], surv[1][:0], surv[2][:0], surv[3][:0])
        recent = _preallocate_recent_pool("recent_fp", key, page_size=page_size, capacity=plan.recent_fp_capacity)
        return ThreePrecisionCache(
            fp_pool=fp_pool, int4_pool=PrecisionPool(name="int4", page_index=_make_page_index(empty, gi, lp)),
            int2_pool=PrecisionPool(name="int2", page_index=_make_page_index(empty, gi, lp)),
            recent_fp_pool=recent, matched_fp=True, bf16_key=arena, generated_k_offset=n,
            evicted_global_indices=gi[tokens[n_surv:]], **common)
    fp_tokens, i4_tokens, i2_tokens = tokens[:s_fp], tokens[s_fp:s_fp + s_i4], tokens[s_fp + s_i4:n_surv]

    fp_v = int4_v = compact_int4_value = None
    if s_fp:
        fp_v = torch.empty((h, s_fp, 128), device=dev, dtype=value.dtype)
        _lib.call("r2o_gather_rows", _lib.ptr(value), h, int(value.shape[1]), _lib.ptr(fp_tokens), s_fp,
                  _lib.ptr(fp_v), s_fp, stream)
    int4_generated = generated_value_precision == "int4"
    if int4_generated:  # the INT4 pool's V is an arena with room for generated flushes (precision_pool.py:935-942)
        compact_int4_value = int4_v = build_compact_int4_value_arena(value, i4_tokens, append_capacity=append_capacity)
    elif s_i4:
        int4_v = fused_gather_pack_int4_value(value, i4_tokens)
    compact_value = build_compact_int2_value_arena(value, i2_tokens, group_size=int2_group_size,
                                                   append_capacity=0 if int4_generated else append_capacity)
    compact_key = bf16_arena = None
    if bf16_keys:  # v_fourq_k_bf16: every pool keeps bf16 K rows (precision_pool.py:878-906)
        bf16_arena = _gather_key_rows(key, tokens[:n_surv], append_capacity, (0, s_fp, s_fp + s_i4))
        reserve = reserve4 = 0  # no compact K arena to flush into (precision_pool.py:404-408)
    else:
        build_key = build_compact_int2_key_arena if cache_variant == "v_fourq_k_int2_compact" \
            else build_compact_int4_key_arena
        compact_key = build_key(key, (fp_tokens, i4_tokens, i2_tokens), append_capacity=append_capacity,
                                superblock_size=key_quantization_superblock)
        key_room = compact_key.capacity - compact_key.active_length
        reserve = min(compact_value.capacity - compact_value.active_length, key_room) // page_size * page_size
        reserve4 = 0 if compact_int4_value is None else \
            min(compact_int4_value.capacity - compact_int4_value.active_length, key_room) // page_size * page_size
    meta, (fp_pi, i4_pi, i2_pi, ring_pi), evicted, (ring_g, ring_l, ring_len) = _build_metadata_arena(
        tab, tokens, gi, lp, page_size=page_size, recent_capacity=plan.recent_fp_capacity, int2_reserve=reserve,
        int4_reserve=reserve4)
    fp_pool = PrecisionPool(name="fp", page_index=fp_pi, fp_v=fp_v)
    int4_pool = PrecisionPool(name="int4", page_index=i4_pi, packed_v=int4_v)
    int2_pool = PrecisionPool(name="int2", page_index=i2_pi, packed_v=compact_value)
    recent = _preallocate_recent_pool("recent_fp", key, page_size=page_size, capacity=plan.recent_fp_capacity,
                                      metadata=(ring_pi, ring_g, ring_l, ring_len))
    if bf16_keys:
        fp_pool.fp_k, int4_pool.fp_k = bf16_arena.view(0, s_fp), bf16_arena.view(s_fp, s_i4)
        int2_pool.fp_k = bf16_arena.view(s_fp + s_i4, s_i2)
        return ThreePrecisionCache(
            fp_pool=fp_pool, int4_pool=int4_pool, int2_pool=int2_pool, recent_fp_pool=recent, matched_fp=False,
            compact_value=compact_value, compact_int4_value=compact_int4_value, static_int4_tokens=s_i4,
            bf16_key=bf16_arena, metadata_arena=meta, evicted_global_indices=evicted, **common)
    return ThreePrecisionCache(
        fp_pool=fp_pool, int4_pool=int4_pool, int2_pool=int2_pool, recent_fp_pool=recent, matched_fp=False,
        compact_key=compact_key, compact_value=compact_value, compact_int4_value=compact_int4_value,
        static_int4_tokens=s_i4, generated_k_offset=compact_key.active_length, metadata_arena=meta,
        evicted_global_indices=evicted,
        **common)


# ------------------------------------------------------------------------- append / flush
@dataclass
class DynamicCacheStats:
    appended_tokens: int = 0
    flushed_superblocks: int = 0
    flushed_tokens: int = 0
    flushed_int4_value_tokens: int = 0
    recent_reallocation_count: int = 0
    local_tail_dequant_tokens: int = 0
    full_dequant_tensor_count: int = 0


def _append_lowbit_page_metadata(pool: PrecisionPool, global_block: torch.Tensor, logical_block: torch.Tensor,
                                 page_size: int) -> None:
    n = int(global_block.numel())
    if n <= 0 or n % page_size:
        raise ValueError("low-bit metadata append must contain complete pages")
    pages = n // page_size
    old = pool.page_index
    dev = global_block.device
    start = pool.token_count
    pool.page_index = PhysicalPageIndex(
        original_page_ids=torch.cat((old.original_page_ids, torch.full((pages,), -1, device=dev, dtype=torch.long))),
        physical_offsets=torch.cat((old.physical_offsets,
                                    start + torch.arange(pages, device=dev, dtype=torch.long) * page_size)),
        lengths=torch.cat((old.lengths, torch.full((pages,), page_size, device=dev, dtype=torch.long))),
        global_token_indices=torch.cat((old.global_token_indices, global_block)),
        logical_positions=torch.cat((old.logical_positions, logical_block)),
    )


def flush_full_recent_pool(cache: ThreePrecisionCache, stats: DynamicCacheStats) -> bool:
    """If the Recent-FP ring is full, move its oldest ``recent_flush_size`` tokens into the cache
    (compact INT4/INT2-K + INT2-V or, with INT4 generated values, INT4-V arenas, or the matched-FP
    pool) and shift the ring: the flush half of
    ``append_generated_token`` (dynamic_fourq_cache.py:185-253).  Returns whether it flushed.  The
    caller re-prepares its executors afterwards."""
    pool = cache.recent_fp_pool
    flush = int(cache.recent_flush_size)
    if pool.active_length is None or pool.capacity < flush or pool.length_device is None:
        raise RuntimeError("Recent-FP pool was not preallocated for dynamic generation")
    if pool.active_length != pool.capacity:
        return False
    h, cap = int(pool.fp_k.shape[0]), int(pool.capacity)
    stream = _lib.stream_of(pool.fp_k.device)
    key_block = pool.fp_k[:, :flush]
    value_block = pool.fp_v[:, :flush]
    # Views of the ring's oldest indices: every consumer below copies them on this stream before
    # the ring shift is launched, so no snapshot is needed.
    global_block = pool.global_index_buffer[:flush]
    logical_block = pool.logical_position_buffer[:flush]
    if cache.matched_fp:  # _append_matched_fp_block (dynamic_fourq_cache.py:145-170)
        _append_lowbit_page_metadata(cache.fp_pool, global_block, logical_block, cache.page_size)
        cache.bf16_key.append_block(key_block)
        n = cache.bf16_key.active_length
        cache.bf16_key.segment_offsets = (0, n, n)
        cache.fp_pool.fp_k = cache.bf16_key.view(0, n)
        cache.fp_pool.fp_v = torch.cat((cache.fp_pool.fp_v, value_block), dim=1)
        cache.generated_k_offset = n
    elif cache.bf16_key is not None:  # dynamic_fourq_cache.py:226-230
        raise RuntimeError("K-BF16/V-FourQ requires an append_fp_only Recent-FP capacity covering the "
                           "requested generation horizon")
    else:
        if cache.compact_key is None:
            raise RuntimeError("compact K cache is missing its compact K arena")
        int4_values = cache.generated_value_precision == "int4"
        if int4_values and cache.compact_int4_value is None:
            raise RuntimeError("generated INT4 V policy is missing its compact arena")
        if not int4_values and cache.compact_value is None:
            raise RuntimeError("compact INT2 K cache is missing its compact INT2 V arena")
        stats.local_tail_dequant_tokens += cache.compact_key.append_superblock(key_block, source_tokens=cap) \
            if flush == 128 else _flush_size_error(flush)
        if int4_values:  # dynamic_fourq_cache.py:212-219
            cache.compact_int4_value.append_block(value_block, source_tokens=cap)
            stats.flushed_int4_value_tokens += flush
            target = cache.int4_pool
        else:
            cache.compact_value.append_superblock(value_block, source_tokens=cap)
            target = cache.int2_pool
        if cache.metadata_arena is not None:  # in place (dynamic_fourq_cache.py:236-243)
            append = cache.metadata_arena.append_int4_pages if int4_values else cache.metadata_arena.append_int2_pages
            append(target, global_block, logical_block, cache.page_size)
        else:
            _append_lowbit_page_metadata(target, global_block, logical_block, cache.page_size)
    _lib.call("r2o_recent_shift", _lib.ptr(pool.fp_k), _lib.ptr(pool.fp_v), h, cap, flush, pool.active_length,
              _lib.ptr(pool.global_index_buffer), _lib.ptr(pool.logical_position_buffer),
              _lib.ptr(pool.length_device), _lib.ptr(pool.page_index.lengths), cache.page_size, stream)
    pool.active_length -= flush
    stats.flushed_superblocks += 1
    stats.flushed_tokens += flush
    return True


def append_generated_token(cache: ThreePrecisionCache, new_key: torch.Tensor, new_value: torch.Tensor, *,
                           global_token_index: int, logical_position: int, stats: DynamicCacheStats) -> bool:
    """Append one token to the Recent-FP ring; when it is full, flush its oldest chunk first
    (dynamic_fourq_cache.py:172-267)."""
    pool = cache.recent_fp_pool
    flush = int(cache.recent_flush_size)
    if pool.active_length is None or pool.capacity < flush or pool.length_device is None:
        raise RuntimeError("Recent-FP pool was not preallocated for dynamic generation")
    if new_key.ndim == 4:
        new_key, new_value = new_key[0], new_value[0]
    if new_key.shape != new_value.shape or new_key.ndim != 3 or int(new_key.shape[1]) != 1:
        raise ValueError("new K/V must be [Hkv,1,D] or [1,Hkv,1,D]")
    _lib.require_device(new_key, "new_key")
    if new_key.dtype != pool.fp_k.dtype or new_value.dtype != pool.fp_v.dtype:
        raise ValueError("new K/V dtype must match the Recent-FP ring")
    h, cap = int(pool.fp_k.shape[0]), int(pool.capacity)
    stream = _lib.stream_of(new_key.device)
    flushed = flush_full_recent_pool(cache, stats)
    nk = new_key.reshape(h, -1).contiguous()
    nv = new_value.reshape(h, -1).contiguous()
    _lib.call("r2o_recent_append", _lib.ptr(pool.fp_k), _lib.ptr(pool.fp_v), h, cap, _lib.ptr(nk), _lib.ptr(nv),
              pool.active_length, int(global_token_index), int(logical_position), _lib.ptr(pool.length_device),
              _lib.ptr(pool.global_index_buffer), _lib.ptr(pool.logical_position_buffer),
              _lib.ptr(pool.page_index.lengths), cache.page_size, stream)
    pool.active_length += 1
    stats.appended_tokens += 1
    return flushed


def _flush_size_error(flush: int) -> int:
    raise ValueError(f"compact K flush requires 128 tokens, the cache flushes {flush}")
