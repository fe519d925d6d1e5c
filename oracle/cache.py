"""numpy restatement of the three-pool SSPA cache and its append/flush (test infrastructure only).

Follows, for the released ``v_fourq_k_int4_compact`` cache with INT2 generated values (INT4 ones with
``gen_values="int4"``: precision_pool.py:935-971, dynamic_fourq_cache.py:212-219,
triton_fourq_attention.py:95-111; and the other K formats: ``v_fourq_k_int2_compact`` keeps K in a per-channel affine INT2 arena,
compact_int2_key.py:14-153; ``v_fourq_k_bf16`` keeps the pools' K rows in the input dtype; the
matched-FP cache keeps every surviving page, K and V, in one FP pool in page order,
precision_pool.py:834-876, with flushes appended to it, dynamic_fourq_cache.py:145-170, 200-204):
  * ``_compact_page_layouts``      precision_pool.py:611-669  (stable FP -> INT4 -> INT2 -> evicted)
  * ``build_three_precision_cache`` precision_pool.py:787-984 (+ arenas in compact_int4_key.py:223-281,
                                   fused_value_pack.py:152-193, 519-575, recent ring :747-784)
  * ``append_generated_token``     dynamic_fourq_cache.py:172-267 (flush: compact_int4_key.py:210-220,
                                   fused_value_pack.py:474-516; ring refresh :108-117)

Pinning: tests/test_oracle_golden.py compares every arena byte, scale, zero point, ring row and
pool count against fixtures written by the reference's own CPU path (tests/golden/make_golden.py),
before and after a flush with a partial K tail.  tests/test_oracle_quant.py checks the
reference's own invariants (tests/test_active_cache_storage.py:72-94: 129 appends on a 128-token
ring give 128 flushed tokens and one active token) and the FP/INT4/INT2 token-order partition.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from .quant import (
    dequantize_int2_key,
    dequantize_int4_key,
    quantize_int2_key_per_channel,
    quantize_int2_value,
    quantize_int4_key_per_channel,
    quantize_int4_value,
    round_to_dtype,
)

# PageClass values (policy/four_quadrant.py:6-12)
EVICTED_PAGE, FP_PAGE, INT4_PAGE, RECENT_FP_PAGE, PROTECTED_FP_PAGE, INT2_PAGE = 0, 1, 2, 3, 4, 5


def _round_up(v: int, m: int) -> int:
    return -(-int(v) // int(m)) * int(m)


def compact_page_layouts(page_offsets, page_lengths, page_classes):
    """Token order of each pool: FP (incl. protected and recent pages), INT4, INT2, evicted.

    Pages are stably sorted by tier (precision_pool.py:621-632); tokens keep page order.
    Returns four int64 arrays of logical token indices.
    """
    classes = np.asarray(page_classes, dtype=np.int64)
    category = np.full(classes.shape, 3, dtype=np.int64)
    category[(classes == FP_PAGE) | (classes == PROTECTED_FP_PAGE) | (classes == RECENT_FP_PAGE)] = 0
    category[classes == INT4_PAGE] = 1
    category[classes == INT2_PAGE] = 2
    order = np.argsort(category, kind="stable")
    out = []
    for tier in range(4):
        pages = order[category[order] == tier]
        parts = [np.arange(page_offsets[p], page_offsets[p] + page_lengths[p], dtype=np.int64) for p in pages]
        out.append(np.concatenate(parts) if parts else np.zeros(0, np.int64))
    return tuple(out)


@dataclass
class OracleCache:
    dtype: str
    hkv: int
    page_size: int
    superblock: int
    group: int
    flush_size: int
    # compact K arena: INT4 (packed [H,cap,D/2], fp16 scale, u8 zero point) or, for the
    # "int2k" variant, INT2 (packed [H,cap,D/4], fp16 scale, fp16 offset held in k_zero)
    k_packed: np.ndarray
    k_scale: np.ndarray
    k_zero: np.ndarray
    k_active: int
    k_capacity: int
    k_segments: tuple
    # value pools
    fp_v: np.ndarray            # [H, S_FP, D] float32 (values of the input dtype)
    v4_packed: np.ndarray       # [H, S_I4, D/2] u8
    v4_scale: np.ndarray        # [H, S_I4, 1] f32
    v2_packed: np.ndarray       # [H, V2cap, D/4] u8
    v2_scale: np.ndarray        # [H, V2cap, D/G, 1] f16
    v2_zero: np.ndarray         # [H, V2cap, D/G, 1] u8
    v2_active: int
    v2_capacity: int
    # Recent-FP ring
    recent_k: np.ndarray        # [H, cap, D] float32
    recent_v: np.ndarray
    recent_active: int
    recent_global: np.ndarray   # [cap] int64
    recent_logical: np.ndarray
    recent_page_lengths: np.ndarray
    # pool bookkeeping
    pool_tokens: list = field(default_factory=list)   # [fp, int4, int2(incl. generated)]
    int2_global: list = field(default_factory=list)
    int2_logical: list = field(default_factory=list)
    int4_global: list = field(default_factory=list)    # INT4 pool's token indices (static, then flushed
    int4_logical: list = field(default_factory=list)   # with INT4 generated values)
    flushed_tokens: int = 0
    tail_dequant_tokens: int = 0
    # BF16-K variants: K rows in physical order [H, cap, D] float32 (values of the input dtype)
    variant: str = "int4k"
    k_rows: np.ndarray | None = None
    # generated values: "int2" (released) or "int4" (the INT4 pool's V rows are an arena of
    # capacity v4_capacity, static tokens first; generated keys start at gen_k_offset)
    gen_values: str = "int2"
    v4_capacity: int = 0
    static_i4: int = 0
    gen_k_offset: int = 0

    @property
    def recent_capacity(self) -> int:
        return int(self.recent_k.shape[1])


def survivor_layout(page_offsets, page_lengths, page_classes):
    """Tokens of every non-evicted page in page order (matched-FP pool, precision_pool.py:834-846)."""
    classes = np.asarray(page_classes, dtype=np.int64)
    parts = [np.arange(page_offsets[p], page_offsets[p] + page_lengths[p], dtype=np.int64)
             for p in np.nonzero(classes != EVICTED_PAGE)[0]]
    return np.concatenate(parts) if parts else np.zeros(0, np.int64)


def build_cache(key, value, page_offsets, page_lengths, page_classes, *, dtype: str,
                page_size: int = 32, superblock: int = 32, group: int = 32,
                recent_capacity: int = 128, append_capacity: int = 260,
                flush_size: int = 128, variant: str = "int4k", gen_values: str = "int2") -> OracleCache:
    """Restatement of ``build_three_precision_cache``: ``variant`` "int4k" (``v_fourq_k_int4_compact``),
    "int2k" (``v_fourq_k_int2_compact``), "bf16k" (``v_fourq_k_bf16``) or "matched" (``matched_fp=True``);
    ``gen_values`` the ``generated_value_precision`` ("int4": the INT4 pool's V rows get
    ``append_capacity`` tokens of room, the INT2-V arena none, precision_pool.py:935-956).

    ``key``/``value`` are float32 arrays holding values of ``dtype`` ([Hkv, S, 128]).
    """
    key = np.asarray(key, np.float32)
    value = np.asarray(value, np.float32)
    h, s, d = key.shape
    fp_t, i4_t, i2_t, ev_t = compact_page_layouts(page_offsets, page_lengths, page_classes)
    if variant == "matched":
        fp_t = survivor_layout(page_offsets, page_lengths, page_classes)
        i4_t = i2_t = np.zeros(0, np.int64)
        ev_t = np.zeros(s - len(fp_t), np.int64)
    elif variant not in ("int4k", "int2k", "bf16k"):
        raise ValueError(f"unknown variant {variant}")
    if len(fp_t) + len(i4_t) + len(i2_t) + len(ev_t) != s:
        raise ValueError("compact physical pools must cover every logical token")
    # compact INT4-K arena over the physical order FP, INT4, INT2 (compact_int4_key.py:223-281)
    ordered = np.concatenate((fp_t, i4_t, i2_t))
    active = len(ordered)
    k_cap = max(128, _round_up(active + append_capacity, 128))
    blocks = k_cap // superblock
    k_packed = np.zeros((h, k_cap, d // (4 if variant == "int2k" else 2)), np.uint8)
    k_scale = np.zeros((h, blocks, d), np.float16)
    k_zero = np.zeros((h, blocks, d), np.float16 if variant == "int2k" else np.uint8)
    k_rows = None
    if variant == "int2k":  # build_compact_int2_key_arena (compact_int2_key.py:125-153): one quantise
        if active:
            p, sc, off = quantize_int2_key_per_channel(key[:, ordered], superblock)
            k_packed[:, :active] = p
            k_scale[:, : sc.shape[1]] = sc
            k_zero[:, : off.shape[1]] = off
    elif variant == "int4k":
        for start in range(0, active, superblock):
            toks = ordered[start : start + superblock]
            p, sc, z = quantize_int4_key_per_channel(key[:, toks], superblock)
            k_packed[:, start : start + len(toks)] = p
            k_scale[:, start // superblock] = sc[:, 0]
            k_zero[:, start // superblock] = z[:, 0]
    else:
        k_rows = np.zeros((h, k_cap, d), np.float32)
        k_rows[:, :active] = key[:, ordered]
    # value pools
    fp_v = value[:, fp_t].copy()
    if gen_values not in ("int2", "int4"):
        raise ValueError("gen_values must be int2 or int4")
    int4_gen = gen_values == "int4" and variant != "matched"
    v4_packed, v4_scale = quantize_int4_value(value[:, i4_t])
    v4_cap = max(1, len(i4_t) + append_capacity) if int4_gen else len(i4_t)  # fused_value_pack.py:302-330
    if int4_gen:
        v4_packed = np.concatenate((v4_packed, np.zeros((h, v4_cap - len(i4_t), d // 2), np.uint8)), axis=1)
        v4_scale = np.concatenate((v4_scale, np.zeros((h, v4_cap - len(i4_t), 1), np.float32)), axis=1)
    v2_cap = max(128, _round_up(len(i2_t) + (0 if int4_gen else append_capacity), 128))
    groups = d // group
    v2_packed = np.zeros((h, v2_cap, d // 4), np.uint8)
    v2_scale = np.zeros((h, v2_cap, groups, 1), np.float16)
    v2_zero = np.zeros((h, v2_cap, groups, 1), np.uint8)
    p2, s2, z2 = quantize_int2_value(value[:, i2_t], group)
    v2_packed[:, : len(i2_t)] = p2
    v2_scale[:, : len(i2_t)] = s2
    v2_zero[:, : len(i2_t)] = z2
    # Recent-FP ring, empty at build time (precision_pool.py:747-784)
    pages = recent_capacity // page_size
    return OracleCache(
        dtype=dtype, hkv=h, page_size=page_size, superblock=superblock, group=group,
        flush_size=flush_size,
        k_packed=k_packed, k_scale=k_scale, k_zero=k_zero, k_active=active, k_capacity=k_cap,
        k_segments=(0, len(fp_t), len(fp_t) + len(i4_t)),
        fp_v=fp_v, v4_packed=v4_packed, v4_scale=v4_scale,
        v2_packed=v2_packed, v2_scale=v2_scale, v2_zero=v2_zero,
        v2_active=len(i2_t), v2_capacity=v2_cap,
        recent_k=np.zeros((h, recent_capacity, d), np.float32),
        recent_v=np.zeros((h, recent_capacity, d), np.float32),
        recent_active=0,
        recent_global=np.full(recent_capacity, -1, np.int64),
        recent_logical=np.full(recent_capacity, -1, np.int64),
        recent_page_lengths=np.zeros(pages, np.int64),
        pool_tokens=[len(fp_t), len(i4_t), len(i2_t)],
        int2_global=list(i2_t), int2_logical=list(i2_t), int4_global=list(i4_t), int4_logical=list(i4_t),
        variant=variant, k_rows=k_rows,
        gen_values=gen_values, v4_capacity=v4_cap, static_i4=len(i4_t), gen_k_offset=active,
    )


def _flush_key_superblock_int2(c: OracleCache, key_block: np.ndarray) -> int:
    """``CompactInt2KeyArena.append_superblock`` (compact_int2_key.py:110-122)."""
    n = key_block.shape[1]
    if c.k_active + 128 > c.k_capacity:
        raise RuntimeError("compact INT2 K capacity exhausted")
    prefix = c.k_active // c.superblock * c.superblock
    tail_count = c.k_active - prefix
    tail = round_to_dtype(dequantize_int2_key(c.k_packed, c.k_scale, c.k_zero, prefix, tail_count, c.superblock),
                          c.dtype)
    merged = np.concatenate((tail, key_block), axis=1)
    p, sc, off = quantize_int2_key_per_channel(merged, c.superblock)
    c.k_packed[:, prefix : prefix + merged.shape[1]] = p
    b0 = prefix // c.superblock
    c.k_scale[:, b0 : b0 + sc.shape[1]] = sc
    c.k_zero[:, b0 : b0 + off.shape[1]] = off
    c.k_active += n
    return tail_count


def _flush_key_superblock(c: OracleCache, key_block: np.ndarray) -> int:
    """``CompactInt4KeyArena.append_superblock`` (compact_int4_key.py:210-220)."""
    if c.variant == "int2k":
        return _flush_key_superblock_int2(c, key_block)
    n = key_block.shape[1]
    if c.k_active + 128 > c.k_capacity:
        raise RuntimeError("compact INT4 K capacity exhausted")
    prefix = c.k_active // c.superblock * c.superblock
    tail_count = c.k_active - prefix
    tail = dequantize_int4_key(c.k_packed, c.k_scale, c.k_zero, prefix, tail_count, c.superblock)
    tail = round_to_dtype(tail, c.dtype)
    merged = np.concatenate((tail, key_block), axis=1)
    p, sc, z = quantize_int4_key_per_channel(merged, c.superblock)
    c.k_packed[:, prefix : prefix + merged.shape[1]] = p
    b0 = prefix // c.superblock
    c.k_scale[:, b0 : b0 + sc.shape[1]] = sc
    c.k_zero[:, b0 : b0 + z.shape[1]] = z
    c.k_active += n
    return tail_count


def _flush_value_int2(c: OracleCache, value_block: np.ndarray) -> None:
    """``CompactInt2ValueArena.append_superblock`` (fused_value_pack.py:474-516)."""
    n = value_block.shape[1]
    dst = c.v2_active
    if dst + n > c.v2_capacity:
        raise RuntimeError(f"compact INT2 V capacity exhausted: need {dst + n}, have {c.v2_capacity}")
    p, s, z = quantize_int2_value(value_block, c.group)
    c.v2_packed[:, dst : dst + n] = p
    c.v2_scale[:, dst : dst + n] = s
    c.v2_zero[:, dst : dst + n] = z
    c.v2_active += n


def _flush_value_int4(c: OracleCache, value_block: np.ndarray) -> None:
    """``CompactInt4ValueArena.append_block`` (fused_value_pack.py:263-299)."""
    n = value_block.shape[1]
    dst = c.pool_tokens[1]
    if dst + n > c.v4_capacity:
        raise RuntimeError(f"compact INT4 V capacity exhausted: need {dst + n}, have {c.v4_capacity}")
    p, s = quantize_int4_value(value_block)
    c.v4_packed[:, dst : dst + n] = p
    c.v4_scale[:, dst : dst + n] = s


def append_token(c: OracleCache, new_k, new_v, *, global_index: int, logical_position: int) -> bool:
    """``append_generated_token`` with the compact INT4-K / INT2-V (or INT4-V) flush.

    ``new_k``/``new_v`` are [Hkv, D] float32 holding values of the cache dtype.
    """
    flushed = False
    cap = c.recent_capacity
    f = c.flush_size
    if c.recent_active == cap:
        key_block = c.recent_k[:, :f].copy()
        value_block = c.recent_v[:, :f].copy()
        g_block = c.recent_global[:f].copy()
        l_block = c.recent_logical[:f].copy()
        if c.variant == "matched":  # _append_matched_fp_block (dynamic_fourq_cache.py:145-170)
            if c.k_active + f > c.k_capacity:
                grown = np.zeros((c.hkv, c.k_capacity + _round_up(f, 128), c.k_rows.shape[2]), np.float32)
                grown[:, : c.k_active] = c.k_rows[:, : c.k_active]
                c.k_rows, c.k_capacity = grown, grown.shape[1]
            c.k_rows[:, c.k_active : c.k_active + f] = key_block
            c.k_active += f
            c.fp_v = np.concatenate((c.fp_v, value_block), axis=1)
            c.pool_tokens[0] += f
        elif c.variant == "bf16k":  # dynamic_fourq_cache.py:226-230
            raise RuntimeError("K-BF16/V-FourQ requires an append_fp_only Recent-FP capacity "
                               "covering the requested generation horizon")
        else:
            c.tail_dequant_tokens += _flush_key_superblock(c, key_block)
            if c.gen_values == "int4":  # dynamic_fourq_cache.py:212-219, metadata :240-243
                _flush_value_int4(c, value_block)
                c.int4_global.extend(g_block.tolist())
                c.int4_logical.extend(l_block.tolist())
                c.pool_tokens[1] += f
            else:
                _flush_value_int2(c, value_block)
                c.int2_global.extend(g_block.tolist())
                c.int2_logical.extend(l_block.tolist())
                c.pool_tokens[2] += f
        rem = c.recent_active - f
        c.recent_k[:, :rem] = c.recent_k[:, f : c.recent_active].copy()
        c.recent_v[:, :rem] = c.recent_v[:, f : c.recent_active].copy()
        c.recent_global[:rem] = c.recent_global[f : c.recent_active].copy()
        c.recent_logical[:rem] = c.recent_logical[f : c.recent_active].copy()
        c.recent_active = rem
        c.flushed_tokens += f
        flushed = True
    pos = c.recent_active
    c.recent_k[:, pos] = np.asarray(new_k, np.float32).reshape(c.hkv, -1)
    c.recent_v[:, pos] = np.asarray(new_v, np.float32).reshape(c.hkv, -1)
    c.recent_global[pos] = int(global_index)
    c.recent_logical[pos] = int(logical_position)
    c.recent_active += 1
    offsets = np.arange(len(c.recent_page_lengths)) * c.page_size
    c.recent_page_lengths[:] = np.clip(c.recent_active - offsets, 0, c.page_size)
    return flushed


def pool_kv(c: OracleCache):
    """Dequantised (K, V) float32 per non-empty pool, in the oracle's pool order FP, INT4, INT2, Recent."""
    from .quant import dequantize_int2_value, dequantize_int4_value, round_to_dtype

    out = []
    s_fp, s_i4, s_i2 = c.pool_tokens
    segs = c.k_segments

    def keys(start, n):
        if c.k_rows is not None:
            return c.k_rows[:, start : start + n]
        if c.variant == "int2k":
            return dequantize_int2_key(c.k_packed, c.k_scale, c.k_zero, start, n, c.superblock)
        return dequantize_int4_key(c.k_packed, c.k_scale, c.k_zero, start, n, c.superblock)

    if s_fp:
        out.append((keys(segs[0], s_fp), c.fp_v))
    if s_i4 and c.gen_values == "int4" and c.variant != "matched":
        # static keys at their segment, generated ones at gen_k_offset (triton_fourq_attention.py:95-111);
        # CompactInt4ValueArena.dequantize_range stays fp32 (fused_value_pack.py:241-256)
        static = min(c.static_i4, s_i4)
        k4 = keys(segs[1], static)
        if s_i4 > static:
            k4 = np.concatenate((k4, keys(c.gen_k_offset, s_i4 - static)), axis=1)
        out.append((k4, dequantize_int4_value(c.v4_packed[:, :s_i4], c.v4_scale[:, :s_i4])))
    elif s_i4:
        # PackedTensor.dequantize rounds the fp32 product back to the input dtype
        # (packed_kv_layout.py:30-32); the compact INT4-K / INT2-V arenas stay fp32.
        out.append((keys(segs[1], s_i4), round_to_dtype(dequantize_int4_value(c.v4_packed, c.v4_scale), c.dtype)))
    if s_i2:
        out.append((keys(segs[2], s_i2),
                    dequantize_int2_value(c.v2_packed[:, :s_i2], c.v2_scale[:, :s_i2], c.v2_zero[:, :s_i2], c.group)))
    if c.recent_active:
        out.append((c.recent_k[:, : c.recent_active], c.recent_v[:, : c.recent_active]))
    return out
