"""torch-CPU restatement of the reference's dequantise-then-attention path (test and CPU-baseline
infrastructure only: imported by tests/ and by bench.py's ``cpu_baseline`` leg, never by the package).

The reference's ``triton_mixed_reference`` (r2omni/sspa/kernels/triton_fourq_attention.py:72-125)
holds the cache as torch tensors and dequantises every pool with torch ops on each call
(``_pool_kv`` :17-38), then forms per-pool softmax states and merges them.  ``TorchCache`` holds an
``OracleCache``'s arenas as torch tensors once, and ``mixed_reference`` repeats the per-call work:
  * INT4-K  ``CompactInt4KeyArena.dequantize_range`` (compact_int4_key.py:175-195): nibbles by
            ``& 15`` / ``>> 4``, per-superblock scale and zero by ``index_select``, (code - z) * s;
  * INT2-K  ``CompactInt2KeyArena.dequantize_range`` (compact_int2_key.py:69-96): code * s + offset;
  * INT4-V  ``PackedTensor.dequantize`` (packed_kv_layout.py:30-32, quantization.py:105-116):
            signed nibbles times the per-token fp32 scale, rounded back to the cache dtype;
  * INT2-V  ``CompactInt2ValueArena.dequantize_range`` (fused_value_pack.py:450-472):
            (crumb - z) * s per group;
  * FP-V / Recent-FP rows ``.float()``;
then ``oracle.attention.partial_state`` / ``merge_state`` (triton_fourq_attention.py:41-69).

Pinning (tests/test_oracle_torch_path.py): on caches of every variant, before and after a flush,
every dequantised pool and the attention output equal those of ``oracle.cache.pool_kv`` /
``oracle.attention.mixed_reference`` bit for bit; those are pinned against the reference's own
golden fixtures.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from .attention import merge_state, partial_state
from .cache import OracleCache


@dataclass
class TorchCache:
    variant: str
    dtype: torch.dtype
    superblock: int
    group: int
    pool_tokens: tuple
    k_segments: tuple
    k_packed: torch.Tensor
    k_scale: torch.Tensor
    k_zero: torch.Tensor
    k_rows: torch.Tensor | None
    fp_v: torch.Tensor
    v4_packed: torch.Tensor
    v4_scale: torch.Tensor
    v2_packed: torch.Tensor
    v2_scale: torch.Tensor
    v2_zero: torch.Tensor
    recent_k: torch.Tensor
    recent_v: torch.Tensor
    int4_generated: bool = False  # INT4 generated values: the INT4 pool's keys in two runs, fp32 values
    static_i4: int = 0
    gen_k_offset: int = 0


def from_oracle(c: OracleCache) -> TorchCache:
    """The cache's active payload as torch tensors (bf16 / fp16 rows in their dtype, as stored)."""
    dt = torch.bfloat16 if c.dtype == "bfloat16" else torch.float16
    rows = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dt)  # noqa: E731
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))  # noqa: E731
    s_i4, s_i2 = c.pool_tokens[1], c.pool_tokens[2]
    return TorchCache(
        variant=c.variant, dtype=dt, superblock=c.superblock, group=c.group, pool_tokens=tuple(c.pool_tokens),
        k_segments=tuple(c.k_segments), k_packed=t(c.k_packed), k_scale=t(c.k_scale), k_zero=t(c.k_zero),
        k_rows=None if c.k_rows is None else rows(c.k_rows),
        fp_v=rows(c.fp_v), v4_packed=t(c.v4_packed[:, :s_i4]), v4_scale=t(c.v4_scale[:, :s_i4]),
        v2_packed=t(c.v2_packed[:, :s_i2]), v2_scale=t(c.v2_scale[:, :s_i2]), v2_zero=t(c.v2_zero[:, :s_i2]),
        recent_k=rows(c.recent_k[:, : c.recent_active]), recent_v=rows(c.recent_v[:, : c.recent_active]),
        int4_generated=c.gen_values == "int4" and c.variant != "matched", static_i4=c.static_i4,
        gen_k_offset=c.gen_k_offset,
    )


def _keys(c: TorchCache, start: int, n: int) -> torch.Tensor:
    if c.k_rows is not None:
        return c.k_rows[:, start : start + n].float()
    payload = c.k_packed[:, start : start + n]
    h = payload.shape[0]
    blocks = torch.arange(start, start + n) // c.superblock
    scale = c.k_scale.index_select(1, blocks).float()
    zero = c.k_zero.index_select(1, blocks).float()
    if c.variant == "int2k":
        codes = torch.stack([(payload >> (2 * i)) & 3 for i in range(4)], dim=-1).reshape(h, n, 128)
        return codes.float() * scale + zero
    codes = torch.stack((payload & 15, (payload >> 4) & 15), dim=-1).reshape(h, n, 128)
    return (codes.float() - zero) * scale


def pool_kv(c: TorchCache):
    """Dequantised (K, V) float32 per non-empty pool, in the order FP, INT4, INT2, Recent."""
    out = []
    s_fp, s_i4, s_i2 = c.pool_tokens
    seg = c.k_segments
    if s_fp:
        out.append((_keys(c, seg[0], s_fp), c.fp_v.float()))
    if s_i4:
        nib = torch.stack((c.v4_packed & 15, (c.v4_packed >> 4) & 15), dim=-1).to(torch.int16)
        signed = torch.where(nib >= 8, nib - 16, nib).reshape(c.v4_packed.shape[0], s_i4, 128)
        v = signed.float() * c.v4_scale.float()
        if c.int4_generated:  # triton_fourq_attention.py:95-111; the compact INT4-V arena stays fp32
            static = min(c.static_i4, s_i4)
            k = _keys(c, seg[1], static)
            if s_i4 > static:
                k = torch.cat((k, _keys(c, c.gen_k_offset, s_i4 - static)), dim=1)
            out.append((k, v))
        else:  # PackedTensor.dequantize rounds to the input dtype (packed_kv_layout.py:30-32)
            out.append((_keys(c, seg[1], s_i4), v.to(c.dtype).float()))
    if s_i2:
        h = c.v2_packed.shape[0]
        codes = torch.stack([(c.v2_packed >> (2 * k)) & 3 for k in range(4)], dim=-1).reshape(h, s_i2, 128)
        grouped = codes.reshape(h, s_i2, 128 // c.group, c.group).float()
        v = ((grouped - c.v2_zero.float()) * c.v2_scale.float()).reshape(h, s_i2, 128)
        out.append((_keys(c, seg[2], s_i2), v))
    if c.recent_k.shape[1]:
        out.append((c.recent_k.float(), c.recent_v.float()))
    return out


def mixed_reference(query: np.ndarray, cache: TorchCache) -> np.ndarray:
    """fp32 attention of one request (query [1, Hq, 128]) over every pool, dequantised on this call."""
    q = torch.from_numpy(np.ascontiguousarray(query, dtype=np.float32))
    scale = int(q.shape[-1]) ** -0.5
    state = None
    for k, v in pool_kv(cache):
        part = partial_state(q, k, v, scale)
        state = part if state is None else merge_state(state, part)
    if state is None:
        raise ValueError("four-quadrant cache has no surviving tokens")
    return (state[2] / state[1].unsqueeze(-1)).numpy()
