"""The reference manager's correctness mode and CPU-side Hadamard, as drop-ins over this package's cache.

``triton_mixed_reference`` (r2omni/sspa/kernels/triton_fourq_attention.py:72-125) is what
``QwenSSPAAttentionManager`` runs with ``kernel_backend="triton_mixed_reference"``
(qwen_sspa_attention.py:98, :1113, :1640-1644): every pool of the cache is dequantised to fp32 with
torch ops on the cache's device, each pool gives a softmax state (max, sum, weighted values) with the
GQA head map kv = h // (Hq / Hkv), the states are merged exactly, and the result is cast to the query
dtype.  It deliberately materialises the dequantised pools, so it is a checking mode, not the decode
path: the decode path is ``SplitKExecutor`` (the HIP kernels).

``normalized_fwht`` (int2_reference.py:18-31) is the orthonormal Walsh-Hadamard transform over the
last dimension in fp32, stride 1 first, which the manager applies to CPU tensors
(qwen_sspa_attention.py:223-235, :1233-1234, :1286); on 128-wide GPU rows ``triton_fwht_128`` runs the
same stage order as one HIP launch.
"""
from __future__ import annotations

import torch

from .cache import ThreePrecisionCache


def normalized_fwht(x: torch.Tensor) -> torch.Tensor:
    """fp32 orthonormal FWHT over the last dimension (a power of two), on the tensor's device."""
    width = int(x.shape[-1])
    if width < 1 or width & (width - 1):
        raise ValueError("Hadamard head dimension must be a positive power of two")
    y = x.float().contiguous()
    span = 1
    while span < width:
        blocks = y.reshape(*y.shape[:-1], width // (2 * span), 2, span)
        lo, hi = blocks[..., 0, :], blocks[..., 1, :]
        y = torch.stack((lo + hi, lo - hi), dim=-2).reshape(y.shape)
        span *= 2
    return y * (width ** -0.5)


def _pool_payload(cache: ThreePrecisionCache, index: int, pool):
    """fp32 (K, V) of one pool, or None when it is empty."""
    n = pool.token_count
    if n == 0:
        return None
    if cache.compact_key is not None and index == 1 and cache.generated_value_precision == "int4":
        # static INT4 keys at their segment, generated ones after the static INT2 segment
        # (triton_fourq_attention.py:95-111)
        static = min(cache.static_int4_tokens, n)
        key = cache.compact_key.dequantize_range(cache.compact_key.segment_offsets[1], static)
        if n > static:
            key = torch.cat((key, cache.compact_key.dequantize_range(cache.generated_k_offset, n - static)), dim=1)
    elif cache.compact_key is not None and index < 3:
        key = cache.compact_key.dequantize_range(cache.compact_key.segment_offsets[index], n)
    elif pool.fp_k is not None:
        key = pool.fp_k[:, :n].float()
    else:
        key = None if pool.packed_k is None else pool.packed_k.dequantize().float()
    if pool.fp_v is not None:
        value = pool.fp_v[:, :n].float()
    else:
        value = None if pool.packed_v is None else pool.packed_v.dequantize().float()
    if key is None or value is None:
        raise ValueError(f"non-empty {pool.name} pool has incomplete payload")
    return key, value


def _softmax_state(q: torch.Tensor, key: torch.Tensor, value: torch.Tensor, scale: float):
    hq, hkv = int(q.shape[1]), int(key.shape[0])
    if hq % hkv:
        raise ValueError("GQA requires Hq divisible by Hkv")
    head_map = torch.arange(hq, device=q.device) // (hq // hkv)
    k, v = key.index_select(0, head_map), value.index_select(0, head_map)
    logits = torch.einsum("bhd,hsd->bhs", q, k) * scale
    peak = logits.amax(dim=-1)
    w = torch.exp(logits - peak.unsqueeze(-1))
    return peak, w.sum(dim=-1), torch.einsum("bhs,hsd->bhd", w, v)


def _merge(a, b):
    peak = torch.maximum(a[0], b[0])
    wa, wb = torch.exp(a[0] - peak), torch.exp(b[0] - peak)
    return peak, a[1] * wa + b[1] * wb, a[2] * wa.unsqueeze(-1) + b[2] * wb.unsqueeze(-1)


def triton_mixed_reference(query: torch.Tensor, cache: ThreePrecisionCache, *,
                           sm_scale: float | None = None) -> torch.Tensor:
    """fp32 dequantise-then-softmax attention of one decode token over every pool of ``cache``.

    ``query`` is [1, Hq, D] or [1, Hq, 1, D]; returns [1, Hq, D] in the query dtype."""
    if query.ndim == 4:
        if int(query.shape[2]) != 1:
            raise ValueError("query must have one decode token")
        query = query[:, :, 0]
    if query.ndim != 3 or int(query.shape[0]) != 1:
        raise ValueError("query must be [1,Hq,D]")
    scale = float(sm_scale) if sm_scale is not None else int(query.shape[-1]) ** -0.5
    q = query.float()
    state = None
    for index, pool in enumerate((cache.fp_pool, cache.int4_pool, cache.int2_pool, cache.recent_fp_pool)):
        payload = _pool_payload(cache, index, pool)
        if payload is None:
            continue
        part = _softmax_state(q, payload[0].to(q.device), payload[1].to(q.device), scale)
        state = part if state is None else _merge(state, part)
    if state is None:
        raise ValueError("four-quadrant cache has no surviving tokens")
    return (state[2] / state[1].unsqueeze(-1)).to(query.dtype)
