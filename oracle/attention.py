"""torch-CPU fp32 restatement of the reference's dequantise-then-softmax oracle (test infrastructure only).

Follows ``triton_mixed_reference`` (r2omni/sspa/kernels/triton_fourq_attention.py:72-125):
for each non-empty pool in the order FP, INT4, INT2, Recent-FP, dequantise K and V to fp32,
form logits q.k * D^-1/2 with ``kv(h) = h // GQA`` (``_partial_state`` :41-55), keep the
per-pool (max, sum, weighted value sum) and merge them exactly (``_merge_state`` :58-69),
then divide.  The fused output transform of the split-K reduce
(triton_fourq_splitk.py:1000-1006) rounds to bf16, applies the orthonormal 128-point FWHT in
fp32 and rounds to bf16 again.

Pinning (tests/test_oracle_golden.py, tests/test_oracle_quant.py):
  * the reference's own outputs on three golden caches (before and after a flush);
  * brute force: a float64 softmax over the concatenated tokens with the GQA head map
    kv = h // GQA (reference tests/test_gqa_contract.py:6-13) equals the pool merge, and any
    partition of the tokens gives the same result (merge invariance);
  * FWHT: H.H = I and FWHT(e0) = 1/sqrt(128) * ones.
"""
from __future__ import annotations

import numpy as np
import torch

from .cache import OracleCache, pool_kv
from .quant import f32_to_bf16_bits, bf16_bits_to_f32, normalized_fwht


def partial_state(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, sm_scale: float):
    """(max, exp_sum, weighted_value_sum) of one pool; query [1,Hq,D], key/value [Hkv,S,D]."""
    hq, hkv = int(query.shape[1]), int(key.shape[0])
    if hq % hkv:
        raise ValueError("GQA requires Hq divisible by Hkv")
    kv_head = torch.arange(hq) // (hq // hkv)
    k = key.index_select(0, kv_head)
    v = value.index_select(0, kv_head)
    logits = torch.einsum("bhd,hsd->bhs", query.float(), k) * sm_scale
    m = logits.amax(dim=-1)
    w = torch.exp(logits - m.unsqueeze(-1))
    return m, w.sum(dim=-1), torch.einsum("bhs,hsd->bhd", w, v)


def merge_state(a, b):
    m = torch.maximum(a[0], b[0])
    wa = torch.exp(a[0] - m)
    wb = torch.exp(b[0] - m)
    return m, a[1] * wa + b[1] * wb, a[2] * wa.unsqueeze(-1) + b[2] * wb.unsqueeze(-1)


def attention_over_pools(query: np.ndarray, pools, sm_scale: float | None = None) -> np.ndarray:
    """Merged attention over a list of (K, V) float32 pools; query [1,Hq,D] -> float32 [1,Hq,D]."""
    q = torch.from_numpy(np.ascontiguousarray(query, dtype=np.float32))
    scale = float(sm_scale) if sm_scale is not None else int(q.shape[-1]) ** -0.5
    state = None
    for k, v in pools:
        part = partial_state(q, torch.from_numpy(np.ascontiguousarray(k, np.float32)),
                             torch.from_numpy(np.ascontiguousarray(v, np.float32)), scale)
        state = part if state is None else merge_state(state, part)
    if state is None:
        raise ValueError("four-quadrant cache has no surviving tokens")
    return (state[2] / state[1].unsqueeze(-1)).numpy()


def mixed_reference(query: np.ndarray, cache: OracleCache, *, append=None) -> np.ndarray:
    """fp32 attention of one request; ``append=(k, v)`` adds the fused-append token to Recent-FP.

    The fused append token takes part in the attention of the same call
    (triton_fourq_splitk.py:634-669: position == recent length is valid when DO_APPEND).
    """
    pools = pool_kv(cache)
    if append is not None:
        ak = np.asarray(append[0], np.float32).reshape(cache.hkv, 1, -1)
        av = np.asarray(append[1], np.float32).reshape(cache.hkv, 1, -1)
        if cache.recent_active:
            rk, rv = pools[-1]
            pools[-1] = (np.concatenate((rk, ak), axis=1), np.concatenate((rv, av), axis=1))
        else:
            pools.append((ak, av))
    return attention_over_pools(query, pools)


def output_transform(out: np.ndarray, hadamard: bool) -> np.ndarray:
    """bf16 output of the split-K reduce; with ``hadamard`` bf16 -> FWHT128 -> bf16 (as float32 values)."""
    y = bf16_bits_to_f32(f32_to_bf16_bits(out))
    if hadamard:
        y = bf16_bits_to_f32(f32_to_bf16_bits(normalized_fwht(y)))
    return y
