"""numpy restatement of the decode-step Qwen mRoPE (+ optional FWHT) — test infrastructure only.

Follows _qwen_qk_mrope_kernel (r2omni/sspa/kernels/triton_qwen_mrope.py:66-121): for every row,
value = x[d], rotated = -x[d + 64] for d < 64 and x[d - 64] otherwise, dimension d takes its
cos/sin from table axis 0, 1 or 2 by d % 64 against the sections, result = value * cos +
rotated * sin in fp32, then the normalized FWHT-128 when asked (int2_reference.py:18-31), then
one rounding to the output dtype.  fp32 arithmetic is done op by op (no fused multiply-add).

Pinning (tests/test_oracle_rope.py): identity tables give the input back; with standard
(duplicated-half) tables every (d, d + 64) pair is the complex product (x_d + i x_{d+64}) *
(cos_d + i sin_d) (float64 brute force); the section-to-axis rule equals the split/concatenate
formulation of transformers' apply_multimodal_rotary_pos_emb, restated independently.

``qwen3_norm_rope`` restates the Qwen3 branch of the decode step (qwen_sspa_attention.py:1228-1235),
whose operations come from transformers 5.15.0 (models/qwen3/modeling_qwen3.py: Qwen3RMSNorm.forward,
apply_rotary_pos_emb, rotate_half), op by op with the rounding of each torch op to the tensor dtype:
v = mean(x^2) (fp32), n = dtype(x * (1 / sqrt(v + eps))), w = dtype(weight * n),
y = dtype(dtype(w * cos) + dtype(rotate_half(w) * sin)), then the optional normalised FWHT rounded
to dtype (triton_fwht_128).  Pinned against those transformers functions evaluated by torch on the
CPU in bf16 and fp16 (tests/test_oracle_rope.py), plus the unit-weight, zero-angle case, which
reduces to a plain RMSNorm.
"""
from __future__ import annotations

import numpy as np

from .quant import normalized_fwht, round_to_dtype

F32 = np.float32


def qwen_mrope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, sections, *, hadamard: bool, dtype: str) -> np.ndarray:
    """x [B, H, T, 128] float32 (already in the input dtype's values); cos/sin [3, B, T, 128]."""
    x = np.asarray(x, dtype=F32)
    d = np.arange(128)
    half = d % 64
    axis = np.where(half < sections[0], 0, np.where(half < sections[0] + sections[1], 1, 2))
    c = np.asarray(cos, dtype=F32)[axis, :, :, d].transpose(1, 2, 0)[:, None]  # [B, 1, T, 128]
    s = np.asarray(sin, dtype=F32)[axis, :, :, d].transpose(1, 2, 0)[:, None]
    other = np.concatenate([x[..., 64:], x[..., :64]], axis=-1)
    rotated = np.where(d < 64, -other, other).astype(F32)
    out = (x * c).astype(F32) + (rotated * s).astype(F32)
    if hadamard:
        out = normalized_fwht(out.astype(F32))
    return round_to_dtype(out.astype(F32), dtype)


def qwen3_norm_rope(x: np.ndarray, weight: np.ndarray, cos: np.ndarray, sin: np.ndarray, *, eps: float,
                    hadamard: bool, dtype: str) -> np.ndarray:
    """x [B, H, T, 128], weight [128], cos/sin [B, T, 128]: values already in ``dtype``."""
    r = lambda v: round_to_dtype(np.asarray(v, dtype=F32), dtype)  # noqa: E731
    x = np.asarray(x, dtype=F32)
    var = (np.sum(x * x, axis=-1, keepdims=True, dtype=F32) / F32(128)).astype(F32)
    inv = (F32(1.0) / np.sqrt((var + F32(eps)).astype(F32))).astype(F32)
    n = r(x * inv)
    w = r(np.asarray(weight, dtype=F32) * n)
    c = np.asarray(cos, dtype=F32)[:, None]
    s = np.asarray(sin, dtype=F32)[:, None]
    rot = np.concatenate([-w[..., 64:], w[..., :64]], axis=-1)
    y = r(r(w * c) + r(rot * s))
    if hadamard:
        y = r(normalized_fwht(y.astype(F32)))
    return y
