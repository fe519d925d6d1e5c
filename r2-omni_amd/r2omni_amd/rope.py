"""Decode-step query/key transforms on the gfx950 HIP kernels.

* ``qwen_qk_mrope`` (``r2o_qk_mrope``): drop-in for ``r2omni.sspa.kernels.triton_qwen_mrope.qwen_qk_mrope``
  (triton_qwen_mrope.py:214-322): same arguments, same validation messages, one launch for every
  (request, head, token) row.
* ``qwen3_qk_norm_rope`` (``r2o_qk_norm_rope``): the Qwen3 branch of the same step
  (qwen_sspa_attention.py:1228-1235: ``q_norm`` / ``k_norm``, ``apply_rotary_pos_emb``, then
  ``triton_fwht_128`` of Q and K when keys are Hadamard-rotated) in one launch, with the rounding of
  every torch op of that sequence.
* ``FusedRotary`` / ``FusedQwen3Rotary``: either transform folded into the split-K call itself
  (``executor(q, append=..., rotary=...)``), so that the step's attention is two launches.
"""
from __future__ import annotations

import ctypes
from collections.abc import Sequence
from dataclasses import dataclass

import torch

from . import _lib

_TABLE_CODES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


@dataclass(frozen=True)
class FusedRotary:
    """The decode step's Qwen mRoPE, folded into the split-K call.

    Given to ``SplitKExecutor.__call__(query, append, rotary=...)`` or ``BatchedDecoder(...,
    rotary=...)``, the query and the appended key and value are the raw projections, and the partial
    kernel applies what ``qwen_qk_mrope(q, k, cos, sin, mrope_section, apply_hadamard=...)`` and the
    manager's value Hadamard (``triton_fwht_128(v)`` when ``value_hadamard``) would (qwen_sspa_attention.py:
    1239-1247, 230-235; triton_qwen_mrope.py:45-124), bit-identically, without their launch; the rotated
    appended rows reach the ring through the fused append.  ``cos`` / ``sin``: [3, B, T, 128] tables of
    the step (token 0 is used), bf16, fp16 or fp32, with unit channel stride and 16-byte aligned
    (axis, request) rows, such as contiguous tables or a token slice of them.  Under a captured graph the tables' storage is read at every replay: write
    each step's values into the same tensors."""
    cos: torch.Tensor
    sin: torch.Tensor
    mrope_section: tuple
    apply_hadamard: bool = False
    value_hadamard: bool = False

    def fill(self, p: _lib.DecodeParams, batch: int, device: torch.device) -> None:
        """Write the rotation into the launch arguments (checks as ``qwen_qk_mrope``'s)."""
        cos, sin = self.cos, self.sin
        if cos.shape != sin.shape or cos.ndim != 4 or int(cos.shape[0]) != 3 or int(cos.shape[-1]) != 128:
            raise ValueError("Qwen fused mRoPE requires cos/sin [3,B,S,D]")
        if int(cos.shape[1]) != batch or int(cos.shape[2]) < 1:
            raise ValueError("Qwen fused mRoPE rotary positions must match Q/K tokens")
        if cos.device != device or sin.device != device:
            raise ValueError("Q/K and rotary tensors must share a device")
        if cos.dtype != sin.dtype or cos.dtype not in _TABLE_CODES:
            raise ValueError("Qwen fused mRoPE cos/sin must share a bf16, fp16 or fp32 dtype")
        sections = tuple(int(v) for v in self.mrope_section)
        if len(sections) != 3 or sum(sections) != 64:
            raise ValueError("Qwen mRoPE sections must contain three values summing to 64")
        if min(sections) < 0:
            raise ValueError("Qwen mRoPE sections must be non-negative")
        esize = cos.element_size()
        piece = 16 // esize
        for t in (cos, sin):  # the kernel reads 16-byte pieces at 32-bit byte offsets from a request's base
            st = t.stride()
            if min(st) < 0 or st[3] != 1 or st[0] % piece or st[1] % piece or t.data_ptr() % 16:
                raise ValueError("Qwen fused mRoPE tables need unit channel stride and 16-byte aligned "
                                 "rows (e.g. contiguous [3, B, T, 128] tables)")
            if (2 * st[0] + 128) * esize >= 1 << 31:
                raise ValueError("Qwen fused mRoPE tables must span less than 2 GiB per request")
        p.rope_mode = 1
        p.rope_cos, p.rope_sin = cos.data_ptr(), sin.data_ptr()
        for i in range(4):
            p.rope_cos_strides[i] = int(cos.stride(i))
            p.rope_sin_strides[i] = int(sin.stride(i))
        p.rope_table_dtype = _TABLE_CODES[cos.dtype]
        p.rope_section0, p.rope_section1 = sections[0], sections[1]
        p.rope_hadamard = int(bool(self.apply_hadamard))
        p.value_hadamard = int(bool(self.value_hadamard))


@dataclass(frozen=True)
class FusedQwen3Rotary:
    """The Qwen3 branch of the decode step, folded into the split-K call.

    Given as ``rotary=`` like ``FusedRotary``: the query and the appended key are the raw projections,
    and the partial kernel applies what ``qwen3_qk_norm_rope(q, k, q_norm_weight, k_norm_weight, cos, sin,
    eps=eps, apply_hadamard=...)`` and the value Hadamard (``value_hadamard``) would
    (qwen_sspa_attention.py:1228-1235, 230-235), bit-identically, without their launch.  ``cos`` /
    ``sin``: [B or 1, T, 128] tables of the step in the rows' dtype (token 0 is used), unit channel
    stride and 16-byte aligned rows; the norm weights [128] in the rows' dtype."""
    cos: torch.Tensor
    sin: torch.Tensor
    q_norm_weight: torch.Tensor
    k_norm_weight: torch.Tensor
    eps: float = 1e-6
    apply_hadamard: bool = False
    value_hadamard: bool = False

    def fill(self, p: _lib.DecodeParams, batch: int, device: torch.device) -> None:
        """Write the rotation into the launch arguments (checks as ``qwen3_qk_norm_rope``'s)."""
        cos, sin = self.cos, self.sin
        if cos.shape != sin.shape or cos.ndim != 3 or int(cos.shape[-1]) != 128 or int(cos.shape[1]) < 1 \
                or int(cos.shape[0]) not in (1, batch):
            raise ValueError("Qwen3 fused norm+RoPE requires cos/sin [B,S,D] matching Q/K tokens")
        if cos.device != device or sin.device != device:
            raise ValueError("Q/K and rotary tensors must share a device")
        code = _lib.dtype_code(cos.dtype) if cos.dtype in (torch.bfloat16, torch.float16) else -1
        if cos.dtype != sin.dtype or code != p.row_dtype:
            raise ValueError("Qwen3 fused norm+RoPE cos/sin must share the Q/K dtype and device")
        for name, w in (("q_norm_weight", self.q_norm_weight), ("k_norm_weight", self.k_norm_weight)):
            if tuple(w.shape) != (128,) or w.dtype != cos.dtype or w.device != device:
                raise ValueError(f"{name} must be a [128] tensor of the Q/K dtype on the Q/K device")
            if not w.is_contiguous() or w.data_ptr() % 16:
                raise ValueError(f"{name} must be contiguous and 16-byte aligned")
        if not self.eps >= 0.0:
            raise ValueError("RMSNorm epsilon must be non-negative")
        for t in (cos, sin):  # the kernel reads 16-byte pieces at 32-bit byte offsets from a request's base
            st = t.stride()
            if st[2] != 1 or min(st) < 0 or st[1] % 8 or (int(t.shape[0]) > 1 and st[0] % 8) or t.data_ptr() % 16:
                raise ValueError("Qwen3 fused norm+RoPE tables need unit channel stride and 16-byte aligned "
                                 "rows (e.g. contiguous [B, T, 128] tables)")
        p.rope_mode = 2
        p.rope_cos, p.rope_sin = cos.data_ptr(), sin.data_ptr()
        for t, dst in ((cos, p.rope_cos_strides), (sin, p.rope_sin_strides)):
            # as a [1, B, T, 128] view: one axis; a table shared by the batch has batch stride 0
            st = t.stride()
            dst[0], dst[1], dst[2], dst[3] = 0, (int(st[0]) if int(t.shape[0]) > 1 else 0), int(st[1]), 1
        p.rope_table_dtype = code
        p.rope_section0, p.rope_section1 = 64, 0
        p.rope_hadamard = int(bool(self.apply_hadamard))
        p.value_hadamard = int(bool(self.value_hadamard))
        p.q_norm_weight, p.k_norm_weight = self.q_norm_weight.data_ptr(), self.k_norm_weight.data_ptr()
        p.norm_eps = float(self.eps)


def _value_operands(value, output, apply_hadamard, what):
    """(V input, V output, whether the launch transforms V) for the optional V of a fused rotation:
    V takes the FWHT only under the Hadamard, and otherwise is returned (or copied into the caller's
    output by ``_copy_value``, once every argument has been checked) unchanged.  Writes nothing."""
    if output is not None and len(output) != (2 if value is None else 3):
        raise ValueError(f"{what} output must hold one tensor per input")
    if value is None:
        return None, None, False
    fold_v = bool(apply_hadamard)
    if fold_v:
        value = value.contiguous()
    if output is None:
        return value, (torch.empty_like(value) if fold_v else value), fold_v
    value_out = output[2]
    if value_out.shape != value.shape or value_out.device != value.device or value_out.dtype != value.dtype \
            or (fold_v and not value_out.is_contiguous()):
        raise ValueError(f"{what} value output must match V" + (" and be contiguous" if fold_v else ""))
    return value, value_out, fold_v


def _copy_value(value, value_out, fold_v) -> None:
    """Without the Hadamard, V reaches the caller's output buffer as a plain copy."""
    if value is not None and not fold_v and value_out is not value:
        value_out.copy_(value)


def qwen_qk_mrope(query: torch.Tensor, key: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                  mrope_section: Sequence[int], *, output: tuple[torch.Tensor, ...] | None = None,
                  apply_hadamard: bool = False, value: torch.Tensor | None = None):
    """Apply Qwen multimodal RoPE (and optionally the orthonormal FWHT-128) to Q and K in one launch.

    With ``value`` ([B, Hkv, T, 128], Q/K's dtype), returns (Q, K, V) and, when ``apply_hadamard``
    is set, folds the decode step's V Hadamard (``triton_fwht_128(value)``,
    qwen_sspa_attention.py:230-235) into the same launch; without it V is returned unchanged, as the
    manager rotates V only under Hadamard.  ``output`` then holds three tensors."""
    if query.ndim != 4 or key.ndim != 4:
        raise ValueError("Qwen fused mRoPE requires rank-4 Q/K")
    if query.shape[0] != key.shape[0]:
        raise ValueError("Qwen fused mRoPE requires equal Q/K batch sizes")
    if query.shape[2] <= 0 or key.shape[2] != query.shape[2]:
        raise ValueError("Qwen fused mRoPE requires equal positive Q/K token counts")
    if query.shape[-1] != 128 or key.shape[-1] != 128:
        raise ValueError("Qwen fused mRoPE currently requires head_dim=128")
    if query.device != key.device or query.dtype != key.dtype:
        raise ValueError("Q/K device and dtype must match")
    if cos.device != query.device or sin.device != query.device:
        raise ValueError("Q/K and rotary tensors must share a device")
    if cos.shape != sin.shape or cos.ndim != 4 or cos.shape[0] != 3:
        raise ValueError("Qwen fused mRoPE requires cos/sin [3,B,S,D]")
    tokens = int(query.shape[2])
    batch_size = int(query.shape[0])
    if cos.shape[1] != batch_size or cos.shape[-2:] != (tokens, 128):
        raise ValueError("Qwen fused mRoPE rotary positions must match Q/K tokens")
    sections = tuple(int(value) for value in mrope_section)
    if len(sections) != 3 or sum(sections) != 64:
        raise ValueError("Qwen mRoPE sections must contain three values summing to 64")
    if min(sections) < 0:
        raise ValueError("Qwen mRoPE sections must be non-negative")
    _lib.require_device(query, "fused Qwen mRoPE input")
    dtype = _lib.dtype_code(query.dtype)
    if cos.dtype != sin.dtype or cos.dtype not in _TABLE_CODES:
        raise ValueError("Qwen fused mRoPE cos/sin must share a bf16, fp16 or fp32 dtype")
    if value is not None:
        if value.shape != key.shape or value.device != key.device or value.dtype != key.dtype:
            raise ValueError("fused Qwen mRoPE value must match K's shape, device and dtype")
    query = query.contiguous()
    key = key.contiguous()
    value, value_out, fold_v = _value_operands(value, output, apply_hadamard, "fused Qwen mRoPE")
    if output is None:
        query_out, key_out = torch.empty_like(query), torch.empty_like(key)
    else:
        query_out, key_out = output[0], output[1]
        if query_out.shape != query.shape or key_out.shape != key.shape:
            raise ValueError("fused Qwen mRoPE output shapes must match Q/K")
        if (query_out.device != query.device or key_out.device != key.device or query_out.dtype != query.dtype
                or key_out.dtype != key.dtype):
            raise ValueError("fused Qwen mRoPE outputs must match Q/K device and dtype")
        if not query_out.is_contiguous() or not key_out.is_contiguous():
            raise ValueError("fused Qwen mRoPE outputs must be contiguous")
    cos_strides = (ctypes.c_int64 * 4)(*[int(v) for v in cos.stride()])
    sin_strides = (ctypes.c_int64 * 4)(*[int(v) for v in sin.stride()])
    _copy_value(value, value_out, fold_v)
    _lib.call("r2o_qkv_mrope", _lib.ptr(query), _lib.ptr(key), _lib.ptr(value) if fold_v else None,
              _lib.ptr(query_out), _lib.ptr(key_out), _lib.ptr(value_out) if fold_v else None, dtype,
              batch_size, int(query.shape[1]), int(key.shape[1]), tokens, _lib.ptr(cos), _lib.ptr(sin),
              _TABLE_CODES[cos.dtype], cos_strides, sin_strides, sections[0], sections[1], int(bool(apply_hadamard)),
              ctypes.c_void_p(_lib.stream_of(query.device)))
    if value is None:
        return query_out, key_out
    return query_out, key_out, value_out


def qwen3_qk_norm_rope(query: torch.Tensor, key: torch.Tensor, q_norm_weight: torch.Tensor,
                       k_norm_weight: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, *, eps: float = 1e-6,
                       apply_hadamard: bool = False, output: tuple[torch.Tensor, ...] | None = None,
                       value: torch.Tensor | None = None):
    """``q_norm(q)``, ``k_norm(k)`` (Qwen3 per-head RMSNorm), ``apply_rotary_pos_emb`` with
    ``cos``/``sin`` [B or 1, T, 128] and, with ``apply_hadamard``, the normalised FWHT-128 of both,
    in one launch.  Q [B, Hq, T, 128] and K [B, Hkv, T, 128] share one dtype (bf16 or fp16) with the
    norm weights and the rotary tables, as in the model.  With ``value`` ([B, Hkv, T, 128]), returns
    (Q, K, V), folding the V Hadamard into the launch as ``qwen_qk_mrope(value=...)`` does."""
    if query.ndim != 4 or key.ndim != 4:
        raise ValueError("Qwen3 fused norm+RoPE requires rank-4 Q/K")
    if query.shape[0] != key.shape[0] or query.shape[2] != key.shape[2] or query.shape[2] <= 0:
        raise ValueError("Qwen3 fused norm+RoPE requires equal Q/K batch sizes and positive token counts")
    if query.shape[-1] != 128 or key.shape[-1] != 128:
        raise ValueError("Qwen3 fused norm+RoPE currently requires head_dim=128")
    if query.device != key.device or query.dtype != key.dtype:
        raise ValueError("Q/K device and dtype must match")
    batch_size, tokens = int(query.shape[0]), int(query.shape[2])
    for name, w in (("q_norm_weight", q_norm_weight), ("k_norm_weight", k_norm_weight)):
        if w.shape != (128,) or w.dtype != query.dtype or w.device != query.device:
            raise ValueError(f"{name} must be a [128] tensor of the Q/K dtype on the Q/K device")
    if cos.shape != sin.shape or cos.ndim != 3 or cos.shape[-2:] != (tokens, 128) \
            or int(cos.shape[0]) not in (1, batch_size):
        raise ValueError("Qwen3 fused norm+RoPE requires cos/sin [B,S,D] matching Q/K tokens")
    if cos.dtype != query.dtype or sin.dtype != query.dtype or cos.device != query.device \
            or sin.device != query.device:
        raise ValueError("Qwen3 fused norm+RoPE cos/sin must share the Q/K dtype and device")
    if not eps >= 0.0:
        raise ValueError("RMSNorm epsilon must be non-negative")
    _lib.require_device(query, "fused Qwen3 norm+RoPE input")
    dtype = _lib.dtype_code(query.dtype)
    if value is not None and (value.shape != key.shape or value.device != key.device or value.dtype != key.dtype):
        raise ValueError("fused Qwen3 norm+RoPE value must match K's shape, device and dtype")
    query, key = query.contiguous(), key.contiguous()
    q_norm_weight, k_norm_weight = q_norm_weight.contiguous(), k_norm_weight.contiguous()
    cos, sin = cos.expand(batch_size, tokens, 128), sin.expand(batch_size, tokens, 128)
    value, value_out, fold_v = _value_operands(value, output, apply_hadamard, "fused Qwen3 norm+RoPE")
    if output is None:
        query_out, key_out = torch.empty_like(query), torch.empty_like(key)
    else:
        query_out, key_out = output[0], output[1]
        if query_out.shape != query.shape or key_out.shape != key.shape or query_out.dtype != query.dtype \
                or key_out.dtype != key.dtype or query_out.device != query.device or key_out.device != key.device:
            raise ValueError("fused Qwen3 norm+RoPE outputs must match Q/K shape, dtype and device")
        if not query_out.is_contiguous() or not key_out.is_contiguous():
            raise ValueError("fused Qwen3 norm+RoPE outputs must be contiguous")
    cos_strides = (ctypes.c_int64 * 3)(*[int(v) for v in cos.stride()])
    sin_strides = (ctypes.c_int64 * 3)(*[int(v) for v in sin.stride()])
    _copy_value(value, value_out, fold_v)
    _lib.call("r2o_qkv_norm_rope", _lib.ptr(query), _lib.ptr(key), _lib.ptr(value) if fold_v else None,
              _lib.ptr(query_out), _lib.ptr(key_out), _lib.ptr(value_out) if fold_v else None, dtype,
              batch_size, int(query.shape[1]), int(key.shape[1]), tokens, _lib.ptr(q_norm_weight),
              _lib.ptr(k_norm_weight), float(eps), _lib.ptr(cos), _lib.ptr(sin), cos_strides, sin_strides,
              int(bool(apply_hadamard)), ctypes.c_void_p(_lib.stream_of(query.device)))
    if value is None:
        return query_out, key_out
    return query_out, key_out, value_out
