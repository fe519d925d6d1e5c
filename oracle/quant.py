"""numpy restatement of the reference quantisers and bit packers (test infrastructure only).

Every function follows the reference's torch CPU path operation by operation in IEEE fp32
(numpy float32 division is correctly rounded, ``np.rint`` rounds half to even like
``torch.round``, ``astype(np.float16)`` rounds to nearest even like ``.to(torch.float16)``).

Pinning (tests/test_oracle_quant.py, tests/test_oracle_golden.py):
  * golden fixtures written by the reference itself (tests/golden/*.npz): packed bytes,
    scales and zero points of all three quantisers, bit-exact;
  * known answers: constant blocks take the 1e-6 step clamp; all-positive blocks get zero
    point 0; +-absmax maps to codes +-7; exact .5 ties go to even; nibble and crumb order
    (low bits = lower channel);
  * round-trip bound |x - dequant(quant(x))| <= step/2 (+ fp16 scale rounding) in range.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32
EPS = F32(1e-6)


# ----------------------------------------------------------------------------- dtype helpers
def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """bfloat16 bit patterns (uint16) -> float32 (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns, round to nearest even (torch ``.to(bfloat16)``)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return rounded.astype(np.uint16)


def round_to_dtype(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round float32 values to ``dtype`` ('bfloat16' or 'float16') and back to float32."""
    if dtype == "bfloat16":
        return bf16_bits_to_f32(f32_to_bf16_bits(x))
    if dtype == "float16":
        return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)
    if dtype == "float32":
        return np.asarray(x, dtype=np.float32)
    raise ValueError(f"unsupported dtype {dtype}")


# ------------------------------------------------------------------------------ INT4 keys
def quantize_int4_key_per_channel(key: np.ndarray, superblock_size: int):
    """Per-channel affine INT4 over ``superblock_size``-token blocks.

    Follows compact_int4_key.py:83-110: mn = min(min x, 0), mx = max(max x, 0),
    step = max((mx - mn) / 15, 1e-6), zp = clamp(rne(-mn / step), 0, 15),
    code = clamp(rne(x / step + zp), 0, 15); scale stored as fp16(step), zero as u8(zp);
    byte j = code[2j] | code[2j+1] << 4.
    """
    if key.ndim != 3 or key.shape[2] % 2:
        raise ValueError("INT4 K must be [H,S,D] with even D")
    if superblock_size not in (32, 64, 128):
        raise ValueError("per-channel INT4 K superblock must be 32, 64, or 128 tokens")
    h, length, d = key.shape
    blocks = max(1, -(-length // superblock_size))
    scale = np.zeros((h, blocks, d), dtype=np.float16)
    zero = np.zeros((h, blocks, d), dtype=np.uint8)
    codes = np.zeros((h, length, d), dtype=np.uint8)
    x = np.asarray(key, dtype=F32)
    for block, start in enumerate(range(0, length, superblock_size)):
        src = x[:, start : start + superblock_size]
        mn = np.minimum(src.min(axis=1), F32(0))
        mx = np.maximum(src.max(axis=1), F32(0))
        step = np.maximum((mx - mn) / F32(15.0), EPS)
        zp = np.clip(np.rint(-mn / step), 0, 15).astype(F32)
        q = np.clip(np.rint(src / step[:, None, :] + zp[:, None, :]), 0, 15)
        codes[:, start : start + src.shape[1]] = q.astype(np.uint8)
        scale[:, block] = step.astype(np.float16)
        zero[:, block] = zp.astype(np.uint8)
    packed = (codes[..., 0::2] | (codes[..., 1::2] << 4)).astype(np.uint8)
    return packed, scale, zero


def dequantize_int4_key(packed, scale, zero, start: int, length: int, superblock_size: int):
    """``CompactInt4KeyArena.dequantize_range`` (compact_int4_key.py:175-195): (code - z) * f32(s)."""
    h = packed.shape[0]
    d = packed.shape[2] * 2
    if length == 0:
        return np.zeros((h, 0, d), dtype=F32)
    payload = packed[:, start : start + length]
    codes = np.stack((payload & 15, (payload >> 4) & 15), axis=-1).reshape(h, length, d)
    blocks = np.arange(start, start + length) // superblock_size
    s = scale[:, blocks].astype(F32)
    z = zero[:, blocks].astype(F32)
    return (codes.astype(F32) - z) * s


# ---------------------------------------------------------------------------- INT4 values
def quantize_int2_key_per_channel(key: np.ndarray, superblock_size: int):
    """Per-channel affine INT2 over ``superblock_size``-token blocks (OScaR form).

    Follows int2_reference.py:159-214 with clip_ratio 1: mn, mx = block min / max (no
    inclusion of 0); range = mx - mn; for range > 0: scale = range / 3, inv = (1 / range) * 3
    (how torch evaluates ``3.0 / range``),
    zero = rne(-mn * inv), offset = -zero * scale; for a constant channel scale = inv = zero = 0
    and offset = mn.  code = clamp(rne(x * inv + zero), 0, 3) (the product rounded to fp32
    before the add); scale and offset stored as fp16; byte j = c[4j] | c[4j+1] << 2 |
    c[4j+2] << 4 | c[4j+3] << 6.  Returns (packed [H,S,D/4] u8, scale, offset [H,blocks,D] f16).
    """
    if key.ndim != 3 or key.shape[2] % 4:
        raise ValueError("INT2 K must be [H,S,D] with D divisible by four")
    if superblock_size not in (32, 64, 128):
        raise ValueError("per-channel INT2 K block size must be 32, 64, or 128")
    h, length, d = key.shape
    blocks = max(1, -(-length // superblock_size))
    scale = np.zeros((h, blocks, d), dtype=np.float16)
    offset = np.zeros((h, blocks, d), dtype=np.float16)
    codes = np.zeros((h, length, d), dtype=np.uint8)
    x = np.asarray(key, dtype=F32)
    for block, start in enumerate(range(0, length, superblock_size)):
        src = x[:, start : start + superblock_size]
        mn = src.min(axis=1)
        mx = src.max(axis=1)
        rng = (mx - mn).astype(F32)
        nonconst = rng > 0
        with np.errstate(divide="ignore", invalid="ignore"):
            sc = np.where(nonconst, rng / F32(3.0), F32(0)).astype(F32)
            # torch evaluates ``3.0 / t`` as ``t.reciprocal() * 3.0`` (Tensor.__rtruediv__): two roundings
            recip = (F32(1.0) / np.maximum(rng, F32(1e-30))).astype(F32)
            inv = np.where(nonconst, (recip * F32(3.0)).astype(F32), F32(0)).astype(F32)
        zp = np.where(nonconst, np.rint(-mn * inv), F32(0)).astype(F32)
        off = np.where(nonconst, -zp * sc, mn).astype(F32)
        prod = (src * inv[:, None, :]).astype(F32)
        q = np.clip(np.rint((prod + zp[:, None, :]).astype(F32)), 0, 3)
        codes[:, start : start + src.shape[1]] = q.astype(np.uint8)
        scale[:, block] = sc.astype(np.float16)
        offset[:, block] = off.astype(np.float16)
    packed = (codes[..., 0::4] | (codes[..., 1::4] << 2) | (codes[..., 2::4] << 4)
              | (codes[..., 3::4] << 6)).astype(np.uint8)
    return packed, scale, offset


def dequantize_int2_key(packed, scale, offset, start: int, length: int, superblock_size: int):
    """``CompactInt2KeyArena.dequantize_range`` (compact_int2_key.py:69-96): code * f32(s) + f32(o)."""
    h = packed.shape[0]
    d = packed.shape[2] * 4
    if length == 0:
        return np.zeros((h, 0, d), dtype=F32)
    payload = packed[:, start : start + length]
    codes = np.stack([(payload >> (2 * i)) & 3 for i in range(4)], axis=-1).reshape(h, length, d)
    blocks = np.arange(start, start + length) // superblock_size
    return (codes.astype(F32) * scale[:, blocks].astype(F32)).astype(F32) + offset[:, blocks].astype(F32)


def quantize_int4_value(value: np.ndarray):
    """Per-token symmetric INT4 (quantization.py:19-50 with dim=2, packing :77-102).

    s = max(max_c |x| / 7, 1e-6) kept in fp32, q = clamp(rne(x / s), -7, 7), nibble = q & 15,
    pairs taken along the flattened C order (low nibble = even channel).
    Returns packed [H,S,D/2] u8 and scale [H,S,1] f32.
    """
    x = np.asarray(value, dtype=F32)
    amax = np.abs(x).max(axis=2, keepdims=True) if x.shape[1] else np.zeros(x.shape[:2] + (1,), F32)
    scale = np.maximum(amax / F32(7.0), EPS).astype(F32)
    q = np.clip(np.rint(x / scale), -7, 7).astype(np.int16)
    nib = (q & 15).astype(np.uint8)
    packed = (nib[..., 0::2] | (nib[..., 1::2] << 4)).astype(np.uint8)
    return packed, scale


def dequantize_int4_value(packed: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """``PackedTensor.dequantize`` for per-token INT4 (packed_kv_layout.py:30-32)."""
    lo = (packed & 15).astype(np.int16)
    hi = ((packed >> 4) & 15).astype(np.int16)
    lo = np.where(lo >= 8, lo - 16, lo)
    hi = np.where(hi >= 8, hi - 16, hi)
    h, s, d2 = packed.shape
    codes = np.stack((lo, hi), axis=-1).reshape(h, s, d2 * 2)
    return codes.astype(F32) * scale.astype(F32)


# ---------------------------------------------------------------------------- INT2 values
def quantize_int2_value(value: np.ndarray, group_size: int):
    """Per-token-group affine INT2 (int2_reference.py:96-151, axis='per_token_group').

    mn = min(min x, 0), mx = max(max x, 0), s = max((mx - mn) / 3, 1e-6) (fp32),
    z = clamp(rne(-mn / s), 0, 3), c = clamp(rne(x / s + z), 0, 3); store fp16(s), u8(z);
    byte j = c[4j] | c[4j+1] << 2 | c[4j+2] << 4 | c[4j+3] << 6.
    Returns packed [H,S,D/4] u8, scale [H,S,D/G,1] f16, zero [H,S,D/G,1] u8.
    """
    x = np.asarray(value, dtype=F32)
    h, s, d = x.shape
    if group_size <= 0 or d % group_size:
        raise ValueError("group_size must be positive and divide head_dim")
    groups = x.reshape(h, s, d // group_size, group_size)
    mn = np.minimum(groups.min(axis=3, keepdims=True) if s else np.zeros((h, 0, d // group_size, 1), F32), F32(0))
    mx = np.maximum(groups.max(axis=3, keepdims=True) if s else np.zeros((h, 0, d // group_size, 1), F32), F32(0))
    scale = np.maximum((mx - mn) / F32(3.0), EPS).astype(F32)
    zero = np.clip(np.rint(-mn / scale), 0, 3).astype(F32)
    codes = np.clip(np.rint(groups / scale + zero), 0, 3).astype(np.uint8).reshape(h, s, d)
    packed = (codes[..., 0::4] | (codes[..., 1::4] << 2) | (codes[..., 2::4] << 4) | (codes[..., 3::4] << 6))
    return packed.astype(np.uint8), scale.astype(np.float16), zero.astype(np.uint8)


def dequantize_int2_value(packed, scale, zero, group_size: int) -> np.ndarray:
    """``CompactInt2ValueArena.dequantize_range`` (fused_value_pack.py:450-472): (c - z) * f32(s)."""
    h, s, d4 = packed.shape
    d = d4 * 4
    codes = np.stack([(packed >> (2 * k)) & 3 for k in range(4)], axis=-1).reshape(h, s, d)
    grouped = codes.reshape(h, s, d // group_size, group_size).astype(F32)
    return ((grouped - zero.astype(F32)) * scale.astype(F32)).reshape(h, s, d)


# ---------------------------------------------------------------------------------- FWHT
def normalized_fwht(x: np.ndarray) -> np.ndarray:
    """Orthonormal Walsh-Hadamard transform over the last dim (int2_reference.py:18-31)."""
    out = np.array(x, dtype=F32, copy=True)
    width = out.shape[-1]
    if width < 1 or width & (width - 1):
        raise ValueError("Hadamard head dimension must be a positive power of two")
    stride = 1
    while stride < width:
        pair = out.reshape(out.shape[:-1] + (-1, 2, stride))
        left, right = pair[..., 0, :].copy(), pair[..., 1, :].copy()
        out = np.stack((left + right, left - right), axis=-2).reshape(out.shape)
        stride *= 2
    return out * F32(width ** -0.5)
