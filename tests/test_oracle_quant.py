"""Known-answer and invariant checks that pin the CPU oracle independently of the fixtures."""
import numpy as np
import torch

from oracle.attention import attention_over_pools, merge_state, output_transform, partial_state
from oracle.cache import append_token, build_cache, compact_page_layouts
from oracle.quant import (
    bf16_bits_to_f32,
    dequantize_int2_key,
    dequantize_int2_value,
    dequantize_int4_key,
    dequantize_int4_value,
    f32_to_bf16_bits,
    normalized_fwht,
    quantize_int2_key_per_channel,
    quantize_int2_value,
    quantize_int4_key_per_channel,
    quantize_int4_value,
)


def test_int4_key_constant_block_takes_step_clamp():
    x = np.zeros((1, 32, 4), np.float32)
    packed, scale, zero = quantize_int4_key_per_channel(x, 32)
    assert np.all(scale.astype(np.float32) == np.float16(np.float32(1e-6)).astype(np.float32))
    assert np.all(zero == 0) and np.all(packed == 0)


def test_int4_key_all_positive_block_has_zero_point_zero_and_top_code():
    x = np.tile(np.linspace(1.0, 15.0, 32, dtype=np.float32)[None, :, None], (1, 1, 2))
    packed, scale, zero = quantize_int4_key_per_channel(x, 32)
    assert np.all(zero == 0)
    assert np.all(scale.astype(np.float32) == 1.0)  # (15 - 0) / 15
    codes = packed & 15
    assert codes[0, -1, 0] == 15 and codes[0, 0, 0] == 1


def test_int4_key_nibble_order_low_bits_are_even_channel():
    x = np.zeros((1, 32, 2), np.float32)
    x[0, :, 0] = 15.0
    x[0, :, 1] = 0.0
    x[0, 0, 1] = 15.0  # channel 1 gets range [0, 15] so its zero point is 0 too
    packed, _, _ = quantize_int4_key_per_channel(x, 32)
    assert packed[0, 0, 0] == 0xFF and packed[0, 1, 0] == 0x0F


def test_int2_key_constant_channel_keeps_its_value_as_offset():
    # OScaR form: a constant channel has scale 0 and offset = the value (no 1e-6 clamp, no zero point)
    x = np.full((1, 32, 4), 2.5, np.float32)
    x[0, :, 1] = -0.75
    packed, scale, offset = quantize_int2_key_per_channel(x, 32)
    assert np.all(scale == 0) and np.all(packed == 0)
    np.testing.assert_array_equal(offset[0, 0].astype(np.float32), [2.5, -0.75, 2.5, 2.5])
    np.testing.assert_array_equal(dequantize_int2_key(packed, scale, offset, 0, 32, 32), x)


def test_int2_key_range_endpoints_and_crumb_order():
    # channel c of token t takes the value (t + c) % 4 on a range [0, 3] (0 is not forced into the
    # range: [1, 4] gives offset 1), so every code is exact and lands in crumb c % 4 of byte c // 4
    t = np.arange(32)[:, None]
    c = np.arange(8)[None, :]
    codes = (t + c) % 4
    x = codes.astype(np.float32)[None]
    packed, scale, offset = quantize_int2_key_per_channel(x, 32)
    assert np.all(scale.astype(np.float32) == 1.0) and np.all(offset == 0)
    want = (codes[:, 0::4] | codes[:, 1::4] << 2 | codes[:, 2::4] << 4 | codes[:, 3::4] << 6).astype(np.uint8)
    np.testing.assert_array_equal(packed[0], want)
    shifted = x + 1.0  # [1, 4]: zero = rne(-1 * 1) -> -1 ... the offset carries the shift exactly
    p2, s2, o2 = quantize_int2_key_per_channel(shifted, 32)
    np.testing.assert_array_equal(dequantize_int2_key(p2, s2, o2, 0, 32, 32), shifted)


def test_int2_key_round_trip_bound():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((2, 96, 128)) * 3).astype(np.float32)
    packed, scale, offset = quantize_int2_key_per_channel(x, 32)
    deq = dequantize_int2_key(packed, scale, offset, 0, 96, 32)
    s32 = np.repeat(scale.astype(np.float32), 32, axis=1)
    # half a step plus the fp16 rounding of scale (3 codes) and offset
    slack = 0.5 * s32 + 3 * np.abs(s32) * 2.0 ** -10 + np.abs(np.repeat(offset.astype(np.float32), 32, axis=1)) * 2.0 ** -10
    assert np.all(np.abs(deq - x) <= slack + 1e-6)


def test_int4_value_absmax_maps_to_plus_minus_seven_and_ties_to_even():
    x = np.zeros((1, 1, 128), np.float32)
    x[0, 0, 0] = 7.0
    x[0, 0, 1] = -7.0
    x[0, 0, 2] = 2.5   # 2.5 / 1 -> ties to even -> 2
    x[0, 0, 3] = 3.5   # -> 4
    packed, scale = quantize_int4_value(x)
    assert scale[0, 0, 0] == 1.0
    assert packed[0, 0, 0] == (7 | ((-7 & 15) << 4))
    assert packed[0, 0, 1] == (2 | (4 << 4))
    deq = dequantize_int4_value(packed, scale)
    assert deq[0, 0, 0] == 7.0 and deq[0, 0, 1] == -7.0


def test_int2_value_crumb_order_and_include_zero_rule():
    # all-positive group [10, 11]: the calibrated range must include 0
    x = np.full((1, 1, 32), 10.0, np.float32)
    x[0, 0, 1] = 11.0
    packed, scale, zero = quantize_int2_value(x, 32)
    assert zero[0, 0, 0, 0] == 0
    assert scale.astype(np.float32)[0, 0, 0, 0] == np.float16(np.float32(11.0) / np.float32(3.0)).astype(np.float32)
    # 10 / (11/3) = 2.727 -> 3 ; 11 -> 3 ; crumbs 3,3,3,3 -> 0xFF
    assert packed[0, 0, 0] == 0xFF
    y = np.zeros((1, 1, 32), np.float32)
    y[0, 0, 0:4] = [0.0, 1.0, 2.0, 3.0]
    p2, s2, z2 = quantize_int2_value(y, 32)
    assert s2[0, 0, 0, 0] == 1.0 and z2[0, 0, 0, 0] == 0
    assert p2[0, 0, 0] == (0 | (1 << 2) | (2 << 4) | (3 << 6))


def test_round_trip_bounds():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((2, 96, 128)).astype(np.float32)
    p, s, z = quantize_int4_key_per_channel(x, 32)
    deq = dequantize_int4_key(p, s, z, 0, 96, 32)
    step = s.astype(np.float32)[:, np.arange(96) // 32]
    # fp16 scale rounding adds at most 2^-11 relative per code step (codes <= 15)
    assert np.all(np.abs(deq - x) <= step * (0.5 + 16 * 2.0 ** -11) + 1e-6)
    p4, s4 = quantize_int4_value(x)
    assert np.all(np.abs(dequantize_int4_value(p4, s4) - x) <= s4 / 2 + 1e-6)
    p2, s2, z2 = quantize_int2_value(x, 32)
    deq2 = dequantize_int2_value(p2, s2, z2, 32)
    st = np.repeat(s2.astype(np.float32)[..., 0], 32, axis=2)
    assert np.all(np.abs(deq2 - x) <= st * (0.5 + 4 * 2.0 ** -11) + 1e-6)


def test_bf16_round_to_nearest_even():
    vals = np.array([1.0, 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, -2.5], np.float32)
    got = bf16_bits_to_f32(f32_to_bf16_bits(vals))
    ref = torch.tensor(vals).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(got, ref)


def test_fwht_is_orthonormal_and_maps_e0_to_constant():
    e0 = np.zeros((1, 128), np.float32)
    e0[0, 0] = 1
    np.testing.assert_allclose(normalized_fwht(e0), np.full((1, 128), 128 ** -0.5), rtol=1e-6)
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 128)).astype(np.float32)
    np.testing.assert_allclose(normalized_fwht(normalized_fwht(x)), x, atol=1e-5)
    # Sylvester matrix
    h = np.array([[1.0]])
    while h.shape[0] < 128:
        h = np.block([[h, h], [h, -h]])
    np.testing.assert_allclose(normalized_fwht(x), x @ h.T / np.sqrt(128), atol=1e-5)


def test_pool_merge_equals_single_softmax_and_is_partition_invariant():
    rng = np.random.default_rng(2)
    q = rng.standard_normal((1, 8, 128)).astype(np.float32)
    k = rng.standard_normal((2, 50, 128)).astype(np.float32)
    v = rng.standard_normal((2, 50, 128)).astype(np.float32)
    whole = attention_over_pools(q, [(k, v)])
    parts = attention_over_pools(q, [(k[:, :7], v[:, :7]), (k[:, 7:31], v[:, 7:31]), (k[:, 31:], v[:, 31:])])
    np.testing.assert_allclose(parts, whole, atol=1e-6)
    # brute force in float64 with the GQA map kv = h // 4
    logits = np.einsum("hd,hsd->hs", q[0].astype(np.float64), np.repeat(k, 4, axis=0)) / np.sqrt(128)
    w = np.exp(logits - logits.max(-1, keepdims=True))
    brute = np.einsum("hs,hsd->hd", w / w.sum(-1, keepdims=True), np.repeat(v, 4, axis=0))
    np.testing.assert_allclose(whole[0], brute, atol=1e-5)


def test_token_order_partition_is_stable_by_tier():
    offsets = np.array([0, 32, 50, 82, 100])
    lengths = np.array([32, 18, 32, 18, 5])
    classes = np.array([5, 1, 2, 4, 5])  # INT2, FP, INT4, PROTECTED(FP), INT2
    fp, i4, i2, ev = compact_page_layouts(offsets, lengths, classes)
    np.testing.assert_array_equal(fp, np.r_[np.arange(32, 50), np.arange(82, 100)])
    np.testing.assert_array_equal(i4, np.arange(50, 82))
    np.testing.assert_array_equal(i2, np.r_[np.arange(0, 32), np.arange(100, 105)])
    assert len(ev) == 0


def test_ring_invariants_match_reference_cache_test():
    # reference tests/test_active_cache_storage.py:72-94: 129 appends on a 128-token ring
    rng = np.random.default_rng(3)
    key = rng.standard_normal((2, 128, 128)).astype(np.float32).astype(np.float16).astype(np.float32)
    offsets = np.arange(4) * 32
    lengths = np.full(4, 32)
    classes = np.array([1, 2, 5, 0])
    c = build_cache(key, key, offsets, lengths, classes, dtype="float16", append_capacity=1024)
    tok = rng.standard_normal((2, 128)).astype(np.float32)
    for i in range(129):
        append_token(c, tok, tok, global_index=128 + i, logical_position=128 + i)
    assert c.flushed_tokens == 128 and c.recent_active == 1
    assert c.pool_tokens[2] == 32 + 128 and c.k_active == 96 + 128


def _bf16_values(rng, shape):
    return bf16_bits_to_f32(f32_to_bf16_bits(rng.standard_normal(shape).astype(np.float32)))


def test_generated_int4_values_reassemble_the_int4_pool():
    """``generated_value_precision="int4"``: the same appends as the released INT2 mode leave the K
    arena byte-identical (only the V tier differs, dynamic_fourq_cache.py:207-224); the INT4 pool
    grows by the flushed tokens, whose keys are the K arena rows after the static INT2 segment (the
    rows the INT2 mode adds to its INT2 pool) and whose values are the per-token INT4 round trip of
    the flushed rows, fp32 (fused_value_pack.py:241-256); the static INT4 values stay those of the
    build, unrounded; the INT2 pool keeps its static tokens."""
    rng = np.random.default_rng(11)
    h, s = 2, 256
    key, value = _bf16_values(rng, (h, s, 128)), _bf16_values(rng, (h, s, 128))
    offsets, lengths = np.arange(8) * 32, np.full(8, 32)
    classes = np.array([1, 2, 5, 2, 0, 5, 2, 4])  # FP 64, INT4 96, INT2 64, evicted 32
    rows_k, rows_v = _bf16_values(rng, (130, h, 128)), _bf16_values(rng, (130, h, 128))
    caches = {}
    for mode in ("int2", "int4"):
        c = build_cache(key, value, offsets, lengths, classes, dtype="bfloat16", append_capacity=260,
                        gen_values=mode)
        for i in range(130):
            append_token(c, rows_k[i], rows_v[i], global_index=s + i, logical_position=s + i)
        caches[mode] = c
    c2, c4 = caches["int2"], caches["int4"]
    for f in ("k_packed", "k_scale", "k_zero"):
        np.testing.assert_array_equal(getattr(c2, f), getattr(c4, f))
    assert c2.k_active == c4.k_active == 224 + 128
    assert c2.pool_tokens == [64, 96, 64 + 128] and c4.pool_tokens == [64, 96 + 128, 64]
    assert c4.static_i4 == 96 and c4.gen_k_offset == 224 and c4.v4_capacity == 96 + 260
    assert c2.v2_capacity == 384 and c4.v2_capacity == 128  # the INT2-V arena gets no append room
    p2, p4 = pool_kv_by_tier(c2), pool_kv_by_tier(c4)
    np.testing.assert_array_equal(p4["int4"][0][:, :96], p2["int4"][0])
    np.testing.assert_array_equal(p4["int4"][0][:, 96:], p2["int2"][0][:, 64:])
    np.testing.assert_array_equal(p4["int2"][0], p2["int2"][0][:, :64])
    np.testing.assert_array_equal(p4["int2"][1], p2["int2"][1][:, :64])
    flushed = np.transpose(rows_v[:128], (1, 0, 2))
    np.testing.assert_array_equal(p4["int4"][1][:, 96:], dequantize_int4_value(*quantize_int4_value(flushed)))
    static_v = dequantize_int4_value(*quantize_int4_value(value[:, np.r_[32:64, 96:128, 192:224]]))  # INT4 pages
    np.testing.assert_array_equal(p4["int4"][1][:, :96], static_v)
    assert not np.array_equal(p2["int4"][1], static_v)  # the released INT4 pool rounds to bf16
    np.testing.assert_array_equal(bf16_bits_to_f32(f32_to_bf16_bits(static_v)), p2["int4"][1])
    # both modes attend over the same tokens
    for c in caches.values():
        assert sum(k.shape[1] for k, _ in pool_kv_by_tier(c).values()) == 64 + 96 + 64 + 130
    # capacity: the INT4-V arena refuses a flush past its room
    c = build_cache(key, value, offsets, lengths, classes, dtype="bfloat16", append_capacity=100, gen_values="int4")
    try:
        for i in range(129):
            append_token(c, rows_k[i], rows_v[i], global_index=s + i, logical_position=s + i)
    except RuntimeError as e:
        assert "capacity exhausted" in str(e)
    else:
        raise AssertionError("a flush past the INT4-V arena's room must raise")


def pool_kv_by_tier(c):
    from oracle.cache import pool_kv

    names = [n for n, k in zip(("fp", "int4", "int2"), c.pool_tokens) if k] + (["recent"] if c.recent_active else [])
    return dict(zip(names, pool_kv(c)))
