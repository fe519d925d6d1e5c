"""Pin the CPU oracle against fixtures written by the reference's own CPU path."""
import numpy as np
import pytest

from golden_io import as_f32, fixture_names, load
from oracle.attention import mixed_reference
from oracle.cache import append_token, build_cache

NAMES = fixture_names()


def _dtype(g):
    return "bfloat16" if "bfloat16" in str(g["dtype"]) else "float16"


def _build(g):
    dt = _dtype(g)
    return build_cache(
        as_f32(g["key"], dt), as_f32(g["value"], dt),
        g["page_offsets"], g["page_lengths"], g["page_classes"],
        dtype=dt, page_size=int(g["page_size"]), superblock=int(g["superblock"]),
        group=int(g["group"]), recent_capacity=128, append_capacity=260,
    )


def _check_snapshot(c, g, prefix, dt):
    k = c.k_active
    blocks = -(-k // c.superblock)
    assert k == int(g[prefix + "k_active"]) and c.k_capacity == int(g[prefix + "k_capacity"])
    assert tuple(c.k_segments) == tuple(int(v) for v in g[prefix + "k_segments"])
    np.testing.assert_array_equal(c.k_packed[:, :k], g[prefix + "k_packed"])
    np.testing.assert_array_equal(c.k_scale[:, :blocks].view(np.uint16), g[prefix + "k_scale"].view(np.uint16))
    np.testing.assert_array_equal(c.k_zero[:, :blocks], g[prefix + "k_zero"])
    a = c.v2_active
    assert a == int(g[prefix + "v2_active"]) and c.v2_capacity == int(g[prefix + "v2_capacity"])
    np.testing.assert_array_equal(c.v2_packed[:, :a], g[prefix + "v2_packed"])
    np.testing.assert_array_equal(c.v2_scale[:, :a].view(np.uint16), g[prefix + "v2_scale"].view(np.uint16))
    np.testing.assert_array_equal(c.v2_zero[:, :a], g[prefix + "v2_zero"])
    np.testing.assert_array_equal(c.v4_packed.reshape(-1), g[prefix + "v4_packed"].reshape(-1))
    np.testing.assert_array_equal(c.v4_scale.view(np.uint32), g[prefix + "v4_scale"].view(np.uint32))
    np.testing.assert_array_equal(c.fp_v, as_f32(g[prefix + "fp_v"], dt))
    r = c.recent_active
    assert r == int(g[prefix + "recent_active"])
    np.testing.assert_array_equal(c.recent_k[:, :r], as_f32(g[prefix + "recent_k"], dt))
    np.testing.assert_array_equal(c.recent_v[:, :r], as_f32(g[prefix + "recent_v"], dt))
    np.testing.assert_array_equal(c.recent_global[:r], g[prefix + "recent_global"])
    np.testing.assert_array_equal(c.recent_page_lengths, g[prefix + "recent_page_lengths"])
    assert list(c.pool_tokens) + [r] == [int(v) for v in g[prefix + "pool_tokens"]]
    np.testing.assert_array_equal(np.array(c.int2_global), g[prefix + "int2_global"])


@pytest.mark.parametrize("name", NAMES)
def test_build_matches_reference(name):
    g = load(name)
    c = _build(g)
    _check_snapshot(c, g, "build_", _dtype(g))
    out = mixed_reference(g["query"], c)
    np.testing.assert_allclose(out, g["build_attn"], rtol=0, atol=2e-6)


@pytest.mark.parametrize("name", NAMES)
def test_append_and_flush_match_reference(name):
    g = load(name)
    dt = _dtype(g)
    c = _build(g)
    ak = as_f32(g["append_k"], dt)
    av = as_f32(g["append_v"], dt)
    seq = g["key"].shape[1]
    flushed = []
    for step in range(ak.shape[0]):
        if append_token(c, ak[step, :, 0], av[step, :, 0], global_index=seq + step, logical_position=seq + step):
            flushed.append(step)
    assert flushed == list(g["flushed_at"])
    assert c.tail_dequant_tokens == int(g["tail_dequant_tokens"])
    _check_snapshot(c, g, "after_", dt)
    out = mixed_reference(g["query"], c)
    np.testing.assert_allclose(out, g["after_attn"], rtol=0, atol=2e-6)


# ------------------------------------------------------------------ BF16-K cache variants
from golden_io import variant_fixture_names  # noqa: E402

VARIANTS = variant_fixture_names()


def _build_variant(g):
    dt = _dtype(g)
    return build_cache(
        as_f32(g["key"], dt), as_f32(g["value"], dt),
        g["page_offsets"], g["page_lengths"], g["page_classes"],
        dtype=dt, page_size=int(g["page_size"]), superblock=int(g["superblock"]),
        group=int(g["group"]), recent_capacity=128, append_capacity=260, variant=str(g["variant"]),
    )


def _check_variant(c, g, prefix, dt):
    s = c.k_active
    if str(g["variant"]) == "int2k":
        blocks = -(-s // c.superblock)
        assert c.k_capacity == int(g[prefix + "k_capacity"])
        np.testing.assert_array_equal(c.k_packed[:, :s], g[prefix + "k_packed"])
        np.testing.assert_array_equal(c.k_scale[:, :blocks].view(np.uint16), g[prefix + "k_scale"].view(np.uint16))
        np.testing.assert_array_equal(c.k_zero[:, :blocks].view(np.uint16), g[prefix + "k_offset"].view(np.uint16))
        assert c.tail_dequant_tokens == int(g[prefix + "tail_dequant_tokens"])
    else:
        np.testing.assert_array_equal(c.k_rows[:, :s], as_f32(g[prefix + "k_rows"], dt))
    assert list(c.pool_tokens) + [c.recent_active] == [int(v) for v in g[prefix + "pool_tokens"]]
    np.testing.assert_array_equal(c.fp_v, as_f32(g[prefix + "fp_v"], dt))
    if str(g["variant"]) in ("bf16k", "int2k"):
        np.testing.assert_array_equal(c.v4_packed.reshape(-1), g[prefix + "v4_packed"].reshape(-1))
        np.testing.assert_array_equal(c.v4_scale.view(np.uint32), g[prefix + "v4_scale"].view(np.uint32))
        a = c.v2_active
        np.testing.assert_array_equal(c.v2_packed[:, :a], g[prefix + "v2_packed"])
        np.testing.assert_array_equal(c.v2_scale[:, :a].view(np.uint16), g[prefix + "v2_scale"].view(np.uint16))
        np.testing.assert_array_equal(c.v2_zero[:, :a], g[prefix + "v2_zero"])
    r = c.recent_active
    np.testing.assert_array_equal(c.recent_k[:, :r], as_f32(g[prefix + "recent_k"], dt))
    np.testing.assert_array_equal(c.recent_v[:, :r], as_f32(g[prefix + "recent_v"], dt))


@pytest.mark.parametrize("name", VARIANTS)
def test_bf16k_variants_build_append_and_attention_match_reference(name):
    g = load(name)
    dt = _dtype(g)
    c = _build_variant(g)
    _check_variant(c, g, "build_", dt)
    np.testing.assert_allclose(mixed_reference(g["query"], c), g["build_attn"], rtol=0, atol=2e-6)
    ak, av = as_f32(g["append_k"], dt), as_f32(g["append_v"], dt)
    seq = g["key"].shape[1]
    flushed, refused = [], -1
    for step in range(ak.shape[0]):
        try:
            if append_token(c, ak[step, :, 0], av[step, :, 0], global_index=seq + step, logical_position=seq + step):
                flushed.append(step)
        except RuntimeError:
            refused = step
            break
    assert flushed == list(g["flushed_at"]) and refused == int(g["refused_at"])
    _check_variant(c, g, "after_", dt)
    np.testing.assert_allclose(mixed_reference(g["query"], c), g["after_attn"], rtol=0, atol=2e-6)


# ------------------------------------------------------------------ generated INT4 values
from golden_io import gen_int4_fixture_names  # noqa: E402

GEN_INT4 = gen_int4_fixture_names()


def _check_gen_int4(c, g, prefix, dt):
    k = c.k_active
    blocks = -(-k // c.superblock)
    assert k == int(g[prefix + "k_active"]) and c.k_capacity == int(g[prefix + "k_capacity"])
    assert tuple(c.k_segments) == tuple(int(v) for v in g[prefix + "k_segments"])
    assert c.gen_k_offset == int(g[prefix + "generated_k_offset"])
    assert c.static_i4 == int(g[prefix + "static_int4_tokens"])
    np.testing.assert_array_equal(c.k_packed[:, :k], g[prefix + "k_packed"])
    np.testing.assert_array_equal(c.k_scale[:, :blocks].view(np.uint16), g[prefix + "k_scale"].view(np.uint16))
    np.testing.assert_array_equal(c.k_zero[:, :blocks], g[prefix + "k_zero"])
    n4 = c.pool_tokens[1]
    assert n4 == int(g[prefix + "v4_active"]) and c.v4_capacity == int(g[prefix + "v4_capacity"])
    np.testing.assert_array_equal(c.v4_packed[:, :n4], g[prefix + "v4_packed"])
    np.testing.assert_array_equal(c.v4_scale[:, :n4].view(np.uint32), g[prefix + "v4_scale"].view(np.uint32))
    a = c.v2_active
    assert a == int(g[prefix + "v2_active"]) and c.v2_capacity == int(g[prefix + "v2_capacity"])
    np.testing.assert_array_equal(c.v2_packed[:, :a], g[prefix + "v2_packed"])
    np.testing.assert_array_equal(c.v2_scale[:, :a].view(np.uint16), g[prefix + "v2_scale"].view(np.uint16))
    np.testing.assert_array_equal(c.v2_zero[:, :a], g[prefix + "v2_zero"])
    np.testing.assert_array_equal(c.fp_v, as_f32(g[prefix + "fp_v"], dt))
    r = c.recent_active
    assert r == int(g[prefix + "recent_active"])
    np.testing.assert_array_equal(c.recent_k[:, :r], as_f32(g[prefix + "recent_k"], dt))
    np.testing.assert_array_equal(c.recent_v[:, :r], as_f32(g[prefix + "recent_v"], dt))
    np.testing.assert_array_equal(c.recent_global[:r], g[prefix + "recent_global"])
    assert list(c.pool_tokens) + [r] == [int(v) for v in g[prefix + "pool_tokens"]]
    np.testing.assert_array_equal(np.array(c.int4_global), g[prefix + "int4_global"])
    np.testing.assert_array_equal(np.array(c.int4_logical), g[prefix + "int4_logical"])
    np.testing.assert_array_equal(np.array(c.int2_global), g[prefix + "int2_global"])


@pytest.mark.parametrize("name", GEN_INT4)
def test_generated_int4_values_match_reference(name):
    """generated_value_precision="int4": the build (INT4-V arena with room, INT2-V arena without),
    the flushes packing the oldest ring values into the INT4-V arena and their indices into the INT4
    pool, and the attention over the INT4 pool's two K runs, each against the reference's own output."""
    g = load(name)
    dt = _dtype(g)
    c = build_cache(as_f32(g["key"], dt), as_f32(g["value"], dt), g["page_offsets"], g["page_lengths"],
                    g["page_classes"], dtype=dt, page_size=int(g["page_size"]), superblock=int(g["superblock"]),
                    group=int(g["group"]), recent_capacity=128, append_capacity=260, gen_values="int4")
    _check_gen_int4(c, g, "build_", dt)
    np.testing.assert_allclose(mixed_reference(g["query"], c), g["build_attn"], rtol=0, atol=2e-6)
    ak, av = as_f32(g["append_k"], dt), as_f32(g["append_v"], dt)
    seq = g["key"].shape[1]
    flushed = []
    for step in range(ak.shape[0]):
        if append_token(c, ak[step, :, 0], av[step, :, 0], global_index=seq + step, logical_position=seq + step):
            flushed.append(step)
    assert flushed == list(g["flushed_at"]) and len(flushed) >= 1
    assert c.tail_dequant_tokens == int(g["tail_dequant_tokens"])
    assert 128 * len(flushed) == int(g["flushed_int4_value_tokens"])
    _check_gen_int4(c, g, "after_", dt)
    np.testing.assert_allclose(mixed_reference(g["query"], c), g["after_attn"], rtol=0, atol=2e-6)


@pytest.mark.parametrize("name", GEN_INT4)
def test_generated_int4_fixture_pins_unrounded_static_values(name):
    """The INT4-V arena's dequantisation stays fp32 (fused_value_pack.py:241-256), where the INT2 mode's
    PackedTensor rounds to the input dtype: the reference's attention output tells the two apart, so the
    oracle's choice is pinned by the fixture, not restated.  The mistake is planted in the oracle."""
    g = load(name)
    dt = _dtype(g)
    c = build_cache(as_f32(g["key"], dt), as_f32(g["value"], dt), g["page_offsets"], g["page_lengths"],
                    g["page_classes"], dtype=dt, page_size=int(g["page_size"]), superblock=int(g["superblock"]),
                    group=int(g["group"]), recent_capacity=128, append_capacity=260, gen_values="int4")
    n4 = c.pool_tokens[1]
    c.gen_values = "int2"  # the INT2 mode's INT4 dequantisation: rounded to the model dtype
    c.v4_packed, c.v4_scale = c.v4_packed[:, :n4], c.v4_scale[:, :n4]
    assert np.abs(mixed_reference(g["query"], c) - g["build_attn"]).max() > 2e-5
