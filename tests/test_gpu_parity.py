"""GPU parity of the HIP path against the CPU oracle and the reference-written golden fixtures.

Bars: packing and quantisation bit-exact; attention output within
max-abs 2e-2 and mean-abs 2e-3 of the fp32 dequantise-then-softmax oracle.
"""
import numpy as np
import pytest
import torch

from golden_io import as_f32, fixture_names, load, variant_fixture_names

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MEAN_ABS = 2e-3


def _cuda():
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    return torch.device("cuda:0")


def _to_torch(arr, dtype, dev):
    if "bfloat16" in str(dtype):
        return torch.from_numpy(np.ascontiguousarray(arr).view(np.int16)).view(torch.bfloat16).to(dev)
    return torch.from_numpy(np.ascontiguousarray(arr)).to(dev)


def _bf16_np(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _bits16(t):
    """16-bit payload of a bf16 or fp16 tensor as uint16 bit patterns (fixtures store fp16 as float16)."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


# --------------------------------------------------------------------------- golden builds
@pytest.mark.parametrize("name", fixture_names())
def test_build_and_flush_bit_exact_against_reference_fixtures(name):
    import r2omni_amd as ro

    dev = _cuda()
    g = load(name)
    dt = str(g["dtype"])
    key = _to_torch(g["key"], dt, dev)
    value = _to_torch(g["value"], dt, dev)
    plan = ro.plan_from_pages(g["page_offsets"], g["page_lengths"], g["page_classes"], recent_fp_capacity=128,
                              device=dev)
    cache = ro.build_three_precision_cache(
        key, value, plan, page_size=int(g["page_size"]), key_quantization_superblock=int(g["superblock"]),
        int2_group_size=int(g["group"]), compact_key_append_capacity=260, recent_flush_size=128)

    def check(prefix):
        torch.cuda.synchronize()
        ck, cv = cache.compact_key, cache.compact_value
        k = ck.active_length
        blocks = -(-k // ck.superblock_size)
        assert k == int(g[prefix + "k_active"]) and ck.capacity == int(g[prefix + "k_capacity"])
        np.testing.assert_array_equal(ck.packed[:, :k].cpu().numpy(), g[prefix + "k_packed"])
        np.testing.assert_array_equal(ck.scale[:, :blocks].cpu().view(torch.int16).numpy(),
                                      g[prefix + "k_scale"].view(np.int16))
        np.testing.assert_array_equal(ck.zero_point[:, :blocks].cpu().numpy(), g[prefix + "k_zero"])
        a = cv.active_length
        assert a == int(g[prefix + "v2_active"]) and cv.capacity == int(g[prefix + "v2_capacity"])
        np.testing.assert_array_equal(cv.packed[:, :a].cpu().numpy(), g[prefix + "v2_packed"])
        np.testing.assert_array_equal(cv.scale[:, :a].cpu().view(torch.int16).numpy(),
                                      g[prefix + "v2_scale"].view(np.int16))
        np.testing.assert_array_equal(cv.zero_point[:, :a].cpu().numpy(), g[prefix + "v2_zero"])
        i4 = cache.int4_pool
        if i4.token_count:
            np.testing.assert_array_equal(i4.packed_v.packed.cpu().numpy(), g[prefix + "v4_packed"])
            np.testing.assert_array_equal(i4.packed_v.scale.cpu().numpy().view(np.uint32),
                                          g[prefix + "v4_scale"].view(np.uint32))
        if cache.fp_pool.token_count:
            got = cache.fp_pool.fp_v.cpu()
            want = _to_torch(g[prefix + "fp_v"], dt, "cpu")
            assert torch.equal(got.view(torch.int16), want.view(torch.int16))
        rec = cache.recent_fp_pool
        r = rec.active_length
        assert r == int(g[prefix + "recent_active"])
        assert int(rec.length_device.item()) == r
        want_k = _to_torch(g[prefix + "recent_k"], dt, "cpu")
        assert torch.equal(rec.fp_k[:, :r].cpu().view(torch.int16), want_k.view(torch.int16))
        np.testing.assert_array_equal(rec.global_index_buffer[:r].cpu().numpy(), g[prefix + "recent_global"])
        np.testing.assert_array_equal(rec.page_index.lengths.cpu().numpy(), g[prefix + "recent_page_lengths"])
        pools = [cache.fp_pool.token_count, cache.int4_pool.token_count, cache.int2_pool.token_count, r]
        assert pools == [int(v) for v in g[prefix + "pool_tokens"]]
        np.testing.assert_array_equal(
            cache.int2_pool.page_index.global_token_indices.cpu().numpy(), g[prefix + "int2_global"])

    stats = ro.DynamicCacheStats()
    check("build_")
    ak = _to_torch(g["append_k"], dt, dev)
    av = _to_torch(g["append_v"], dt, dev)
    seq = int(g["key"].shape[1])
    flushed = []
    for step in range(int(ak.shape[0])):
        if ro.append_generated_token(cache, ak[step], av[step], global_token_index=seq + step,
                                     logical_position=seq + step, stats=stats):
            flushed.append(step)
    assert flushed == list(g["flushed_at"])
    assert stats.local_tail_dequant_tokens == int(g["tail_dequant_tokens"])
    check("after_")


# ------------------------------------------------------------------------ decode parity
def _oracle_for(data, cfg):
    from oracle.cache import append_token, build_cache
    from oracle.quant import bf16_bits_to_f32

    f32 = lambda t: bf16_bits_to_f32(_bf16_np(t))  # noqa: E731
    c = build_cache(f32(data.key), f32(data.value), data.page_offsets.numpy(), data.page_lengths.numpy(),
                    data.page_classes.numpy(), dtype="bfloat16", page_size=cfg.page, superblock=cfg.superblock,
                    group=cfg.group, recent_capacity=128, append_capacity=260, variant=cfg.variant,
                    gen_values=cfg.gen_values)
    hist = int(data.key.shape[1])
    rk, rv = f32(data.recent_k), f32(data.recent_v)
    for i in range(rk.shape[0]):
        append_token(c, rk[i], rv[i], global_index=hist + i, logical_position=hist + i)
    return c


def _compare(got_bf16, want_f32, what):
    got = got_bf16.float().cpu().numpy()
    err = np.abs(got - want_f32)
    assert np.isfinite(got).all(), what
    assert err.max() <= MAX_ABS, f"{what}: max-abs {err.max():.3e}"
    assert err.mean() <= MEAN_ABS, f"{what}: mean-abs {err.mean():.3e}"
    return float(err.max()), float(err.mean())


SMALL = [
    # hq, hkv, total tokens, tier probs, recent, superblock, group
    (16, 2, 1024 + 64, (0.2, 0.5, 0.3), 64, 32, 32),
    (16, 2, 2048 + 128, (0.0, 1.0, 0.0), 0, 32, 32),
    (28, 4, 1536 + 100, (0.15, 0.45, 0.4), 100, 32, 32),
    (32, 8, 1024 + 128, (0.0, 0.0, 1.0), 128, 128, 128),
    (16, 2, 640 + 17, (1.0, 0.0, 0.0), 17, 64, 64),
]


@pytest.mark.parametrize("case", range(len(SMALL)))
@pytest.mark.parametrize("hadamard", [False, True])
def test_decode_matches_oracle(case, hadamard):
    import r2omni_amd as ro
    from r2omni_amd.workloads import DecodeConfig, build_request_cache, make_request
    from oracle.attention import mixed_reference, output_transform
    from oracle.quant import bf16_bits_to_f32

    dev = _cuda()
    hq, hkv, total, probs, recent, sb, grp = SMALL[case]
    cfg = DecodeConfig("t", hq, hkv, (total,), probs, recent=recent, superblock=sb, group=grp)
    hist = ((total - recent) // 64) * 64
    data = make_request(cfg, hist + recent, seed=100 + case, device=dev)
    cache = build_request_cache(cfg, data)
    ws = ro.allocate_splitk_workspace(cache, num_query_heads=hq)
    ex = ro.prepare_splitk_executor(cache, ws, output_hadamard=hadamard)
    out = ex(data.query.contiguous())
    torch.cuda.synchronize()
    oc = _oracle_for(data, cfg)
    q = bf16_bits_to_f32(_bf16_np(data.query))
    want = output_transform(mixed_reference(q, oc), hadamard)
    _compare(out, want, f"case {case} hadamard {hadamard}")


def test_decode_long_group_combine():
    """One KV head over 40k tokens: several hundred partial slots merged by one combine group."""
    import r2omni_amd as ro
    from r2omni_amd.workloads import DecodeConfig, build_request_cache, make_request
    from oracle.attention import mixed_reference, output_transform
    from oracle.quant import bf16_bits_to_f32

    dev = _cuda()
    cfg = DecodeConfig("long", 8, 1, (40960 + 128,), (0.15, 0.45, 0.4), recent=128, superblock=32, group=32)
    data = make_request(cfg, 40960 + 128, seed=77, device=dev)
    cache = build_request_cache(cfg, data)
    ws = ro.allocate_splitk_workspace(cache, num_query_heads=8)
    ex = ro.prepare_splitk_executor(cache, ws, output_hadamard=True)
    sizes = torch.diff(ex.group_begin.cpu())
    print(f"long group: {int(sizes.max())} slots", flush=True)
    oc = _oracle_for(data, cfg)
    q = bf16_bits_to_f32(_bf16_np(data.query))
    want = output_transform(mixed_reference(q, oc), True)
    for call in range(2):
        out = ex(data.query.contiguous())
        torch.cuda.synchronize()
        _compare(out, want, f"long group call {call}")


def _misaligned(t):
    """The same values as a contiguous view whose data pointer is one element past t's storage start."""
    buf = torch.empty(t.numel() + 1, device=t.device, dtype=t.dtype)
    buf[1:] = t.flatten()
    return buf[1:].view(t.shape)


@pytest.mark.parametrize("variant", ["int4k", "int2k"])
def test_fused_append_then_flush_matches_oracle(variant):
    import r2omni_amd as ro
    from r2omni_amd.workloads import DecodeConfig, build_request_cache, make_request
    from oracle.attention import mixed_reference, output_transform
    from oracle.cache import append_token
    from oracle.quant import bf16_bits_to_f32

    dev = _cuda()
    cfg = DecodeConfig("t", 16, 2, (0,), (0.2, 0.5, 0.3), recent=120, variant=variant)
    data = make_request(cfg, 1280 + 120, seed=7, device=dev)
    cache = build_request_cache(cfg, data)
    oc = _oracle_for(data, cfg)
    ws = ro.allocate_splitk_workspace(cache, num_query_heads=16, reserve_tokens=260)
    ex = ro.prepare_splitk_executor(cache, ws)
    gen = torch.Generator(device=dev).manual_seed(8)
    stats = ro.DynamicCacheStats()
    hist = int(data.key.shape[1]) + 120
    for step in range(20):
        q = torch.randn(1, 16, 128, generator=gen, device=dev).to(torch.bfloat16)
        k = torch.randn(1, 2, 128, generator=gen, device=dev).to(torch.bfloat16)
        v = torch.randn(1, 2, 128, generator=gen, device=dev).to(torch.bfloat16)
        pos = hist + step
        rec = cache.recent_fp_pool
        if rec.active_length < rec.capacity:
            # odd steps pass the rows as views 2 bytes past a 16-byte boundary (copied by the executor)
            ka, va = (_misaligned(k), _misaligned(v)) if step % 2 else (k, v)
            assert (ka.data_ptr() % 16 != 0) == bool(step % 2)
            out = ex(q, append=(ka, va, pos, pos))
            rec.active_length += 1  # the caller advances the host length after a fused append
            kf, vf = bf16_bits_to_f32(_bf16_np(k[0])), bf16_bits_to_f32(_bf16_np(v[0]))
            want = mixed_reference(bf16_bits_to_f32(_bf16_np(q)), oc, append=(kf, vf))
            append_token(oc, kf, vf, global_index=pos, logical_position=pos)
        else:
            assert ro.append_generated_token(cache, k[0][:, None], v[0][:, None], global_token_index=pos,
                                             logical_position=pos, stats=stats)
            ex = ro.prepare_splitk_executor(cache, ws)
            kf, vf = bf16_bits_to_f32(_bf16_np(k[0])), bf16_bits_to_f32(_bf16_np(v[0]))
            append_token(oc, kf, vf, global_index=pos, logical_position=pos)
            out = ex(q)
            want = mixed_reference(bf16_bits_to_f32(_bf16_np(q)), oc)
        torch.cuda.synchronize()
        _compare(out, output_transform(want, False), f"step {step}")
    assert stats.flushed_tokens == 128
    # the ring, lengths and arenas agree with the oracle after the flush
    assert cache.recent_fp_pool.active_length == oc.recent_active
    assert int(cache.recent_fp_pool.length_device.item()) == oc.recent_active
    rec, r_act = cache.recent_fp_pool, oc.recent_active  # ring rows written by the fused appends
    np.testing.assert_array_equal(bf16_bits_to_f32(_bf16_np(rec.fp_k[:, :r_act])), oc.recent_k[:, :r_act])
    np.testing.assert_array_equal(bf16_bits_to_f32(_bf16_np(rec.fp_v[:, :r_act])), oc.recent_v[:, :r_act])
    _check_k_arena(cache, oc)


@pytest.mark.parametrize("variant", ["int4k", "int2k"])
def test_ragged_batch_matches_per_request_oracle(variant):
    import r2omni_amd as ro
    from r2omni_amd.workloads import DecodeConfig, build_request_cache, make_request
    from oracle.attention import mixed_reference, output_transform
    from oracle.quant import bf16_bits_to_f32

    dev = _cuda()
    cfg = DecodeConfig("t", 28, 4, (0,), (0.15, 0.45, 0.4), recent=128, variant=variant)
    totals = (512 + 128, 1024 + 128, 2048 + 128, 3072 + 128)
    datas = [make_request(cfg, t, seed=200 + i, device=dev) for i, t in enumerate(totals)]
    caches = [build_request_cache(cfg, d) for d in datas]
    wss = [ro.allocate_splitk_workspace(c, num_query_heads=28) for c in caches]
    exs = [ro.prepare_splitk_executor(c, w, output_hadamard=True) for c, w in zip(caches, wss)]
    batched = ro.stack_homogeneous_splitk_executors(exs)
    q = torch.cat([d.query for d in datas]).contiguous()
    out = batched(q)
    torch.cuda.synchronize()
    for r, d in enumerate(datas):
        want = output_transform(mixed_reference(bf16_bits_to_f32(_bf16_np(d.query)), _oracle_for(d, cfg)), True)
        _compare(out[r : r + 1], want, f"request {r}")


# ------------------------------------------------------- other K formats (BF16-K, INT2-K)
VARIANT_CASES = [0, 2, 4]  # mixed tiers with a partial ring, GQA 7 over 4 KV heads, FP-only pages


def _check_k_arena(cache, oc):
    """The GPU K arena equals the oracle's, bit for bit, in the same physical order."""
    from oracle.quant import bf16_bits_to_f32

    if cache.bf16_key is not None:  # key rows in the model dtype (bf16 or fp16): exact as fp32
        kb = cache.bf16_key
        assert kb.active_length == oc.k_active
        got_rows = kb.rows[:, : kb.active_length].float().cpu().numpy()
        np.testing.assert_array_equal(got_rows, oc.k_rows[:, : oc.k_active])
        return
    ck = cache.compact_key
    k = ck.active_length
    blocks = -(-k // ck.superblock_size)
    assert k == oc.k_active and ck.capacity == oc.k_capacity
    np.testing.assert_array_equal(ck.packed[:, :k].cpu().numpy(), oc.k_packed[:, :k])
    np.testing.assert_array_equal(ck.scale[:, :blocks].cpu().view(torch.int16).numpy().view(np.uint16),
                                  oc.k_scale[:, :blocks].view(np.uint16))
    zp = ck.zero_point[:, :blocks].cpu()
    want = oc.k_zero[:, :blocks]
    if zp.dtype == torch.float16:
        np.testing.assert_array_equal(zp.view(torch.int16).numpy().view(np.uint16), want.view(np.uint16))
    else:
        np.testing.assert_array_equal(zp.numpy(), want)


@pytest.mark.parametrize("variant,case", [(v, c) for v in ("matched", "bf16k") for c in VARIANT_CASES]
                         + [("int2k", c) for c in range(len(SMALL))])
@pytest.mark.parametrize("hadamard", [False, True])
def test_k_format_variants_decode_matches_oracle(variant, case, hadamard):
    import r2omni_amd as ro
    from r2omni_amd.workloads import DecodeConfig, build_request_cache, make_request
    from oracle.attention import mixed_reference, output_transform
    from oracle.quant import bf16_bits_to_f32

    dev = _cuda()
    hq, hkv, total, probs, recent, sb, grp = SMALL[case]
    cfg = DecodeConfig("t", hq, hkv, (total,), probs, recent=recent, superblock=sb, group=grp, variant=variant)
    hist = ((total - recent) // 64) * 64
    data = make_request(cfg, hist + recent, seed=300 + case, device=dev)
    cache = build_request_cache(cfg, data)
    if variant == "int2k":
        assert cache.compact_key is not None and cache.compact_key.bit_width == 2
    else:
        assert cache.bf16_key is not None and cache.compact_key is None
    ws = ro.allocate_splitk_workspace(cache, num_query_heads=hq)
    ex = ro.prepare_splitk_executor(cache, ws, output_hadamard=hadamard)
    out = ex(data.query.contiguous())
    torch.cuda.synchronize()
    oc = _oracle_for(data, cfg)
    _check_k_arena(cache, oc)
    q = bf16_bits_to_f32(_bf16_np(data.query))
    want = output_transform(mixed_reference(q, oc), hadamard)
    _compare(out, want, f"{variant} case {case} hadamard {hadamard}")


# ------------------------------------------------------------- INT4 generated values
@pytest.mark.parametrize("variant", ["int4k", "int2k"])
def test_generated_int4_values_flush_matches_oracle(variant):
    """``generated_value_precision="int4"``: the INT4 pool's values live in a compact INT4-V arena
    with append room; a flush packs the ring's oldest 128 values into it (bit-exact against the
    oracle), appends their page metadata to the INT4 pool in place, and the decode over the
    two-run INT4 pool (static keys at their segment, generated keys after the INT2 segment) and
    the torch mixed reference both match the oracle."""
    import r2omni_amd as ro
    from r2omni_amd.workloads import DecodeConfig, build_request_cache, make_request
    from oracle.attention import mixed_reference, output_transform
    from oracle.cache import append_token
    from oracle.quant import bf16_bits_to_f32

    dev = _cuda()
    cfg = DecodeConfig("t", 16, 2, (0,), (0.2, 0.5, 0.3), recent=120, variant=variant, gen_values="int4")
    data = make_request(cfg, 1280 + 120, seed=9, device=dev)
    cache = build_request_cache(cfg, data)
    oc = _oracle_for(data, cfg)
    a4 = cache.compact_int4_value
    assert a4 is not None and cache.int4_pool.packed_v is a4 and cache.generated_value_precision == "int4"
    static = cache.static_int4_tokens
    assert static == oc.static_i4 == a4.active_length and a4.capacity == oc.v4_capacity
    assert cache.compact_value.capacity == oc.v2_capacity
    np.testing.assert_array_equal(a4.packed[:, :static].cpu().numpy(), oc.v4_packed[:, :static])
    np.testing.assert_array_equal(a4.scale[:, :static].cpu().numpy(), oc.v4_scale[:, :static])
    ws = ro.allocate_splitk_workspace(cache, num_query_heads=16, reserve_tokens=260)
    ex = ro.prepare_splitk_executor(cache, ws)
    gen = torch.Generator(device=dev).manual_seed(10)
    stats = ro.DynamicCacheStats()
    s_hist = int(data.key.shape[1])
    pos0 = s_hist + 120
    for step in range(20):
        q = torch.randn(1, 16, 128, generator=gen, device=dev).to(torch.bfloat16)
        k = torch.randn(1, 2, 128, generator=gen, device=dev).to(torch.bfloat16)
        v = torch.randn(1, 2, 128, generator=gen, device=dev).to(torch.bfloat16)
        pos = pos0 + step
        kf, vf = bf16_bits_to_f32(_bf16_np(k[0])), bf16_bits_to_f32(_bf16_np(v[0]))
        qf = bf16_bits_to_f32(_bf16_np(q))
        rec = cache.recent_fp_pool
        if rec.active_length < rec.capacity:
            out = ex(q, append=(k, v, pos, pos))
            rec.active_length += 1
            want = mixed_reference(qf, oc, append=(kf, vf))
            append_token(oc, kf, vf, global_index=pos, logical_position=pos)
        else:
            assert ro.append_generated_token(cache, k[0][:, None], v[0][:, None], global_token_index=pos,
                                             logical_position=pos, stats=stats)
            ex = ro.prepare_splitk_executor(cache, ws)
            append_token(oc, kf, vf, global_index=pos, logical_position=pos)
            out = ex(q)
            want = mixed_reference(qf, oc)
            ref = ro.triton_mixed_reference(q, cache)
            _compare(ref, output_transform(want, False), "torch mixed reference after the flush")
        torch.cuda.synchronize()
        _compare(out, output_transform(want, False), f"step {step}")
    assert stats.flushed_tokens == stats.flushed_int4_value_tokens == 128
    n4 = cache.int4_pool.token_count
    assert n4 == oc.pool_tokens[1] == static + 128 == a4.active_length
    assert cache.int2_pool.token_count == oc.pool_tokens[2] == cache.compact_value.active_length
    np.testing.assert_array_equal(a4.packed[:, :n4].cpu().numpy(), oc.v4_packed[:, :n4])
    np.testing.assert_array_equal(a4.scale[:, :n4].cpu().numpy(), oc.v4_scale[:, :n4])
    pi = cache.int4_pool.page_index
    assert pi.global_token_indices[static:].tolist() == list(range(s_hist, s_hist + 128))
    assert pi.logical_positions[static:].tolist() == list(range(s_hist, s_hist + 128))
    assert pi.global_token_indices.data_ptr() == cache.metadata_arena.int4_global_index_buffer.data_ptr()
    _check_k_arena(cache, oc)


def test_matched_fp_fused_append_then_flush_matches_oracle():
    """Matched-FP: the 129th generated token moves the ring's first 128 rows into the FP pool."""
    import r2omni_amd as ro
    from r2omni_amd.workloads import DecodeConfig, build_request_cache, make_request
    from oracle.attention import mixed_reference, output_transform
    from oracle.cache import append_token
    from oracle.quant import bf16_bits_to_f32

    dev = _cuda()
    cfg = DecodeConfig("t", 16, 2, (0,), (0.2, 0.5, 0.3), recent=120, variant="matched")
    data = make_request(cfg, 1280 + 120, seed=9, device=dev)
    cache = build_request_cache(cfg, data)
    oc = _oracle_for(data, cfg)
    ws = ro.allocate_splitk_workspace(cache, num_query_heads=16, reserve_tokens=260)
    ex = ro.prepare_splitk_executor(cache, ws)
    gen = torch.Generator(device=dev).manual_seed(10)
    stats = ro.DynamicCacheStats()
    hist = int(data.key.shape[1]) + 120
    fp_before = cache.fp_pool.token_count
    for step in range(20):
        q = torch.randn(1, 16, 128, generator=gen, device=dev).to(torch.bfloat16)
        k = torch.randn(1, 2, 128, generator=gen, device=dev).to(torch.bfloat16)
        v = torch.randn(1, 2, 128, generator=gen, device=dev).to(torch.bfloat16)
        pos = hist + step
        kf, vf = bf16_bits_to_f32(_bf16_np(k[0])), bf16_bits_to_f32(_bf16_np(v[0]))
        rec = cache.recent_fp_pool
        if rec.active_length < rec.capacity:
            out = ex(q, append=(k, v, pos, pos))
            rec.active_length += 1
            want = mixed_reference(bf16_bits_to_f32(_bf16_np(q)), oc, append=(kf, vf))
            append_token(oc, kf, vf, global_index=pos, logical_position=pos)
        else:
            assert ro.append_generated_token(cache, k[0][:, None], v[0][:, None], global_token_index=pos,
                                             logical_position=pos, stats=stats)
            ex = ro.prepare_splitk_executor(cache, ws)
            append_token(oc, kf, vf, global_index=pos, logical_position=pos)
            out = ex(q)
            want = mixed_reference(bf16_bits_to_f32(_bf16_np(q)), oc)
        torch.cuda.synchronize()
        _compare(out, output_transform(want, False), f"matched step {step}")
    assert stats.flushed_tokens == 128
    assert cache.fp_pool.token_count == fp_before + 128 == oc.pool_tokens[0]
    assert cache.recent_fp_pool.active_length == oc.recent_active
    kb = cache.bf16_key
    assert kb.active_length == oc.k_active
    np.testing.assert_array_equal(bf16_bits_to_f32(_bf16_np(kb.rows[:, : kb.active_length])),
                                  oc.k_rows[:, : oc.k_active])
    np.testing.assert_array_equal(bf16_bits_to_f32(_bf16_np(cache.fp_pool.fp_v)), oc.fp_v)


def test_bf16k_ring_overflow_is_refused():
    """v_fourq_k_bf16 has no low-bit flush: a full ring refuses the next token (dynamic_fourq_cache.py:226-230)."""
    import r2omni_amd as ro
    from r2omni_amd.workloads import DecodeConfig, build_request_cache, make_request

    dev = _cuda()
    cfg = DecodeConfig("t", 16, 2, (0,), (0.2, 0.5, 0.3), recent=128, variant="bf16k")
    data = make_request(cfg, 1024 + 128, seed=11, device=dev)
    cache = build_request_cache(cfg, data)
    assert cache.recent_fp_pool.active_length == cache.recent_fp_pool.capacity
    k = torch.zeros(2, 1, 128, device=dev, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="K-BF16/V-FourQ"):
        ro.append_generated_token(cache, k, k, global_token_index=5000, logical_position=5000,
                                  stats=ro.DynamicCacheStats())


@pytest.mark.parametrize("name", variant_fixture_names())
def test_k_format_variant_build_and_appends_bit_exact_against_reference_fixtures(name):
    """BF16-K / INT2-K builds and appends against the reference's own cache state, then decode
    against the oracle."""
    import r2omni_amd as ro
    from oracle.attention import mixed_reference
    from oracle.cache import append_token, build_cache
    from oracle.quant import bf16_bits_to_f32

    dev = _cuda()
    g = load(name)
    dt = str(g["dtype"])
    variant = str(g["variant"])
    key = _to_torch(g["key"], dt, dev)
    value = _to_torch(g["value"], dt, dev)
    plan = ro.plan_from_pages(g["page_offsets"], g["page_lengths"], g["page_classes"], recent_fp_capacity=128,
                              device=dev)
    kwargs = dict(page_size=int(g["page_size"]), key_quantization_superblock=int(g["superblock"]),
                  int2_group_size=int(g["group"]), compact_key_append_capacity=260, recent_flush_size=128)
    if variant == "matched":
        cache = ro.build_three_precision_cache(key, value, plan, matched_fp=True, **kwargs)
    elif variant == "int2k":
        cache = ro.build_three_precision_cache(key, value, plan, cache_variant="v_fourq_k_int2_compact", **kwargs)
    else:
        cache = ro.build_three_precision_cache(key, value, plan, cache_variant="v_fourq_k_bf16", **kwargs)
    oc = build_cache(as_f32(g["key"], dt), as_f32(g["value"], dt), g["page_offsets"], g["page_lengths"],
                     g["page_classes"], dtype=dt.replace("torch.", ""), page_size=int(g["page_size"]), superblock=int(g["superblock"]),
                     group=int(g["group"]), recent_capacity=128, append_capacity=260, variant=variant)
    q = torch.from_numpy(g["query"]).to(dev).to(torch.bfloat16)
    qf = bf16_bits_to_f32(_bf16_np(q))

    def check(prefix):
        torch.cuda.synchronize()
        if variant == "int2k":
            ck = cache.compact_key
            k = ck.active_length
            blocks = -(-k // ck.superblock_size)
            assert ck.capacity == int(g[prefix + "k_capacity"])
            np.testing.assert_array_equal(ck.packed[:, :k].cpu().numpy(), g[prefix + "k_packed"])
            np.testing.assert_array_equal(ck.scale[:, :blocks].cpu().view(torch.int16).numpy().view(np.uint16),
                                          g[prefix + "k_scale"].view(np.uint16))
            np.testing.assert_array_equal(ck.zero_point[:, :blocks].cpu().view(torch.int16).numpy().view(np.uint16),
                                          g[prefix + "k_offset"].view(np.uint16))
            assert stats.local_tail_dequant_tokens == int(g[prefix + "tail_dequant_tokens"])
        else:
            kb = cache.bf16_key
            rows = kb.rows[:, : kb.active_length].cpu().view(torch.int16).numpy().view(np.uint16)
            np.testing.assert_array_equal(rows, g[prefix + "k_rows"])
        pools = [cache.fp_pool.token_count, cache.int4_pool.token_count, cache.int2_pool.token_count,
                 cache.recent_fp_pool.active_length]
        assert pools == [int(v) for v in g[prefix + "pool_tokens"]]
        fp_v = cache.fp_pool.fp_v[:, : cache.fp_pool.token_count] if cache.fp_pool.token_count else None
        if fp_v is not None:
            np.testing.assert_array_equal(_bits16(fp_v), g[prefix + "fp_v"].view(np.uint16))
        if variant in ("bf16k", "int2k"):
            i4 = cache.int4_pool
            if i4.token_count:
                np.testing.assert_array_equal(i4.packed_v.packed.cpu().numpy().reshape(-1),
                                              g[prefix + "v4_packed"].reshape(-1))
                np.testing.assert_array_equal(i4.packed_v.scale.cpu().numpy().view(np.uint32).reshape(-1),
                                              g[prefix + "v4_scale"].view(np.uint32).reshape(-1))
            cv = cache.compact_value
            a = cv.active_length
            np.testing.assert_array_equal(cv.packed[:, :a].cpu().numpy(), g[prefix + "v2_packed"])
            np.testing.assert_array_equal(cv.scale[:, :a].cpu().view(torch.int16).numpy().view(np.uint16),
                                          g[prefix + "v2_scale"].view(np.uint16))
            np.testing.assert_array_equal(cv.zero_point[:, :a].cpu().numpy(), g[prefix + "v2_zero"])
        r = cache.recent_fp_pool.active_length
        np.testing.assert_array_equal(_bits16(cache.recent_fp_pool.fp_k[:, :r]),
                                      g[prefix + "recent_k"].view(np.uint16))
        ws = ro.allocate_splitk_workspace(cache, num_query_heads=int(q.shape[1]))
        out = ro.prepare_splitk_executor(cache, ws)(q)  # bf16 query over bf16 or fp16 rows
        torch.cuda.synchronize()
        _compare(out, mixed_reference(qf, oc), f"{name} {prefix}decode")

    stats = ro.DynamicCacheStats()
    check("build_")
    ak = _to_torch(g["append_k"], dt, dev)
    av = _to_torch(g["append_v"], dt, dev)
    seq = int(g["key"].shape[1])
    flushed, refused = [], -1
    for step in range(int(ak.shape[0])):
        try:
            if ro.append_generated_token(cache, ak[step], av[step], global_token_index=seq + step,
                                         logical_position=seq + step, stats=stats):
                flushed.append(step)
        except RuntimeError:
            refused = step
            break
        append_token(oc, as_f32(g["append_k"][step, :, 0], dt), as_f32(g["append_v"][step, :, 0], dt),
                     global_index=seq + step, logical_position=seq + step)
    assert flushed == list(g["flushed_at"]) and refused == int(g["refused_at"])
    check("after_")


# ------------------------------------------------------------- generated INT4 values (fixtures)
from golden_io import gen_int4_fixture_names  # noqa: E402


@pytest.mark.parametrize("name", gen_int4_fixture_names())
def test_generated_int4_values_bit_exact_against_reference_fixtures(name):
    """generated_value_precision="int4" on the GPU against the reference's own cache states: the build
    (the INT4-V arena with room, the INT2-V arena without), every append and flush (the oldest ring
    values packed into the INT4-V arena, their indices into the INT4 pool), then the decode against
    the reference's attention output and against the oracle on the same bf16 query."""
    import r2omni_amd as ro
    from oracle.attention import mixed_reference
    from oracle.cache import append_token, build_cache
    from oracle.quant import bf16_bits_to_f32

    dev = _cuda()
    g = load(name)
    dt = str(g["dtype"])
    key = _to_torch(g["key"], dt, dev)
    value = _to_torch(g["value"], dt, dev)
    plan = ro.plan_from_pages(g["page_offsets"], g["page_lengths"], g["page_classes"], recent_fp_capacity=128,
                              device=dev)
    cache = ro.build_three_precision_cache(
        key, value, plan, page_size=int(g["page_size"]), key_quantization_superblock=int(g["superblock"]),
        int2_group_size=int(g["group"]), compact_key_append_capacity=260, recent_flush_size=128,
        generated_value_precision="int4")
    oc = build_cache(as_f32(g["key"], dt), as_f32(g["value"], dt), g["page_offsets"], g["page_lengths"],
                     g["page_classes"], dtype=dt.replace("torch.", ""), page_size=int(g["page_size"]),
                     superblock=int(g["superblock"]), group=int(g["group"]), recent_capacity=128,
                     append_capacity=260, gen_values="int4")
    q = torch.from_numpy(g["query"]).to(dev).to(torch.bfloat16)
    qf = bf16_bits_to_f32(_bf16_np(q))

    def check(prefix):
        torch.cuda.synchronize()
        ck, cv, v4 = cache.compact_key, cache.compact_value, cache.compact_int4_value
        k = ck.active_length
        blocks = -(-k // ck.superblock_size)
        assert k == int(g[prefix + "k_active"]) and ck.capacity == int(g[prefix + "k_capacity"])
        assert cache.generated_k_offset == int(g[prefix + "generated_k_offset"])
        assert cache.static_int4_tokens == int(g[prefix + "static_int4_tokens"])
        np.testing.assert_array_equal(ck.packed[:, :k].cpu().numpy(), g[prefix + "k_packed"])
        np.testing.assert_array_equal(_bits16(ck.scale[:, :blocks]), g[prefix + "k_scale"].view(np.uint16))
        np.testing.assert_array_equal(ck.zero_point[:, :blocks].cpu().numpy(), g[prefix + "k_zero"])
        n4 = v4.active_length
        assert n4 == int(g[prefix + "v4_active"]) and v4.capacity == int(g[prefix + "v4_capacity"])
        np.testing.assert_array_equal(v4.packed[:, :n4].cpu().numpy(), g[prefix + "v4_packed"])
        np.testing.assert_array_equal(v4.scale[:, :n4].cpu().numpy().view(np.uint32),
                                      g[prefix + "v4_scale"].view(np.uint32))
        a = cv.active_length
        assert a == int(g[prefix + "v2_active"]) and cv.capacity == int(g[prefix + "v2_capacity"])
        np.testing.assert_array_equal(cv.packed[:, :a].cpu().numpy(), g[prefix + "v2_packed"])
        np.testing.assert_array_equal(_bits16(cv.scale[:, :a]), g[prefix + "v2_scale"].view(np.uint16))
        np.testing.assert_array_equal(cv.zero_point[:, :a].cpu().numpy(), g[prefix + "v2_zero"])
        if cache.fp_pool.token_count:
            np.testing.assert_array_equal(_bits16(cache.fp_pool.fp_v), g[prefix + "fp_v"].view(np.uint16))
        rec = cache.recent_fp_pool
        r = rec.active_length
        assert r == int(g[prefix + "recent_active"]) == int(rec.length_device.item())
        np.testing.assert_array_equal(_bits16(rec.fp_k[:, :r]), g[prefix + "recent_k"].view(np.uint16))
        np.testing.assert_array_equal(_bits16(rec.fp_v[:, :r]), g[prefix + "recent_v"].view(np.uint16))
        np.testing.assert_array_equal(rec.global_index_buffer[:r].cpu().numpy(), g[prefix + "recent_global"])
        i4, i2 = cache.int4_pool, cache.int2_pool
        pools = [cache.fp_pool.token_count, i4.token_count, i2.token_count, r]
        assert pools == [int(v) for v in g[prefix + "pool_tokens"]]
        np.testing.assert_array_equal(i4.page_index.global_token_indices[: i4.token_count].cpu().numpy(),
                                      g[prefix + "int4_global"])
        np.testing.assert_array_equal(i4.page_index.logical_positions[: i4.token_count].cpu().numpy(),
                                      g[prefix + "int4_logical"])
        np.testing.assert_array_equal(i2.page_index.global_token_indices[: i2.token_count].cpu().numpy(),
                                      g[prefix + "int2_global"])
        ws = ro.allocate_splitk_workspace(cache, num_query_heads=int(q.shape[1]))
        out = ro.prepare_splitk_executor(cache, ws)(q)
        torch.cuda.synchronize()
        print(f"[gen-int4] {name} {prefix}decode", flush=True)
        _compare(out, mixed_reference(qf, oc), f"{name} {prefix}decode vs oracle")
        _compare(out, g[prefix + "attn"].reshape(out.shape), f"{name} {prefix}decode vs reference")

    stats = ro.DynamicCacheStats()
    check("build_")
    ak = _to_torch(g["append_k"], dt, dev)
    av = _to_torch(g["append_v"], dt, dev)
    seq = int(g["key"].shape[1])
    flushed = []
    for step in range(int(ak.shape[0])):
        if ro.append_generated_token(cache, ak[step], av[step], global_token_index=seq + step,
                                     logical_position=seq + step, stats=stats):
            flushed.append(step)
        append_token(oc, as_f32(g["append_k"][step, :, 0], dt), as_f32(g["append_v"][step, :, 0], dt),
                     global_index=seq + step, logical_position=seq + step)
    assert flushed == list(g["flushed_at"])
    assert stats.local_tail_dequant_tokens == int(g["tail_dequant_tokens"])
    check("after_")
