"""fp16 caches (the reference runner's --model_dtype float16, benchmark_mixed_active.py:1255-1263):
FP-V rows, the Recent-FP ring and BF16-K rows in fp16, decoded by the fp16-row kernel instances.
The reference converts its rows to fp16 for every dot (triton_fourq_splitk.py:25-59) and writes a
bf16 output (:1653-1655); the oracle is the same fp32 dequantise-then-softmax attention over the
fp16 values.  Bars as for bf16: max-abs 2e-2, mean-abs 2e-3; ring rows bit-exact after appends."""
import numpy as np
import pytest
import torch

from test_gpu_parity import SMALL, _check_k_arena, _compare, _cuda

pytestmark = pytest.mark.gpu


def _f32(t):
    return t.detach().float().cpu().numpy()


def _oracle16(data, cfg):
    from oracle.cache import append_token, build_cache

    c = build_cache(_f32(data.key), _f32(data.value), data.page_offsets.numpy(), data.page_lengths.numpy(),
                    data.page_classes.numpy(), dtype="float16", page_size=cfg.page, superblock=cfg.superblock,
                    group=cfg.group, recent_capacity=128, append_capacity=260, variant=cfg.variant)
    hist = int(data.key.shape[1])
    for i in range(int(data.recent_k.shape[0])):
        append_token(c, _f32(data.recent_k[i]), _f32(data.recent_v[i]), global_index=hist + i, logical_position=hist + i)
    return c


@pytest.mark.parametrize("variant", ["int4k", "int2k", "bf16k", "matched"])
@pytest.mark.parametrize("case", [0, 2, 3])
def test_fp16_cache_decode_matches_oracle(variant, case):
    import r2omni_amd as ro
    from r2omni_amd.workloads import DecodeConfig, build_request_cache, make_request
    from oracle.attention import mixed_reference, output_transform

    dev = _cuda()
    hq, hkv, total, probs, recent, sb, grp = SMALL[case]
    cfg = DecodeConfig("t", hq, hkv, (total,), probs, recent=recent, superblock=sb, group=grp, variant=variant,
                       dtype="float16")
    hist = ((total - recent) // 64) * 64
    data = make_request(cfg, hist + recent, seed=700 + case, device=dev)
    cache = build_request_cache(cfg, data)
    assert cache.recent_fp_pool.fp_k.dtype == torch.float16
    oc = _oracle16(data, cfg)
    _check_k_arena(cache, oc)
    for hadamard in (False, True):
        ex = ro.prepare_splitk_executor(cache, ro.allocate_splitk_workspace(cache, num_query_heads=hq),
                                        output_hadamard=hadamard)
        for qdt in (torch.float16, torch.bfloat16):  # the query may come in either dtype
            q = data.query.to(qdt).contiguous()
            out = ex(q)
            torch.cuda.synchronize()
            assert out.dtype == torch.bfloat16
            _compare(out, output_transform(mixed_reference(_f32(q), oc), hadamard),
                     f"fp16 {variant} case {case} hadamard {hadamard} query {qdt}")


def test_fp16_fused_append_then_flush_matches_oracle():
    """The manager's loop on an fp16 cache: fused appends, the flush of the full ring into fp16-derived
    INT4-K / INT2-V, then fused appends again; ring rows and K arena bit-exact."""
    import r2omni_amd as ro
    from r2omni_amd.workloads import DecodeConfig, build_request_cache, make_request
    from oracle.attention import mixed_reference, output_transform
    from oracle.cache import append_token

    dev = _cuda()
    cfg = DecodeConfig("t", 16, 2, (0,), (0.2, 0.5, 0.3), recent=120, dtype="float16")
    data = make_request(cfg, 1280 + 120, seed=710, device=dev)
    cache = build_request_cache(cfg, data)
    oc = _oracle16(data, cfg)
    ws = ro.allocate_splitk_workspace(cache, num_query_heads=16)
    ex = ro.prepare_splitk_executor(cache, ws)
    gen = torch.Generator(device=dev).manual_seed(711)
    stats = ro.DynamicCacheStats()
    pos = int(data.key.shape[1]) + 120
    for step in range(14):
        q = torch.randn(1, 16, 128, generator=gen, device=dev).to(torch.float16)
        k = torch.randn(1, 2, 128, generator=gen, device=dev).to(torch.float16)
        v = torch.randn(1, 2, 128, generator=gen, device=dev).to(torch.float16)
        rec = cache.recent_fp_pool
        if rec.active_length < rec.capacity:
            out = ex(q, append=(k, v, pos, pos))
            rec.active_length += 1
            want = mixed_reference(_f32(q), oc, append=(_f32(k[0]), _f32(v[0])))
            append_token(oc, _f32(k[0]), _f32(v[0]), global_index=pos, logical_position=pos)
        else:
            assert ro.append_generated_token(cache, k[0][:, None], v[0][:, None], global_token_index=pos,
                                             logical_position=pos, stats=stats)
            ex = ro.prepare_splitk_executor(cache, ws)
            append_token(oc, _f32(k[0]), _f32(v[0]), global_index=pos, logical_position=pos)
            out = ex(q)
            want = mixed_reference(_f32(q), oc)
        torch.cuda.synchronize()
        _compare(out, output_transform(want, False), f"fp16 step {step}")
        pos += 1
    assert stats.flushed_tokens == 128
    rec, r = cache.recent_fp_pool, oc.recent_active
    np.testing.assert_array_equal(_f32(rec.fp_k[:, :r]), oc.recent_k[:, :r])
    np.testing.assert_array_equal(_f32(rec.fp_v[:, :r]), oc.recent_v[:, :r])
    _check_k_arena(cache, oc)
    with pytest.raises(ValueError, match="like the Recent-FP ring"):
        ex(q, append=(k.to(torch.bfloat16), v.to(torch.bfloat16), pos, pos))


@pytest.mark.parametrize("use_graph", [False, True])
def test_fp16_batched_decoder_through_a_flush(use_graph):
    import r2omni_amd as ro
    from r2omni_amd.workloads import DecodeConfig, build_request_cache, make_request
    from oracle.attention import mixed_reference, output_transform
    from oracle.cache import append_token

    dev = _cuda()
    cfg = DecodeConfig("t", 28, 4, (0,), (0.15, 0.45, 0.4), recent=126, dtype="float16")
    datas = [make_request(cfg, t + 126, seed=720 + i, device=dev) for i, t in enumerate((640, 1280))]
    caches = [build_request_cache(cfg, d) for d in datas]
    ocs = [_oracle16(d, cfg) for d in datas]
    dec = ro.BatchedDecoder(caches, num_query_heads=28, output_hadamard=True, use_graph=use_graph)
    gen = torch.Generator(device=dev).manual_seed(721)
    pos = [int(d.key.shape[1]) + 126 for d in datas]
    for step in range(5):  # the third step flushes both rings inside the batch
        q = torch.randn(2, 28, 128, generator=gen, device=dev).to(torch.float16)
        k = torch.randn(2, 4, 128, generator=gen, device=dev).to(torch.float16)
        v = torch.randn(2, 4, 128, generator=gen, device=dev).to(torch.float16)
        out = dec.step(q, k, v, global_token_index=pos, logical_position=pos)
        torch.cuda.synchronize()
        for r in range(2):
            append_token(ocs[r], _f32(k[r]), _f32(v[r]), global_index=pos[r], logical_position=pos[r])
            _compare(out[r : r + 1], output_transform(mixed_reference(_f32(q[r : r + 1]), ocs[r]), True),
                     f"fp16 batch step {step} request {r}")
        pos = [p + 1 for p in pos]
    assert sum(st.flushed_tokens for st in dec.stats) == 256
