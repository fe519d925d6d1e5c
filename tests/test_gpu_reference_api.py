"""The package's triton_mixed_reference (the manager's correctness mode, run as torch ops on the cache's
device) against the CPU oracle: every cache variant, at build time and after a flush, within one
output rounding (the GPU sums in another order), and against the decode executor at the decode bar."""
import numpy as np
import pytest
import torch

from test_gpu_parity import _bf16_np, _compare, _cuda, _oracle_for

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("variant", ["int4k", "int2k", "bf16k", "matched"])
def test_triton_mixed_reference_matches_oracle(variant):
    import r2omni_amd as ro
    from r2omni_amd.workloads import DecodeConfig, build_request_cache, make_request
    from oracle.attention import mixed_reference
    from oracle.cache import append_token
    from oracle.quant import bf16_bits_to_f32

    dev = _cuda()
    recent = 60 if variant == "bf16k" else 127  # v_fourq_k_bf16 has no flush
    cfg = DecodeConfig("t", 28, 4, (0,), (0.15, 0.45, 0.4), recent=recent, variant=variant)
    data = make_request(cfg, 1536 + recent, seed=600, device=dev)
    cache = build_request_cache(cfg, data)
    oc = _oracle_for(data, cfg)
    f32 = lambda t: bf16_bits_to_f32(_bf16_np(t))  # noqa: E731
    gen = torch.Generator(device=dev).manual_seed(601)
    stats = ro.DynamicCacheStats()
    pos = int(data.key.shape[1]) + recent
    for step in range(3):
        q = torch.randn(1, 28, 128, generator=gen, device=dev).to(torch.bfloat16)
        print(f"[reference] {variant} step {step}: pools {[p.token_count for p in cache.pools]}", flush=True)
        got = ro.triton_mixed_reference(q, cache)
        assert got.dtype == torch.bfloat16 and tuple(got.shape) == (1, 28, 128)
        want = mixed_reference(f32(q), oc)
        g = got.float().cpu().numpy()
        assert np.all(np.abs(g - want) <= np.abs(want) * 2.0 ** -7 + 1e-6), f"step {step}"
        ex = ro.prepare_splitk_executor(cache, ro.allocate_splitk_workspace(cache, num_query_heads=28))
        _compare(ex(q), g, f"{variant} executor vs reference step {step}")
        k = torch.randn(4, 1, 128, generator=gen, device=dev).to(torch.bfloat16)
        v = torch.randn(4, 1, 128, generator=gen, device=dev).to(torch.bfloat16)
        ro.append_generated_token(cache, k, v, global_token_index=pos, logical_position=pos, stats=stats)
        append_token(oc, f32(k[:, 0]), f32(v[:, 0]), global_index=pos, logical_position=pos)
        pos += 1
        torch.cuda.synchronize()
    assert stats.flushed_tokens == (0 if variant == "bf16k" else 128)
    with pytest.raises(ValueError, match="one decode token"):
        ro.triton_mixed_reference(torch.zeros(1, 28, 2, 128, device=dev, dtype=torch.bfloat16), cache)


def test_triton_mixed_reference_on_an_fp16_cache():
    """fp16 caches (the reference runner's --model_dtype float16) in the correctness mode."""
    import r2omni_amd as ro
    from golden_io import as_f32, load
    from oracle.attention import mixed_reference
    from oracle.cache import build_cache

    dev = _cuda()
    g = load("qwen_pages64_fp16")
    key = torch.from_numpy(np.ascontiguousarray(g["key"])).to(dev)
    value = torch.from_numpy(np.ascontiguousarray(g["value"])).to(dev)
    assert key.dtype == torch.float16
    plan = ro.plan_from_pages(g["page_offsets"], g["page_lengths"], g["page_classes"], recent_fp_capacity=128,
                              device=dev)
    cache = ro.build_three_precision_cache(key, value, plan, page_size=int(g["page_size"]),
                                           key_quantization_superblock=int(g["superblock"]),
                                           int2_group_size=int(g["group"]), compact_key_append_capacity=260)
    oc = build_cache(as_f32(g["key"], "float16"), as_f32(g["value"], "float16"), g["page_offsets"],
                     g["page_lengths"], g["page_classes"], dtype="float16", page_size=int(g["page_size"]),
                     superblock=int(g["superblock"]), group=int(g["group"]))
    q = torch.randn(1, int(g["query"].shape[1]), 128, generator=torch.Generator(device=dev).manual_seed(602),
                    device=dev).to(torch.float16)
    got = ro.triton_mixed_reference(q, cache)
    assert got.dtype == torch.float16
    want = mixed_reference(q.float().cpu().numpy(), oc)
    assert np.all(np.abs(got.float().cpu().numpy() - want) <= np.abs(want) * 2.0 ** -10 + 1e-6)
