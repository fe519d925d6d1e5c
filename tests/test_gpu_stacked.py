"""Stacked executors keep private Recent-FP rings and lengths, as the reference's batched executor
does (triton_fourq_splitk.py:2194-2241, :1543-1546): the manager may stack one B=1 executor B times
(enable_homogeneous_decode_batch, qwen_sspa_attention.py:278-317) and advance its own cache's host
length after every fused append (:1824-1826) without the requests sharing a ring."""
import numpy as np
import pytest
import torch

from test_gpu_parity import _bf16_np, _compare, _cuda, _oracle_for

pytestmark = pytest.mark.gpu


def test_stacked_same_executor_twice_with_fused_appends():
    import r2omni_amd as ro
    from r2omni_amd.workloads import DecodeConfig, build_request_cache, make_request
    from oracle.attention import mixed_reference, output_transform
    from oracle.cache import append_token
    from oracle.quant import bf16_bits_to_f32

    dev = _cuda()
    cfg = DecodeConfig("t", 16, 2, (0,), (0.2, 0.5, 0.3), recent=126)
    data = make_request(cfg, 1024 + 126, seed=21, device=dev)
    cache = build_request_cache(cfg, data)
    src = cache.recent_fp_pool
    src_k, src_v = src.fp_k.clone(), src.fp_v.clone()
    src_global = src.global_index_buffer.clone()
    ws = ro.allocate_splitk_workspace(cache, num_query_heads=16)
    ex = ro.prepare_splitk_executor(cache, ws, output_hadamard=True)
    batched = ro.stack_homogeneous_splitk_executors((ex,) * 2)
    print("[stacked] (ex,)*2 over a 1150-token cache, ring 126/128", flush=True)
    ocs = [_oracle_for(data, cfg) for _ in range(2)]
    f32 = lambda t: bf16_bits_to_f32(_bf16_np(t))  # noqa: E731
    gen = torch.Generator(device=dev).manual_seed(22)
    hist = int(data.key.shape[1]) + 126
    for step in range(2):
        q = torch.randn(2, 16, 128, generator=gen, device=dev).to(torch.bfloat16)
        k = torch.randn(2, 2, 128, generator=gen, device=dev).to(torch.bfloat16)
        v = torch.randn(2, 2, 128, generator=gen, device=dev).to(torch.bfloat16)
        pos = hist + step
        out = batched(q, append=(k, v, pos, pos))
        src.active_length += 1  # the manager's bookkeeping on request 0's source cache
        torch.cuda.synchronize()
        for r in range(2):
            want = mixed_reference(f32(q[r : r + 1]), ocs[r], append=(f32(k[r]), f32(v[r])))
            append_token(ocs[r], f32(k[r]), f32(v[r]), global_index=pos, logical_position=pos)
            _compare(out[r : r + 1], output_transform(want, True), f"step {step} request {r}")
    assert batched.batched_recent_lengths == [128, 128]
    for r in range(2):
        ring = batched.batched_recent[r]
        assert int(ring.length_device.item()) == 128
        np.testing.assert_array_equal(f32(ring.fp_k), ocs[r].recent_k[:, :128])
        np.testing.assert_array_equal(f32(ring.fp_v), ocs[r].recent_v[:, :128])
        np.testing.assert_array_equal(ring.global_index_buffer.cpu().numpy(), ocs[r].recent_global[:128])
        np.testing.assert_array_equal(ring.page_index.lengths.cpu().numpy(), ocs[r].recent_page_lengths)
    # the source cache's ring was never written (its host length is the caller's business)
    assert int(src.length_device.item()) == 126
    assert torch.equal(src.fp_k.view(torch.int16), src_k.view(torch.int16))
    assert torch.equal(src.fp_v.view(torch.int16), src_v.view(torch.int16))
    assert torch.equal(src.global_index_buffer, src_global)
    # both private rings are full: a third fused append is refused before any launch
    q = torch.zeros(2, 16, 128, device=dev, dtype=torch.bfloat16)
    kv = torch.zeros(2, 2, 128, device=dev, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="full Recent-FP pool"):
        batched(q, append=(kv, kv, hist + 2, hist + 2))
    # decoding without an append still reads the 128 private rows of each request
    out = batched(q)
    torch.cuda.synchronize()
    for r in range(2):
        _compare(out[r : r + 1], output_transform(mixed_reference(np.zeros((1, 16, 128), np.float32), ocs[r]), True),
                 f"no-append request {r}")


def test_batched_decoder_refuses_a_repeated_cache():
    import r2omni_amd as ro
    from r2omni_amd.workloads import DecodeConfig, build_request_cache, make_request

    dev = _cuda()
    cfg = DecodeConfig("t", 16, 2, (0,), (0.2, 0.5, 0.3), recent=64)
    cache = build_request_cache(cfg, make_request(cfg, 512 + 64, seed=23, device=dev))
    with pytest.raises(ValueError, match="distinct caches"):
        ro.BatchedDecoder([cache, cache], num_query_heads=16, use_graph=False)
