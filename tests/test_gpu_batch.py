"""GPU checks of BatchedDecoder: flushes inside a ragged batch, eager and HIP-graph replay.

Every step of every request is compared with the CPU oracle (append then dequantise-then-softmax),
to the same bar as the other decode tests (max-abs 2e-2, mean-abs 2e-3).
"""
import numpy as np
import pytest
import torch

from test_gpu_parity import _bf16_np, _check_k_arena, _compare, _cuda, _oracle_for

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("use_graph", [True, False])
@pytest.mark.parametrize("variant,gen_values", [("int4k", "int2"), ("int2k", "int2"), ("matched", "int2"),
                                                ("int4k", "int4")])
def test_batched_decoder_flushes_inside_the_batch(variant, gen_values, use_graph):
    import r2omni_amd as ro
    from r2omni_amd.workloads import DecodeConfig, build_request_cache, make_request
    from oracle.attention import mixed_reference
    from oracle.cache import append_token
    from oracle.quant import bf16_bits_to_f32

    dev = _cuda()
    hq, hkv = 28, 4
    # ragged histories, rings 3, 7 and 12 tokens short of full: each request flushes at a different step
    shapes = [(1024, 125), (2048, 121), (640, 116)]
    cfgs, datas, caches, oracles = [], [], [], []
    for r, (hist, recent) in enumerate(shapes):
        cfg = DecodeConfig("b", hq, hkv, (0,), (0.15, 0.45, 0.4), recent=recent, variant=variant,
                           gen_values=gen_values)
        data = make_request(cfg, hist + recent, seed=500 + r, device=dev)
        cfgs.append(cfg)
        datas.append(data)
        caches.append(build_request_cache(cfg, data))
        oracles.append(_oracle_for(data, cfg))
    dec = ro.BatchedDecoder(caches, num_query_heads=hq, output_hadamard=False,
                            use_graph=use_graph)
    gen = torch.Generator(device=dev).manual_seed(9)
    pos = [hist + recent for hist, recent in shapes]
    steps = 16
    for step in range(steps):
        q = torch.randn(3, hq, 128, generator=gen, device=dev).to(torch.bfloat16)
        k = torch.randn(3, hkv, 128, generator=gen, device=dev).to(torch.bfloat16)
        v = torch.randn(3, hkv, 128, generator=gen, device=dev).to(torch.bfloat16)
        print(f"[batch {variant} gen={gen_values} graph={use_graph}] step {step}", flush=True)
        out = dec.step(q, k, v, global_token_index=pos, logical_position=pos)
        torch.cuda.synchronize()
        for r in range(3):
            kf, vf = bf16_bits_to_f32(_bf16_np(k[r])), bf16_bits_to_f32(_bf16_np(v[r]))
            append_token(oracles[r], kf, vf, global_index=pos[r], logical_position=pos[r])
            want = mixed_reference(bf16_bits_to_f32(_bf16_np(q[r : r + 1])), oracles[r])
            _compare(out[r : r + 1], want, f"{variant} graph={use_graph} step {step} request {r}")
        pos = [p + 1 for p in pos]
    for r, (c, oc, st) in enumerate(zip(caches, oracles, dec.stats)):
        rec = c.recent_fp_pool
        assert rec.active_length == oc.recent_active, r
        assert int(rec.length_device.item()) == oc.recent_active, r
        np.testing.assert_array_equal(rec.global_index_buffer[: rec.active_length].cpu().numpy(),
                                      oc.recent_global[: oc.recent_active])
        np.testing.assert_array_equal(rec.logical_position_buffer[: rec.active_length].cpu().numpy(),
                                      oc.recent_logical[: oc.recent_active])
        assert st.flushed_tokens == 128 and st.appended_tokens == steps
        r_act = rec.active_length  # every ring row the fused appends wrote, bit for bit
        np.testing.assert_array_equal(bf16_bits_to_f32(_bf16_np(rec.fp_k[:, :r_act])), oc.recent_k[:, :r_act])
        np.testing.assert_array_equal(bf16_bits_to_f32(_bf16_np(rec.fp_v[:, :r_act])), oc.recent_v[:, :r_act])
        _check_k_arena(c, oc)
        if gen_values == "int4":  # the flushed values went to the INT4-V arena, bit for bit
            a4, n4 = c.compact_int4_value, c.int4_pool.token_count
            assert st.flushed_int4_value_tokens == 128 and n4 == oc.pool_tokens[1] == a4.active_length
            np.testing.assert_array_equal(a4.packed[:, :n4].cpu().numpy(), oc.v4_packed[:, :n4])
            np.testing.assert_array_equal(a4.scale[:, :n4].cpu().numpy(), oc.v4_scale[:, :n4])
    assert dec.replans == 1 + 3  # the initial plan and one per flushing step
    if use_graph:
        assert dec.graph_captures == dec.replans


def test_batched_decoder_positions_that_jump_are_rewritten():
    """A step whose positions are not the previous ones + 1 rewrites the device positions."""
    import r2omni_amd as ro
    from r2omni_amd.workloads import DecodeConfig, build_request_cache, make_request

    dev = _cuda()
    cfg = DecodeConfig("b", 16, 2, (0,), (0.2, 0.5, 0.3), recent=64)
    caches = [build_request_cache(cfg, make_request(cfg, 1024 + 64, seed=600 + r, device=dev)) for r in range(2)]
    dec = ro.BatchedDecoder(caches, num_query_heads=16, use_graph=True)
    q = torch.zeros(2, 16, 128, device=dev, dtype=torch.bfloat16)
    k = torch.zeros(2, 2, 128, device=dev, dtype=torch.bfloat16)
    dec.step(q, k, k, global_token_index=[5000, 7000], logical_position=[5000, 7000])
    dec.step(q, k, k, global_token_index=[5001, 7001], logical_position=[5001, 7001])
    dec.step(q, k, k, global_token_index=[9000, 7002], logical_position=[9100, 7002])
    torch.cuda.synchronize()
    for c, want_g, want_l in zip(caches, ([5000, 5001, 9000], [7000, 7001, 7002]),
                                 ([5000, 5001, 9100], [7000, 7001, 7002])):
        rec = c.recent_fp_pool
        assert rec.active_length == 67
        assert rec.global_index_buffer[64:67].cpu().tolist() == want_g
        assert rec.logical_position_buffer[64:67].cpu().tolist() == want_l


def test_decode_step_graph_over_layers_matches_oracle():
    """Two layers in one captured step graph, each compared with its own oracle across a flush."""
    import r2omni_amd as ro
    from r2omni_amd.workloads import DecodeConfig, build_request_cache, make_request
    from oracle.attention import mixed_reference
    from oracle.cache import append_token
    from oracle.quant import bf16_bits_to_f32

    dev = _cuda()
    hq, hkv = 16, 2
    shapes = [(768, 126), (1280, 126)]
    layers, oracles = [], []
    for layer in range(2):
        caches, ocs = [], []
        for r, (hist, recent) in enumerate(shapes):
            cfg = DecodeConfig("g", hq, hkv, (0,), (0.2, 0.5, 0.3), recent=recent)
            data = make_request(cfg, hist + recent, seed=700 + 10 * layer + r, device=dev)
            caches.append(build_request_cache(cfg, data))
            ocs.append(_oracle_for(data, cfg))
        layers.append(ro.BatchedDecoder(caches, num_query_heads=hq, use_graph=False))
        oracles.append(ocs)
    step_graph = ro.DecodeStepGraph(layers)
    gen = torch.Generator(device=dev).manual_seed(11)
    pos = [hist + recent for hist, recent in shapes]
    for step in range(5):  # the rings fill at step 2 and flush at step 2 (every layer, every request)
        qs, ks, vs = [], [], []
        for d in layers:
            qs.append(torch.randn(2, hq, 128, generator=gen, device=dev).to(torch.bfloat16))
            ks.append(torch.randn(2, hkv, 128, generator=gen, device=dev).to(torch.bfloat16))
            vs.append(torch.randn(2, hkv, 128, generator=gen, device=dev).to(torch.bfloat16))
            d.query_buffer.copy_(qs[-1])
            d.key_buffer.copy_(ks[-1])
            d.value_buffer.copy_(vs[-1])
        print(f"[step graph] step {step}", flush=True)
        outs = step_graph.step_in_place(global_token_index=pos, logical_position=pos)
        torch.cuda.synchronize()
        for layer in range(2):
            for r in range(2):
                kf = bf16_bits_to_f32(_bf16_np(ks[layer][r]))
                vf = bf16_bits_to_f32(_bf16_np(vs[layer][r]))
                append_token(oracles[layer][r], kf, vf, global_index=pos[r], logical_position=pos[r])
                want = mixed_reference(bf16_bits_to_f32(_bf16_np(qs[layer][r : r + 1])), oracles[layer][r])
                _compare(outs[layer][r : r + 1], want, f"step graph step {step} layer {layer} request {r}")
        pos = [p + 1 for p in pos]
    assert step_graph.graph_captures == 2  # the first step and the flush step


@pytest.mark.parametrize("use_graph", [True, False])
def test_steps_queued_behind_a_busy_stream_across_re_plans(use_graph):
    """Steps issued without any host synchronisation while the stream is held busy, across the three
    re-plans of a ragged batch: each re-plan uploads its work items on the upload stream while the
    launches of the previous plan are still queued, and every step must still match the oracle
    (outputs copied out on the stream, compared after one synchronisation at the end)."""
    import r2omni_amd as ro
    from r2omni_amd.workloads import DecodeConfig, build_request_cache, make_request
    from oracle.attention import mixed_reference
    from oracle.cache import append_token
    from oracle.quant import bf16_bits_to_f32

    dev = _cuda()
    hq, hkv = 16, 2
    shapes = [(1024, 125), (2048, 121), (640, 116)]
    caches, oracles = [], []
    for r, (hist, recent) in enumerate(shapes):
        cfg = DecodeConfig("q", hq, hkv, (0,), (0.15, 0.45, 0.4), recent=recent)
        data = make_request(cfg, hist + recent, seed=800 + r, device=dev)
        caches.append(build_request_cache(cfg, data))
        oracles.append(_oracle_for(data, cfg))
    dec = ro.BatchedDecoder(caches, num_query_heads=hq, use_graph=use_graph)
    gen = torch.Generator(device=dev).manual_seed(13)
    steps = 16
    q = torch.randn(steps, 3, hq, 128, generator=gen, device=dev).to(torch.bfloat16)
    k = torch.randn(steps, 3, hkv, 128, generator=gen, device=dev).to(torch.bfloat16)
    v = torch.randn(steps, 3, hkv, 128, generator=gen, device=dev).to(torch.bfloat16)
    pos0 = [hist + recent for hist, recent in shapes]
    torch.cuda.synchronize()
    print(f"[queued steps graph={use_graph}] issuing {steps} steps behind a busy stream", flush=True)
    torch.cuda._sleep(50_000_000)  # a bounded spin: the steps below queue up behind it
    outs = []
    for step in range(steps):
        pos = [p + step for p in pos0]
        outs.append(dec.step(q[step], k[step], v[step], global_token_index=pos, logical_position=pos).clone())
    torch.cuda.synchronize()
    assert dec.replans == 1 + 3
    for step in range(steps):
        for r in range(3):
            p = pos0[r] + step
            append_token(oracles[r], bf16_bits_to_f32(_bf16_np(k[step, r])), bf16_bits_to_f32(_bf16_np(v[step, r])),
                         global_index=p, logical_position=p)
            want = mixed_reference(bf16_bits_to_f32(_bf16_np(q[step, r : r + 1])), oracles[r])
            _compare(outs[step][r : r + 1], want, f"queued graph={use_graph} step {step} request {r}")
