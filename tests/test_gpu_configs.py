"""Parity at the full sizes of the benchmark configurations 0-4 (the bench's layer-0 data).

Each configuration is built on the GPU from ``workloads.CONFIGS`` with the seeds bench.py uses for
its first layer cache, and checked against the CPU oracle built from the same bf16 K/V:
  * every arena byte, scale and zero point (compact K, INT4-V, INT2-V), the FP-V rows and the
    Recent-FP ring, bit for bit;
  * the decode of every request within max-abs 2e-2 / mean-abs 2e-3 of the fp32
    dequantise-then-softmax oracle (triton_fourq_attention.py:72-125), through the executor the
    bench times (stacked for the ragged batch), with the output FWHT on and, for the ragged
    batch, off;
  * configuration 1: its 64 single-token steps (the first flushes the full ring into INT4-K and
    INT2-V, dynamic_fourq_cache.py:172-267; the other 63 are fused appends), each step's output
    against the oracle, and the arenas and ring after the last step;
  * configuration 4: the 28-layer decoder at 8 x 32768 tokens (properties and one layer's
    attention against the oracle, see its test).
"""
import numpy as np
import pytest
import torch

from test_gpu_parity import MAX_ABS, MEAN_ABS, _bf16_np, _check_k_arena, _cuda

pytestmark = pytest.mark.gpu


def _f32(t):
    """bf16 or fp16 values as float32 (exact for both)."""
    if t.dtype == torch.float16:
        return t.detach().float().cpu().numpy()
    from oracle.quant import bf16_bits_to_f32

    return bf16_bits_to_f32(_bf16_np(t))


def _layer0(cfg_id, dev, gen_values="int2"):
    """The bench's layer-0 requests of configuration ``cfg_id`` (seed 1000 * layer + request)."""
    import dataclasses

    from r2omni_amd.workloads import CONFIGS, build_request_cache, make_request

    cfg = dataclasses.replace(CONFIGS[cfg_id], gen_values=gen_values)
    datas = [make_request(cfg, total, seed=r, device=dev) for r, total in enumerate(cfg.lengths)]
    caches = [build_request_cache(cfg, d) for d in datas]
    return cfg, datas, caches


def _oracle(data, cfg):
    from oracle.cache import append_token, build_cache

    oc = build_cache(_f32(data.key), _f32(data.value), data.page_offsets.numpy(), data.page_lengths.numpy(),
                     data.page_classes.numpy(), dtype=cfg.dtype, page_size=cfg.page, superblock=cfg.superblock,
                     group=cfg.group, recent_capacity=128, append_capacity=260, variant=cfg.variant,
                     gen_values=cfg.gen_values)
    hist = int(data.key.shape[1])
    rk, rv = _f32(data.recent_k), _f32(data.recent_v)
    for i in range(rk.shape[0]):
        append_token(oc, rk[i], rv[i], global_index=hist + i, logical_position=hist + i)
    return oc


def _check_arenas(cache, oc, what):
    """K arena, value pools and ring of the GPU cache equal the oracle's, bit for bit."""
    _check_k_arena(cache, oc)
    h = oc.hkv
    assert [cache.fp_pool.token_count, cache.int4_pool.token_count,
            0 if cache.compact_value is None else cache.compact_value.active_length] == list(oc.pool_tokens), what
    if cache.fp_pool.token_count:
        np.testing.assert_array_equal(_f32(cache.fp_pool.fp_v[:, : cache.fp_pool.token_count]), oc.fp_v)
    i4 = cache.int4_pool
    if i4.token_count:  # the PackedTensor of the released mode, or the INT4-V arena (rows up to its capacity)
        n = i4.token_count
        np.testing.assert_array_equal(i4.packed_v.packed.cpu().numpy().reshape(h, -1, 64)[:, :n], oc.v4_packed[:, :n])
        np.testing.assert_array_equal(i4.packed_v.scale.cpu().numpy().reshape(h, -1, 1)[:, :n].view(np.uint32),
                                      oc.v4_scale[:, :n].view(np.uint32))
    cv = cache.compact_value
    if cv is not None and cv.active_length:
        a = cv.active_length
        np.testing.assert_array_equal(cv.packed[:, :a].cpu().numpy(), oc.v2_packed[:, :a])
        np.testing.assert_array_equal(cv.scale[:, :a].cpu().view(torch.int16).numpy().view(np.uint16),
                                      oc.v2_scale[:, :a].view(np.uint16))
        np.testing.assert_array_equal(cv.zero_point[:, :a].cpu().numpy(), oc.v2_zero[:, :a])
    rec = cache.recent_fp_pool
    r = rec.active_length
    assert r == oc.recent_active and int(rec.length_device.item()) == r, what
    np.testing.assert_array_equal(_f32(rec.fp_k[:, :r]), oc.recent_k[:, :r])
    np.testing.assert_array_equal(_f32(rec.fp_v[:, :r]), oc.recent_v[:, :r])
    np.testing.assert_array_equal(rec.global_index_buffer[:r].cpu().numpy(), oc.recent_global[:r])
    np.testing.assert_array_equal(rec.page_index.lengths.cpu().numpy(), oc.recent_page_lengths)


def _errors(got_bf16, want, what):
    got = got_bf16.float().cpu().numpy()
    err = np.abs(got - want)
    assert np.isfinite(got).all(), what
    assert err.max() <= MAX_ABS and err.mean() <= MEAN_ABS, f"{what}: max-abs {err.max():.3e} mean-abs {err.mean():.3e}"
    return float(err.max()), float(err.mean())


@pytest.mark.parametrize("cfg_id", [0, 2, 3])
def test_config_full_size_arenas_and_decode_match_oracle(cfg_id):
    import r2omni_amd as ro
    from oracle.attention import mixed_reference, output_transform

    dev = _cuda()
    print(f"[cfg{cfg_id}] building the layer-0 caches at full size", flush=True)
    cfg, datas, caches = _layer0(cfg_id, dev)
    torch.cuda.synchronize()
    ocs = []
    for r, (d, c) in enumerate(zip(datas, caches)):
        oc = _oracle(d, cfg)
        _check_arenas(c, oc, f"cfg{cfg_id} request {r}")
        ocs.append(oc)
    print(f"[cfg{cfg_id}] arenas bit-exact for {len(caches)} request(s), "
          f"{sum(c.compact_key.active_length for c in caches)} history tokens per head", flush=True)
    want_raw = [mixed_reference(_f32(d.query), oc) for d, oc in zip(datas, ocs)]
    q = torch.cat([d.query for d in datas]).contiguous()
    for hadamard in ((False, True) if len(caches) > 1 else (True,)):
        exs = [ro.prepare_splitk_executor(c, ro.allocate_splitk_workspace(c, num_query_heads=cfg.hq),
                                          output_hadamard=hadamard) for c in caches]
        ex = exs[0] if len(exs) == 1 else ro.stack_homogeneous_splitk_executors(exs)
        print(f"[cfg{cfg_id}] decode, hadamard {hadamard}, {ex.n_items} work items", flush=True)
        out = ex(q)
        torch.cuda.synchronize()
        for r in range(len(caches)):
            mx, mn = _errors(out[r : r + 1], output_transform(want_raw[r], hadamard),
                             f"cfg{cfg_id} request {r} hadamard {hadamard}")
            print(f"[cfg{cfg_id}] request {r} ({cfg.lengths[r]} tokens): max-abs {mx:.2e} mean-abs {mn:.2e}",
                  flush=True)


@pytest.mark.parametrize("gen_values", ["int2", "int4"])
def test_config1_sixty_four_steps_with_flush_match_oracle(gen_values):
    """Configuration 1's decode loop as the manager runs it (qwen_sspa_attention.py:1794-1826): the
    first token finds the ring full and goes through append_generated_token (flush of 128 tokens
    into INT4-K and INT2-V, or INT4-V with INT4 generated values, then the ring append) and a
    re-prepared executor; the next 63 are fused into the split-K call."""
    import r2omni_amd as ro
    from oracle.attention import mixed_reference, output_transform
    from oracle.cache import append_token

    dev = _cuda()
    print(f"[cfg1] building the layer-0 cache at full size, generated values {gen_values}", flush=True)
    cfg, (data,), (cache,) = _layer0(1, dev, gen_values)
    oc = _oracle(data, cfg)
    _check_arenas(cache, oc, "cfg1 build")
    ws = ro.allocate_splitk_workspace(cache, num_query_heads=cfg.hq)
    ex = ro.prepare_splitk_executor(cache, ws, output_hadamard=True)
    stats = ro.DynamicCacheStats()
    gen = torch.Generator(device=dev).manual_seed(101)
    pos = int(data.key.shape[1]) + cfg.recent
    worst = [0.0, 0.0]
    for step in range(64):
        q = torch.randn(1, cfg.hq, 128, generator=gen, device=dev).to(torch.bfloat16)
        k = torch.randn(1, cfg.hkv, 128, generator=gen, device=dev).to(torch.bfloat16)
        v = torch.randn(1, cfg.hkv, 128, generator=gen, device=dev).to(torch.bfloat16)
        rec = cache.recent_fp_pool
        if rec.active_length < rec.capacity:
            out = ex(q, append=(k, v, pos, pos))
            rec.active_length += 1
            want = mixed_reference(_f32(q), oc, append=(_f32(k[0]), _f32(v[0])))
            append_token(oc, _f32(k[0]), _f32(v[0]), global_index=pos, logical_position=pos)
        else:
            assert step == 0, "only the first step finds the ring full"
            assert ro.append_generated_token(cache, k[0][:, None], v[0][:, None], global_token_index=pos,
                                             logical_position=pos, stats=stats)
            ex = ro.prepare_splitk_executor(cache, ws, output_hadamard=True)
            assert append_token(oc, _f32(k[0]), _f32(v[0]), global_index=pos, logical_position=pos)
            out = ex(q)
            want = mixed_reference(_f32(q), oc)
        torch.cuda.synchronize()
        mx, mn = _errors(out, output_transform(want, True), f"cfg1 step {step}")
        worst = [max(worst[0], mx), max(worst[1], mn)]
        if step in (0, 1, 63):
            print(f"[cfg1] step {step}: max-abs {mx:.2e} mean-abs {mn:.2e}", flush=True)
        pos += 1
    assert stats.flushed_tokens == 128 and cache.recent_fp_pool.active_length == 64
    assert stats.flushed_int4_value_tokens == (128 if gen_values == "int4" else 0)
    _check_arenas(cache, oc, "cfg1 after 64 steps")
    print(f"[cfg1] 64 steps: worst max-abs {worst[0]:.2e}, worst mean-abs {worst[1]:.2e}", flush=True)


def test_config4_e2e_decode_properties():
    """Configuration 4 at full size: a random-init 28-layer Qwen2.5-Omni-7B decoder prefilled to
    8 x 32768 tokens, then greedy steps on this path (bench.py's E2EQwenDecoder).  The first step
    flushes every ring inside the batch; after it, the last layer's attention output of every request
    is checked against the oracle (cache rebuilt on the CPU from the same K/V, the step's token
    appended with its flush) and the arenas against the oracle's bit for bit.  After the last step the
    same checks run again on that layer, its oracle cache taking every step's appended token (the first
    one's flush, then the ring appends), so the fused appends of later steps are pinned too (the last
    layer's raw projections are the ones left in the shared projection buffer).  Logits stay finite,
    and the tokens of the HIP-graph run equal those of the eager run and of a run with a separate
    rotation launch (the decoder folds the mRoPE / FWHT into the attention call)."""
    import bench
    import r2omni_amd as ro
    from oracle.attention import mixed_reference, output_transform
    from oracle.cache import append_token

    dev = _cuda()
    steps = 4
    print("[cfg4] random-init 28-layer 7B decoder, prefill 8 x 32768 tokens", flush=True)
    model = bench.E2EQwenDecoder(dev, batch=8, context=32768, n_layers=28)
    model.prefill()
    layer = model.n_layers - 1
    cfg = model.cache_config()
    checked = {}
    rows = {}  # (layer, step) -> the step's rotated q, k, v rows (float32)

    def step_rows(d):
        if d.rotary is not None:  # raw projections in the bound inputs: the rows the call rotated
            rot = d.rotary
            qr, _ = ro.qwen_qk_mrope(d.query_buffer[:, :, None], d.key_buffer[:, :, None], rot.cos, rot.sin,
                                     rot.mrope_section, apply_hadamard=rot.apply_hadamard)
            return _f32(qr[:, :, 0]), _f32(d.executor.rotated_k), _f32(d.executor.rotated_v)
        return _f32(d.query_buffer), _f32(d.key_buffer), _f32(d.value_buffer)

    def check_layer(step, d, lay):
        out = d.workspace.output.clone()
        q = rows[(lay, step)][0]
        worst = []
        for s_i in range(model.batch):
            oc = _oracle(model.request_data(lay, s_i), cfg)
            for i in range(step + 1):  # the tokens of steps 0 .. step (the first flushes the full ring)
                _, k, v = rows[(lay, i)]
                flushed = append_token(oc, k[s_i], v[s_i], global_index=model.context + i,
                                       logical_position=model.context + i)
                assert flushed == (i == 0), f"cfg4 layer {lay} step {i}: flush expected only at the first step"
            _check_arenas(d.caches[s_i], oc, f"cfg4 layer {lay} step {step} request {s_i}")
            worst.append(_errors(out[s_i : s_i + 1], output_transform(mixed_reference(q[s_i : s_i + 1], oc), True),
                                 f"cfg4 layer {lay} step {step} request {s_i}"))
        checked[(lay, step)] = worst
        print(f"[cfg4] layer {lay} step {step}, 8 requests: worst max-abs {max(c[0] for c in worst):.2e}, "
              f"worst mean-abs {max(c[1] for c in worst):.2e}", flush=True)

    def inspect(step, decs):
        rows[(layer, step)] = step_rows(decs[layer])
        if step in (0, steps - 1):
            check_layer(step, decs[layer], layer)

    print("[cfg4] eager decode", flush=True)
    _, eager_tokens, eager_finite = model.decode(steps, False, inspect)
    print("[cfg4] HIP-graph decode", flush=True)
    _, graph_tokens, graph_finite = model.decode(steps, True)
    print("[cfg4] HIP-graph decode with a separate rotation launch", flush=True)
    _, sep_tokens, sep_finite = model.decode(steps, True, fused_rotation=False)
    assert sorted(checked) == [(layer, 0), (layer, steps - 1)] and all(len(w) == model.batch for w in checked.values())
    assert eager_finite and graph_finite and sep_finite
    assert torch.equal(eager_tokens, graph_tokens) and torch.equal(sep_tokens, graph_tokens)
    print(f"[cfg4] tokens of {steps} greedy steps equal in both modes", flush=True)


TIER_CASES = {
    # (key variant, V tier probabilities BF16/INT4/INT2, superblock = group)
    "bf16v": ("int4k", (1.0, 0.0, 0.0), 32),
    "int4v": ("int4k", (0.0, 1.0, 0.0), 32),
    "int2v": ("int4k", (0.0, 0.0, 1.0), 32),
    "int2v_int2k_sb128": ("int2k", (0.0, 0.0, 1.0), 128),
}


@pytest.mark.parametrize("case", sorted(TIER_CASES))
def test_value_tier_error_at_full_size(case):
    """The attention error of each value tier alone over a 65,536-token request at the cfg2 head
    geometry (Hq 28 / Hkv 4): BF16-V and Recent-FP tiles feed P to the MFMA in bf16, INT4-V and INT2-V
    tiles feed P' = p * scale in f16, where the reference's B=1 kernel keeps P in fp32
    (triton_fourq_splitk.py:456-931).  Every case stays inside the parity bar."""
    import dataclasses

    import r2omni_amd as ro
    from oracle.attention import mixed_reference, output_transform
    from r2omni_amd.workloads import CONFIGS, build_request_cache, make_request

    dev = _cuda()
    variant, probs, sb = TIER_CASES[case]
    cfg = dataclasses.replace(CONFIGS[2], name=case, lengths=(65536,), tier_probs=probs, variant=variant,
                              superblock=sb, group=sb)
    data = make_request(cfg, 65536, seed=7, device=dev)
    cache = build_request_cache(cfg, data)
    oc = _oracle(data, cfg)
    _check_arenas(cache, oc, case)
    ex = ro.prepare_splitk_executor(cache, ro.allocate_splitk_workspace(cache, num_query_heads=cfg.hq),
                                    output_hadamard=False)
    out = ex(data.query)
    torch.cuda.synchronize()
    mx, mn = _errors(out, output_transform(mixed_reference(_f32(data.query), oc), False), case)
    print(f"[tier {case}] 65536 tokens, {ex.n_items} work items: max-abs {mx:.2e} mean-abs {mn:.2e}", flush=True)


def test_config2_fp16_model_full_size_matches_oracle():
    """Configuration 2 for an fp16 model (the reference runner's --model_dtype float16,
    benchmark_mixed_active.py:1255-1263) at full size: arenas and fp16 rows bit-exact against the
    oracle, the decode of every request (the fp16-row kernel instances) within the bar."""
    import dataclasses

    import r2omni_amd as ro
    from oracle.attention import mixed_reference, output_transform
    from r2omni_amd.workloads import CONFIGS, build_request_cache, make_request

    dev = _cuda()
    cfg = dataclasses.replace(CONFIGS[2], dtype="float16")
    datas = [make_request(cfg, total, seed=r, device=dev) for r, total in enumerate(cfg.lengths)]
    caches = [build_request_cache(cfg, d) for d in datas]
    torch.cuda.synchronize()
    assert caches[0].recent_fp_pool.fp_k.dtype == torch.float16
    ocs = []
    for r, (d, c) in enumerate(zip(datas, caches)):
        oc = _oracle(d, cfg)
        _check_arenas(c, oc, f"cfg2 fp16 request {r}")
        ocs.append(oc)
    exs = [ro.prepare_splitk_executor(c, ro.allocate_splitk_workspace(c, num_query_heads=cfg.hq),
                                      output_hadamard=True) for c in caches]
    ex = ro.stack_homogeneous_splitk_executors(exs)
    q = torch.cat([d.query for d in datas]).contiguous()
    out = ex(q)
    torch.cuda.synchronize()
    for r, (d, oc) in enumerate(zip(datas, ocs)):
        mx, mn = _errors(out[r : r + 1], output_transform(mixed_reference(_f32(d.query), oc), True),
                         f"cfg2 fp16 request {r}")
        print(f"[cfg2 fp16] request {r} ({cfg.lengths[r]} tokens): max-abs {mx:.2e} mean-abs {mn:.2e}", flush=True)
