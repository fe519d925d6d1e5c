"""r2o_decode_noalloc (partial states in the library's per-GPU device array) against the workspace
entry points r2o_decode_partial + r2o_decode_combine: the same kernels on the same inputs, so the
outputs must be bit-identical, on consecutive calls whose second input is smaller (fewer work
items, so the array holds stale partials of the first call beyond the second's slots)."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _cuda():
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    return torch.device("cuda:0")


def _executor(cfg, totals, seed, dev, hadamard):
    import r2omni_amd as ro
    from r2omni_amd.workloads import build_request_cache, make_request

    datas = [make_request(cfg, t, seed=seed + i, device=dev) for i, t in enumerate(totals)]
    caches = [build_request_cache(cfg, d) for d in datas]
    exs = [ro.prepare_splitk_executor(c, ro.allocate_splitk_workspace(c, num_query_heads=cfg.hq),
                                      output_hadamard=hadamard) for c in caches]
    ex = exs[0] if len(exs) == 1 else ro.stack_homogeneous_splitk_executors(exs)
    return ex, torch.cat([d.query for d in datas]).contiguous(), caches


def _noalloc(ex, q, out):
    """One r2o_decode_noalloc call through the C-ABI, with NULL workspace pointers."""
    from r2omni_amd import _lib

    p = ex._params(q, out, None)
    p.partial_max = p.partial_sum = p.partial_out = None
    return _lib.load().r2o_decode_noalloc(ctypes.byref(p), ctypes.c_void_p(_lib.stream_of(q.device)))


def test_noalloc_matches_the_workspace_entry_points_on_consecutive_calls():
    from r2omni_amd.workloads import DecodeConfig

    dev = _cuda()
    big_cfg = DecodeConfig("big", 28, 4, (0,), (0.15, 0.45, 0.4), recent=128)
    small_cfg = DecodeConfig("small", 16, 2, (0,), (0.2, 0.5, 0.3), recent=64)
    big, qb, _ = _executor(big_cfg, (4096 + 128, 8192 + 128, 2048 + 128), 400, dev, True)
    small, qs, _ = _executor(small_cfg, (1024 + 64,), 410, dev, False)
    assert small.n_items < big.n_items <= 1024
    for name, ex, q in (("big", big, qb), ("small", small, qs), ("big again", big, qb)):
        print(f"[noalloc] {name}: {ex.n_items} work items, batch {q.shape[0]}", flush=True)
        want = ex(q).clone()
        out = torch.full_like(want, 7.0)
        assert _noalloc(ex, q, out) == 0
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), name


def test_noalloc_fused_append_matches_the_workspace_call():
    """The fused Recent-FP append runs in the same combine launch: output, ring rows and device
    length equal those of the workspace call on an identical cache."""
    from r2omni_amd.workloads import DecodeConfig

    dev = _cuda()
    cfg = DecodeConfig("append", 16, 2, (0,), (0.2, 0.5, 0.3), recent=100)
    ex_a, q, (ca,) = _executor(cfg, (2048 + 100,), 420, dev, True)
    ex_b, _, (cb,) = _executor(cfg, (2048 + 100,), 420, dev, True)
    gen = torch.Generator(device=dev).manual_seed(421)
    for step in range(2):
        print(f"[noalloc] fused append step {step}", flush=True)
        k = torch.randn(1, 2, 128, generator=gen, device=dev).to(torch.bfloat16)
        v = torch.randn(1, 2, 128, generator=gen, device=dev).to(torch.bfloat16)
        pos = 2148 + step
        want = ex_a(q, append=(k, v, pos, pos)).clone()
        got = ex_b.call_noalloc(q, append=(k, v, pos, pos), out=torch.empty_like(want))
        ca.recent_fp_pool.active_length += 1
        cb.recent_fp_pool.active_length += 1
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), step
    ra, rb = ca.recent_fp_pool, cb.recent_fp_pool
    assert int(rb.length_device.item()) == int(ra.length_device.item()) == 102
    assert torch.equal(rb.fp_k.view(torch.int16), ra.fp_k.view(torch.int16))
    assert torch.equal(rb.fp_v.view(torch.int16), ra.fp_v.view(torch.int16))
    assert torch.equal(rb.global_index_buffer, ra.global_index_buffer)


def test_noalloc_rejects_more_work_items_than_it_holds():
    """Checked on the host before any launch."""
    from r2omni_amd import _lib
    from r2omni_amd.workloads import DecodeConfig

    dev = _cuda()
    cfg = DecodeConfig("small", 16, 2, (0,), (0.2, 0.5, 0.3), recent=64)
    ex, q, _ = _executor(cfg, (1024 + 64,), 430, dev, False)
    p = ex._params(q, ex.workspace.output, None)
    p.n_items = _lib.NOALLOC_MAX_ITEMS + 1
    assert _lib.load().r2o_decode_noalloc(ctypes.byref(p), None) == 1
    ex.n_items = _lib.NOALLOC_MAX_ITEMS + 1
    with pytest.raises(ValueError, match="at most"):
        ex.call_noalloc(q)


def test_noalloc_init_checks_the_device_index():
    from r2omni_amd import _lib

    _cuda()
    lib = _lib.load()
    assert lib.r2o_decode_noalloc_init(-1) == 1
    assert lib.r2o_decode_noalloc_init(torch.cuda.device_count()) == 1
    assert lib.r2o_decode_noalloc_init(0) == 0
    assert lib.r2o_decode_noalloc_init(0) == 0  # looked up once; later calls return at once


def test_noalloc_call_captured_in_a_graph_replays_the_eager_result():
    """The callers r2o_decode_noalloc is for capture it: after the set-up call (made by the first
    call_noalloc, outside the capture) the captured launch pair replays bit-identical outputs, also
    when an eager workspace-free call of another cache overwrote the partial-state array between
    the replays."""
    from r2omni_amd.batch import _capture_launches
    from r2omni_amd.workloads import DecodeConfig

    dev = _cuda()
    cfg = DecodeConfig("graph", 28, 4, (0,), (0.15, 0.45, 0.4), recent=128)
    ex, q, _ = _executor(cfg, (4096 + 128, 2048 + 128), 440, dev, True)
    small_cfg = DecodeConfig("small", 16, 2, (0,), (0.2, 0.5, 0.3), recent=64)
    small, qs, _ = _executor(small_cfg, (1024 + 64,), 450, dev, False)
    want_small = small(qs).clone()
    want = ex(q).clone()
    out = torch.full_like(want, 3.0)
    ex.call_noalloc(q, out=out)  # set-up outside the capture
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))
    out.fill_(5.0)
    side = torch.cuda.Stream(device=dev)
    graph = _capture_launches(dev, side, lambda: ex.call_noalloc(q, out=out))
    for replay in range(3):
        print(f"[noalloc] graph replay {replay}", flush=True)
        out.fill_(float(replay + 11))
        other = small.call_noalloc(qs, out=torch.empty_like(want_small))  # the same array, other contents
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(other.view(torch.int16), want_small.view(torch.int16)), replay
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), replay
