"""GPU parity at the edges of the decode path's geometry: the largest and smallest GQA groups, a
one-page cache, and the largest ragged batch the launch accepts (32 requests), each against the CPU
oracle to the decode bar (max-abs 2e-2, mean-abs 2e-3)."""
import pytest
import torch

from test_gpu_parity import _bf16_np, _compare, _cuda, _oracle_for

pytestmark = pytest.mark.gpu

EDGE = [
    # name, hq, hkv, historical tokens, ring tokens, tier probs (BF16, INT4, INT2), superblock, group
    ("gqa16", 32, 2, 1536, 50, (0.2, 0.5, 0.3), 32, 32),
    ("gqa1", 4, 4, 1024, 31, (0.3, 0.4, 0.3), 64, 64),
    ("gqa2_int2", 8, 4, 2048, 128, (0.0, 0.0, 1.0), 128, 128),
    ("one_page", 16, 2, 64, 5, (0.0, 1.0, 0.0), 32, 32),
    ("one_page_bf16", 16, 2, 64, 0, (1.0, 0.0, 0.0), 32, 32),
]


@pytest.mark.parametrize("case", [e[0] for e in EDGE])
@pytest.mark.parametrize("hadamard", [False, True])
def test_edge_geometries_match_oracle(case, hadamard):
    import r2omni_amd as ro
    from r2omni_amd.workloads import DecodeConfig, build_request_cache, make_request
    from oracle.attention import mixed_reference, output_transform
    from oracle.quant import bf16_bits_to_f32

    dev = _cuda()
    _, hq, hkv, hist, recent, probs, sb, grp = next(e for e in EDGE if e[0] == case)
    cfg = DecodeConfig(case, hq, hkv, (hist + recent,), probs, recent=recent, superblock=sb, group=grp)
    data = make_request(cfg, hist + recent, seed=900 + hq + hkv + hist, device=dev)
    cache = build_request_cache(cfg, data)
    ws = ro.allocate_splitk_workspace(cache, num_query_heads=hq)
    ex = ro.prepare_splitk_executor(cache, ws, output_hadamard=hadamard)
    print(f"[edge] {case} hadamard={hadamard}: {ex.n_items} items", flush=True)
    out = ex(data.query.contiguous())
    torch.cuda.synchronize()
    want = output_transform(mixed_reference(bf16_bits_to_f32(_bf16_np(data.query)), _oracle_for(data, cfg)), hadamard)
    _compare(out, want, f"{case} hadamard={hadamard}")


def test_largest_ragged_batch_matches_per_request_oracle():
    """32 requests (the launch maximum) of different lengths, tier mixes and ring fills in one launch."""
    import r2omni_amd as ro
    from r2omni_amd.workloads import DecodeConfig, build_request_cache, make_request
    from oracle.attention import mixed_reference, output_transform
    from oracle.quant import bf16_bits_to_f32

    dev = _cuda()
    gen = torch.Generator().manual_seed(31)
    datas, caches, cfgs = [], [], []
    for r in range(32):
        hist = 64 * int(torch.randint(1, 24, (1,), generator=gen))
        recent = int(torch.randint(0, 129, (1,), generator=gen))
        probs = [(0.15, 0.45, 0.4), (0.0, 1.0, 0.0), (0.0, 0.0, 1.0), (1.0, 0.0, 0.0)][r % 4]
        cfg = DecodeConfig("b32", 28, 4, (hist + recent,), probs, recent=recent)
        data = make_request(cfg, hist + recent, seed=1300 + r, device=dev)
        cfgs.append(cfg)
        datas.append(data)
        caches.append(build_request_cache(cfg, data))
    wss = [ro.allocate_splitk_workspace(c, num_query_heads=28) for c in caches]
    exs = [ro.prepare_splitk_executor(c, w, output_hadamard=True) for c, w in zip(caches, wss)]
    batched = ro.stack_homogeneous_splitk_executors(exs)
    print(f"[edge] batch of 32: {batched.n_items} items", flush=True)
    q = torch.cat([d.query for d in datas]).contiguous()
    out = batched(q)
    torch.cuda.synchronize()
    for r, (d, cfg) in enumerate(zip(datas, cfgs)):
        want = output_transform(mixed_reference(bf16_bits_to_f32(_bf16_np(d.query)), _oracle_for(d, cfg)), True)
        _compare(out[r : r + 1], want, f"batch of 32, request {r}")


def test_batch_above_the_launch_maximum_is_refused():
    import r2omni_amd as ro
    from r2omni_amd.workloads import DecodeConfig, build_request_cache, make_request

    dev = _cuda()
    cfg = DecodeConfig("b33", 16, 2, (64 + 8,), (0.0, 1.0, 0.0), recent=8)
    caches = [build_request_cache(cfg, make_request(cfg, 72, seed=1400 + r, device=dev)) for r in range(33)]
    exs = [ro.prepare_splitk_executor(c, ro.allocate_splitk_workspace(c, num_query_heads=16)) for c in caches]
    with pytest.raises(ValueError, match="at most 32 requests"):
        ro.stack_homogeneous_splitk_executors(exs)


def test_inline_slot_ranges_equal_device_ranges():
    """r2o_decode_combine with the host copy of group_begin (the slot ranges travel in the launch
    arguments) and without it (the ranges are read from the device array): the same output bits,
    for a ragged batch of 4 (16 groups)."""
    import ctypes

    import r2omni_amd as ro
    from r2omni_amd import _lib
    from r2omni_amd.workloads import DecodeConfig, build_request_cache, make_request

    dev = _cuda()
    cfg = DecodeConfig("inline", 28, 4, (740, 1252, 2276, 3300), (0.15, 0.45, 0.4), recent=100)
    datas = [make_request(cfg, n, seed=1400 + r, device=dev) for r, n in enumerate(cfg.lengths)]
    caches = [build_request_cache(cfg, d) for d in datas]
    exs = [ro.prepare_splitk_executor(c, ro.allocate_splitk_workspace(c, num_query_heads=28), output_hadamard=True)
           for c in caches]
    ex = ro.stack_homogeneous_splitk_executors(exs)
    q = torch.cat([d.query for d in datas]).contiguous()
    lib, stream = _lib.load(), ctypes.c_void_p(_lib.stream_of(dev))
    outs = []
    for host_ranges in (True, False):
        out = torch.empty_like(ex.workspace.output)
        p = ex._params(q, out, None)
        assert bool(p.group_begin_host) == (ex.host_group_begin is not None)
        if not host_ranges:
            p.group_begin_host = None
        _lib.check(lib.r2o_decode_partial(ctypes.byref(p), stream), "r2o_decode_partial")
        _lib.check(lib.r2o_decode_combine(ctypes.byref(p), stream), "r2o_decode_combine")
        outs.append(out)
    torch.cuda.synchronize()
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))


@pytest.mark.parametrize("rotary", [False, True])
def test_token_axis_forms_of_the_rows_give_the_same_call(rotary):
    """The manager's rows arrive as [B, H, 1, 128] or [B, H, 128]; contiguous ones are checked as they
    are and strided ones (with the folded rotation) are sliced: both forms give the same output and the
    same ring rows, bit for bit, over three appends on a stacked executor."""
    import r2omni_amd as ro
    from r2omni_amd.workloads import DecodeConfig, build_request_cache, make_request

    dev = _cuda()
    hq, hkv = 28, 4
    cfg = DecodeConfig("axis", hq, hkv, (0,), (0.15, 0.45, 0.4), recent=100)
    datas = [make_request(cfg, t, seed=960 + i, device=dev) for i, t in enumerate((1024 + 100, 1536 + 100))]

    def executor():
        exs = []
        for d in datas:
            c = build_request_cache(cfg, d)
            exs.append(ro.prepare_splitk_executor(c, ro.allocate_splitk_workspace(c, num_query_heads=hq),
                                                  output_hadamard=True))
        return ro.stack_homogeneous_splitk_executors(exs)

    ex3, ex4 = executor(), executor()
    gen = torch.Generator(device=dev).manual_seed(961)
    pos = [1124, 1636]
    for step in range(3):
        q = torch.randn(2, hq, 128, generator=gen, device=dev).to(torch.bfloat16)
        k = torch.randn(2, hkv, 128, generator=gen, device=dev).to(torch.bfloat16)
        v = torch.randn(2, hkv, 128, generator=gen, device=dev).to(torch.bfloat16)
        rot = None
        if rotary:
            ang = torch.rand(3, 2, 1, 64, generator=gen, device=dev) * 6.0
            ang = torch.cat([ang, ang], dim=-1)
            rot = ro.FusedRotary(ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16), (16, 24, 24), True, True)
        print(f"[edge] token-axis forms, rotary={rotary}, step {step}", flush=True)
        a = ex3(q, append=(k, v, pos, pos), rotary=rot).clone()
        b = ex4(q[:, :, None], append=(k[:, :, None], v[:, :, None], pos, pos), rotary=rot).clone()
        torch.cuda.synchronize()
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"step {step}"
        pos = [p + 1 for p in pos]
    for ra, rb in zip(ex3.batched_recent, ex4.batched_recent):
        assert torch.equal(ra.fp_k.view(torch.int16), rb.fp_k.view(torch.int16))
        assert torch.equal(ra.fp_v.view(torch.int16), rb.fp_v.view(torch.int16))
        assert int(ra.length_device.item()) == int(rb.length_device.item()) == 103
