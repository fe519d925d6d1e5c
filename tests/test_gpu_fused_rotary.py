"""The decode step's rotation folded into the split-K call (FusedRotary): the partial kernel rotates the
raw query and appended key (Qwen mRoPE, optionally the FWHT) and the appended value (FWHT) itself.  The
reference path is the separate launch (qwen_qk_mrope, triton_fwht_128; qwen_sspa_attention.py:1239-1247,
230-235) followed by the call on the rotated rows; the same arithmetic in the same order, so outputs and
ring rows must be bit-identical, step after step, through a flush."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _cuda():
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    return torch.device("cuda:0")


def _caches(cfg, totals, seed, dev):
    from r2omni_amd.workloads import build_request_cache, make_request

    datas = [make_request(cfg, t, seed=seed + i, device=dev) for i, t in enumerate(totals)]
    return [build_request_cache(cfg, d) for d in datas], datas


def _executor(caches, hq, dev):
    import r2omni_amd as ro

    exs = [ro.prepare_splitk_executor(c, ro.allocate_splitk_workspace(c, num_query_heads=hq), output_hadamard=True)
           for c in caches]
    return exs[0] if len(exs) == 1 else ro.stack_homogeneous_splitk_executors(exs)


def _tables(gen, b, dev, dtype, contiguous=True):
    """mRoPE tables [3, B, 1, 128] with a different angle per axis, so the sections matter."""
    ang = torch.rand(3, b, 1, 64, generator=gen, device=dev) * 6.0
    ang = torch.cat([ang, ang], dim=-1)
    cos, sin = ang.cos().to(dtype), ang.sin().to(dtype)
    if not contiguous:  # the same values with a padded last-but-one layout
        cos = torch.cat([cos, cos], dim=2)[:, :, :1]
        sin = torch.cat([sin, sin], dim=2)[:, :, :1]
    return cos, sin


def _bits(t):
    return t.contiguous().view(torch.int16)


CASES = [
    # totals (64-token pages + a 100-token ring), rows dtype, hadamard, value hadamard, table dtype,
    # sections, inputs as views of one padded projection row
    ((2048 + 100,), torch.bfloat16, True, True, torch.bfloat16, (16, 24, 24), False),
    ((1536 + 100, 1024 + 100), torch.bfloat16, True, False, torch.float32, (16, 24, 24), True),
    ((1024 + 100,), torch.bfloat16, False, True, torch.bfloat16, (8, 8, 48), True),
    ((1024 + 100, 2048 + 100), torch.float16, True, True, torch.float16, (20, 20, 24), False),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_fused_rotary_call_equals_separate_rotation(case):
    import r2omni_amd as ro
    from r2omni_amd.workloads import DecodeConfig

    dev = _cuda()
    totals, rows, had, vhad, tdt, sections, strided = CASES[case]
    cfg = DecodeConfig("rot", 28, 4, (0,), (0.15, 0.45, 0.4), recent=100,
                       dtype="float16" if rows == torch.float16 else "bfloat16")
    b = len(totals)
    ca, _ = _caches(cfg, totals, 600 + case, dev)
    cb, _ = _caches(cfg, totals, 600 + case, dev)
    ex_a, ex_b = _executor(ca, 28, dev), _executor(cb, 28, dev)
    gen = torch.Generator(device=dev).manual_seed(610 + case)
    pos = [int(c.compact_key.active_length) + c.recent_fp_pool.active_length for c in ca]
    print(f"[rotary] case {case}: batch {b}, rows {rows}, hadamard {had}/{vhad}, tables {tdt}, "
          f"sections {sections}, strided {strided}", flush=True)
    for step in range(3):
        qkv = torch.randn(b, (28 + 8) * 128 + (64 if strided else 0), generator=gen, device=dev).to(rows)
        q = qkv[:, : 28 * 128].view(b, 28, 128)
        k = qkv[:, 28 * 128 : 32 * 128].view(b, 4, 128)
        v = qkv[:, 32 * 128 : 36 * 128].view(b, 4, 128)
        if not strided:
            q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        cos, sin = _tables(gen, b, dev, tdt, contiguous=not strided)
        qr, kr = ro.qwen_qk_mrope(q[:, :, None], k[:, :, None], cos, sin, sections, apply_hadamard=had)
        vr = ro.triton_fwht_128(v.contiguous()) if vhad else v.contiguous()
        want = ex_a(qr[:, :, 0].contiguous(), append=(kr, vr[:, :, None], pos, pos)).clone()
        got = ex_b(q, append=(k, v, pos, pos), rotary=ro.FusedRotary(cos, sin, sections, had, vhad)).clone()
        if b == 1:
            ca[0].recent_fp_pool.active_length += 1
            cb[0].recent_fp_pool.active_length += 1
        pos = [p + 1 for p in pos]
        torch.cuda.synchronize()
        assert torch.equal(_bits(got), _bits(want)), f"case {case} step {step}: output"
    rings_a = ex_a.batched_recent or [c.recent_fp_pool for c in ca]
    rings_b = ex_b.batched_recent or [c.recent_fp_pool for c in cb]
    for ra, rb in zip(rings_a, rings_b):
        assert torch.equal(_bits(rb.fp_k), _bits(ra.fp_k)) and torch.equal(_bits(rb.fp_v), _bits(ra.fp_v))
        assert torch.equal(rb.global_index_buffer, ra.global_index_buffer)
        assert int(rb.length_device.item()) == int(ra.length_device.item())


def test_strided_rows_need_the_folded_rotation():
    """Without a rotation the call takes contiguous rows, as the reference's does
    (triton_fourq_splitk.py:1255-1261, 1300-1310); views of a projection row are for rotated calls."""
    from r2omni_amd.workloads import DecodeConfig

    dev = _cuda()
    cfg = DecodeConfig("rot", 16, 2, (0,), (0.2, 0.5, 0.3), recent=64)
    ca, _ = _caches(cfg, (1024 + 64, 1024 + 64), 640, dev)
    ex = _executor(ca, 16, dev)
    wide = torch.zeros(2, 20 * 128 + 64, device=dev, dtype=torch.bfloat16)  # padded projection rows
    q = wide[:, : 16 * 128].view(2, 16, 128)
    k = wide[:, 16 * 128 : 18 * 128].view(2, 2, 128)
    with pytest.raises(ValueError, match="query does not match"):
        ex(q)
    with pytest.raises(ValueError, match="append K/V must be contiguous"):
        ex(q.contiguous(), append=(k, k.clone(), [0, 0], [0, 0]))


def test_fused_rotary_without_append_rotates_the_query_only():
    import r2omni_amd as ro
    from r2omni_amd.workloads import DecodeConfig

    dev = _cuda()
    cfg = DecodeConfig("rot", 16, 2, (0,), (0.2, 0.5, 0.3), recent=64)
    ca, _ = _caches(cfg, (1024 + 64,), 620, dev)
    ex = _executor(ca, 16, dev)
    gen = torch.Generator(device=dev).manual_seed(621)
    q = torch.randn(1, 16, 128, generator=gen, device=dev).to(torch.bfloat16)
    k = torch.randn(1, 2, 128, generator=gen, device=dev).to(torch.bfloat16)
    cos, sin = _tables(gen, 1, dev, torch.bfloat16)
    qr, _ = ro.qwen_qk_mrope(q[:, :, None], k[:, :, None], cos, sin, (16, 24, 24), apply_hadamard=True)
    want = ex(qr[:, :, 0].contiguous()).clone()
    got = ex(q, rotary=ro.FusedRotary(cos, sin, (16, 24, 24), True, True)).clone()
    torch.cuda.synchronize()
    assert torch.equal(_bits(got), _bits(want))


@pytest.mark.parametrize("use_graph", [False, True])
def test_batched_decoder_with_fused_rotary_through_a_flush(use_graph):
    """140 steps of a 2-request decoder (a flush inside the batch at the ring's 128th token), its inputs
    bound to views of one fused-projection buffer and its tables rewritten in place every step, against
    a decoder fed by the separate rotation: outputs bit-identical at every step, rings equal after."""
    import r2omni_amd as ro
    from r2omni_amd.workloads import DecodeConfig

    dev = _cuda()
    cfg = DecodeConfig("rot", 28, 4, (0,), (0.15, 0.45, 0.4), recent=120)
    totals = (1024 + 120, 2048 + 120)
    ca, _ = _caches(cfg, totals, 630, dev)
    cb, _ = _caches(cfg, totals, 630, dev)
    b, sections = 2, (16, 24, 24)
    cos_buf = torch.empty(3, b, 1, 128, device=dev, dtype=torch.bfloat16)
    sin_buf = torch.empty_like(cos_buf)
    dec_a = ro.BatchedDecoder(ca, num_query_heads=28, output_hadamard=True, use_graph=use_graph)
    dec_b = ro.BatchedDecoder(cb, num_query_heads=28, output_hadamard=True, use_graph=use_graph,
                              rotary=ro.FusedRotary(cos_buf, sin_buf, sections, True, True))
    qkv = torch.empty(b, 36 * 128 + 128, device=dev, dtype=torch.bfloat16)  # a padded projection row
    dec_b.bind_inputs(qkv[:, : 28 * 128].view(b, 28, 128), qkv[:, 28 * 128 : 32 * 128].view(b, 4, 128),
                      qkv[:, 32 * 128 : 36 * 128].view(b, 4, 128))
    gen = torch.Generator(device=dev).manual_seed(631)
    pos = [int(c.compact_key.active_length) + c.recent_fp_pool.active_length for c in ca]
    for step in range(140):
        qkv.copy_(torch.randn(qkv.shape, generator=gen, device=dev))
        cos, sin = _tables(gen, b, dev, torch.bfloat16)
        cos_buf.copy_(cos)
        sin_buf.copy_(sin)
        q = qkv[:, : 28 * 128].view(b, 28, 1, 128)
        k = qkv[:, 28 * 128 : 32 * 128].view(b, 4, 1, 128)
        v = qkv[:, 32 * 128 : 36 * 128].view(b, 4, 1, 128)
        ro.qwen_qk_mrope(q, k, cos_buf, sin_buf, sections, apply_hadamard=True, value=v,
                         output=(dec_a.query_buffer.view(b, 28, 1, 128), dec_a.key_buffer.view(b, 4, 1, 128),
                                 dec_a.value_buffer.view(b, 4, 1, 128)))
        want = dec_a.step_in_place(global_token_index=pos, logical_position=pos)
        got = dec_b.step_in_place(global_token_index=pos, logical_position=pos)
        torch.cuda.synchronize()
        if step % 20 == 0 or step == 139:
            print(f"[rotary] decoder graph={use_graph} step {step}", flush=True)
        assert torch.equal(_bits(got), _bits(want)), f"step {step}"
        pos = [p + 1 for p in pos]
    assert dec_b.replans == dec_a.replans + 1 >= 3  # the flushes re-planned both (and bind_inputs dec_b)
    for x, y in zip(ca, cb):
        ra, rb = x.recent_fp_pool, y.recent_fp_pool
        assert ra.active_length == rb.active_length
        assert torch.equal(_bits(rb.fp_k), _bits(ra.fp_k)) and torch.equal(_bits(rb.fp_v), _bits(ra.fp_v))
        assert torch.equal(y.compact_key.packed, x.compact_key.packed)


QWEN3_CASES = [
    # totals, rows dtype, hadamard (Q/K), value hadamard, tables per request (else one shared row),
    # inputs as views of one padded projection row
    ((2048 + 100,), torch.bfloat16, True, True, False, False),
    ((1536 + 100, 1024 + 100), torch.bfloat16, True, False, True, True),
    ((1024 + 100, 2048 + 100), torch.float16, False, True, True, False),
    ((1024 + 100, 1536 + 100), torch.float16, True, True, False, True),
]


@pytest.mark.parametrize("case", range(len(QWEN3_CASES)))
def test_fused_qwen3_call_equals_separate_norm_rope(case):
    """The Qwen3 branch folded into the call (FusedQwen3Rotary) against qwen3_qk_norm_rope and the V
    FWHT as separate launches before the call (qwen_sspa_attention.py:1228-1235, 230-235): outputs
    and ring rows bit-identical over 3 steps."""
    import r2omni_amd as ro
    from r2omni_amd.workloads import DecodeConfig

    dev = _cuda()
    totals, rows, had, vhad, per_request, strided = QWEN3_CASES[case]
    cfg = DecodeConfig("q3", 28, 4, (0,), (0.15, 0.45, 0.4), recent=100,
                       dtype="float16" if rows == torch.float16 else "bfloat16")
    b = len(totals)
    ca, _ = _caches(cfg, totals, 650 + case, dev)
    cb, _ = _caches(cfg, totals, 650 + case, dev)
    ex_a, ex_b = _executor(ca, 28, dev), _executor(cb, 28, dev)
    gen = torch.Generator(device=dev).manual_seed(660 + case)
    wq = (1.0 + 0.3 * torch.randn(128, generator=gen, device=dev)).to(rows)
    wk = (1.0 + 0.3 * torch.randn(128, generator=gen, device=dev)).to(rows)
    pos = [int(c.compact_key.active_length) + c.recent_fp_pool.active_length for c in ca]
    print(f"[qwen3] case {case}: batch {b}, rows {rows}, hadamard {had}/{vhad}, per-request tables "
          f"{per_request}, strided {strided}", flush=True)
    for step in range(3):
        qkv = torch.randn(b, 36 * 128 + (64 if strided else 0), generator=gen, device=dev).to(rows)
        q = qkv[:, : 28 * 128].view(b, 28, 128)
        k = qkv[:, 28 * 128 : 32 * 128].view(b, 4, 128)
        v = qkv[:, 32 * 128 : 36 * 128].view(b, 4, 128)
        if not strided:
            q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        ang = torch.rand(b if per_request else 1, 1, 64, generator=gen, device=dev) * 6.0
        ang = torch.cat([ang, ang], dim=-1)
        cos, sin = ang.cos().to(rows), ang.sin().to(rows)
        qr, kr = ro.qwen3_qk_norm_rope(q[:, :, None], k[:, :, None], wq, wk, cos, sin, eps=1e-6,
                                       apply_hadamard=had)
        vr = ro.triton_fwht_128(v.contiguous()) if vhad else v.contiguous()
        want = ex_a(qr[:, :, 0].contiguous(), append=(kr, vr[:, :, None], pos, pos)).clone()
        got = ex_b(q, append=(k, v, pos, pos),
                   rotary=ro.FusedQwen3Rotary(cos, sin, wq, wk, 1e-6, had, vhad)).clone()
        if b == 1:
            ca[0].recent_fp_pool.active_length += 1
            cb[0].recent_fp_pool.active_length += 1
        pos = [p + 1 for p in pos]
        torch.cuda.synchronize()
        assert torch.equal(_bits(got), _bits(want)), f"case {case} step {step}: output"
    rings_a = ex_a.batched_recent or [c.recent_fp_pool for c in ca]
    rings_b = ex_b.batched_recent or [c.recent_fp_pool for c in cb]
    for ra, rb in zip(rings_a, rings_b):
        assert torch.equal(_bits(rb.fp_k), _bits(ra.fp_k)) and torch.equal(_bits(rb.fp_v), _bits(ra.fp_v))
