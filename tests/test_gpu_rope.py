"""GPU parity of the decode-step mRoPE (+ FWHT) kernel against the CPU oracle."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

CASES = [
    # batch, hq, hkv, tokens, q dtype, table dtype, hadamard, shared-batch (stride 0) tables
    (1, 28, 4, 1, torch.bfloat16, torch.bfloat16, False, False),
    (4, 28, 4, 1, torch.bfloat16, torch.float32, True, False),
    (2, 16, 2, 3, torch.float16, torch.float32, False, True),
    (3, 32, 8, 2, torch.bfloat16, torch.bfloat16, True, True),
]


def _np32(t):
    return t.detach().float().cpu().numpy()


@pytest.mark.parametrize("case", range(len(CASES)))
def test_qk_mrope_matches_oracle(case):
    import r2omni_amd as ro
    from oracle.rope import qwen_mrope

    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    dev = torch.device("cuda:0")
    b, hq, hkv, t, qdt, tdt, had, shared = CASES[case]
    gen = torch.Generator().manual_seed(10 + case)
    q = torch.randn(b, hq, t, 128, generator=gen).to(qdt).to(dev)
    k = torch.randn(b, hkv, t, 128, generator=gen).to(qdt).to(dev)
    inv = 1.0 / (1e6 ** (torch.arange(0, 128, 2, dtype=torch.float64) / 128))
    pos = torch.randint(0, 8000, (3, 1 if shared else b, t), generator=gen).double()
    ang = pos[..., None] * inv
    ang = torch.cat([ang, ang], dim=-1)
    cos, sin = ang.cos().to(tdt).to(dev), ang.sin().to(tdt).to(dev)
    if shared:
        cos, sin = cos.expand(3, b, t, 128), sin.expand(3, b, t, 128)
    sections = (16, 24, 24)
    qo, ko = ro.qwen_qk_mrope(q, k, cos, sin, sections, apply_hadamard=had)
    torch.cuda.synchronize()
    name = "bfloat16" if qdt == torch.bfloat16 else "float16"
    cs, sn = _np32(cos), _np32(sin)
    for got, x in ((qo, q), (ko, k)):
        want = qwen_mrope(_np32(x), cs, sn, sections, hadamard=had, dtype=name)
        # the same fp32 operations in the same order (the FWHT in the reference's stage order): bit-exact
        np.testing.assert_array_equal(_np32(got), want)


def test_qk_mrope_rejects_bad_sections_and_shapes():
    import r2omni_amd as ro

    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    dev = torch.device("cuda:0")
    q = torch.zeros(1, 4, 1, 128, dtype=torch.bfloat16, device=dev)
    k = torch.zeros(1, 2, 1, 128, dtype=torch.bfloat16, device=dev)
    cs = torch.zeros(3, 1, 1, 128, dtype=torch.float32, device=dev)
    with pytest.raises(ValueError, match="sum"):
        ro.qwen_qk_mrope(q, k, cs, cs, (16, 24, 23))
    with pytest.raises(ValueError, match="rank-4"):
        ro.qwen_qk_mrope(q[0], k, cs, cs, (16, 24, 24))


NORM_CASES = [
    # batch, hq, hkv, tokens, dtype, hadamard, tables shared across the batch
    (1, 32, 8, 1, torch.bfloat16, False, False),
    (4, 32, 8, 1, torch.bfloat16, True, False),
    (2, 16, 2, 3, torch.float16, False, True),
    (3, 28, 4, 2, torch.float16, True, False),
]


@pytest.mark.parametrize("case", range(len(NORM_CASES)))
def test_qwen3_qk_norm_rope_matches_oracle(case):
    import r2omni_amd as ro
    from oracle.rope import qwen3_norm_rope
    from test_oracle_rope import _rope_tables_1d, _ulp_steps

    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    dev = torch.device("cuda:0")
    b, hq, hkv, t, dt, had, shared = NORM_CASES[case]
    print(f"[qwen3 norm+rope] case {case}", flush=True)
    gen = torch.Generator().manual_seed(30 + case)
    q = (torch.randn(b, hq, t, 128, generator=gen) * 3).to(dt)
    k = (torch.randn(b, hkv, t, 128, generator=gen) * 3).to(dt)
    wq, wk = (torch.rand(128, generator=gen) * 2).to(dt), (torch.rand(128, generator=gen) * 2).to(dt)
    cos, sin = _rope_tables_1d(1 if shared else b, t, gen, dt)
    qo, ko = ro.qwen3_qk_norm_rope(q.to(dev), k.to(dev), wq.to(dev), wk.to(dev), cos.to(dev), sin.to(dev),
                                   eps=1e-6, apply_hadamard=had)
    torch.cuda.synchronize()
    name = "bfloat16" if dt == torch.bfloat16 else "float16"
    cs, sn = np.broadcast_to(_np32(cos), (b, t, 128)), np.broadcast_to(_np32(sin), (b, t, 128))
    for got, x, w in ((qo, q, wq), (ko, k, wk)):
        want = qwen3_norm_rope(_np32(x), _np32(w), cs, sn, eps=1e-6, hadamard=had, dtype=name)
        steps = _ulp_steps(_np32(got), want, name)
        # the squares are summed in another order than numpy's (and the FWHT's sums too): a rounding
        # may move by a step, rarely
        assert steps.max() <= (3 if had else 2) and (steps == 0).mean() >= 0.99, (steps.max(), (steps == 0).mean())


def test_qwen3_qk_norm_rope_rejects_mismatched_arguments():
    import r2omni_amd as ro

    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    dev = torch.device("cuda:0")
    q = torch.zeros(1, 4, 1, 128, dtype=torch.bfloat16, device=dev)
    k = torch.zeros(1, 2, 1, 128, dtype=torch.bfloat16, device=dev)
    w = torch.ones(128, dtype=torch.bfloat16, device=dev)
    cs = torch.zeros(1, 1, 128, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="cos/sin"):
        ro.qwen3_qk_norm_rope(q, k, w, w, cs.float(), cs.float())
    with pytest.raises(ValueError, match="q_norm_weight"):
        ro.qwen3_qk_norm_rope(q, k, w.float(), w, cs, cs)
    with pytest.raises(ValueError, match="rank-4"):
        ro.qwen3_qk_norm_rope(q[0], k, w, w, cs, cs)


def _exact_where_normal(got, want32, dtype):
    """Bit equality of got with want32 rounded to dtype, outside fp16's subnormal range."""
    want = torch.from_numpy(np.ascontiguousarray(want32)).to(dtype)
    normal = torch.from_numpy(np.abs(want32) >= (2.0 ** -14 if dtype == torch.float16 else 0.0))
    return torch.equal(got.cpu().view(torch.int16)[normal], want.view(torch.int16)[normal])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fwht128_is_the_reference_stage_order_bit_exact(dtype):
    """triton_fwht_128 (r2o_fwht128) runs the reference's stages (stride 1 .. 64, left + right and
    left - right, then the float32 scale): bit-exact to the oracle's float32 restatement of
    that order, rounded once to the dtype."""
    import r2omni_amd as ro
    from oracle.quant import normalized_fwht

    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    gen = torch.Generator().manual_seed(21)
    x = (torch.randn(1024, 128, generator=gen) * 4).to(dtype)
    got = ro.triton_fwht_128(x.to("cuda:0"))
    torch.cuda.synchronize()
    assert _exact_where_normal(got, normalized_fwht(_np32(x)), dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_lane_butterflies_are_bit_exact(dtype):
    """The in-register FWHT of the mRoPE and combine kernels (DPP within rows, permlane swaps
    across rows, stride 64 inside the lane last): with identity tables (cos 1, sin 0) the mRoPE
    output is that FWHT of the input, bit-exact to the reference's stage order (stride 1 .. 64,
    triton_qwen_mrope.py:23-32) evaluated in float32 on the CPU."""
    import r2omni_amd as ro
    from oracle.quant import normalized_fwht

    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    dev = torch.device("cuda:0")
    gen = torch.Generator().manual_seed(22)
    q = (torch.randn(2, 28, 3, 128, generator=gen) * 4).to(dtype)
    k = (torch.randn(2, 4, 3, 128, generator=gen) * 4).to(dtype)
    cos = torch.ones(3, 2, 3, 128, dtype=torch.float32, device=dev)
    sin = torch.zeros(3, 2, 3, 128, dtype=torch.float32, device=dev)
    qo, ko = ro.qwen_qk_mrope(q.to(dev), k.to(dev), cos, sin, (16, 24, 24), apply_hadamard=True)
    torch.cuda.synchronize()
    for got, x in ((qo, q), (ko, k)):
        rows = _np32(x).reshape(-1, 128)
        assert _exact_where_normal(got.reshape(-1, 128), normalized_fwht(rows), dtype)


@pytest.mark.parametrize("case", range(len(CASES)))
def test_qkv_mrope_folds_the_v_hadamard(case):
    """qwen_qk_mrope(value=V): Q and K bit-identical to the two-tensor call; with the Hadamard on, V
    is its FWHT (bit-exact to the reference's stage order), written into a caller's buffer when
    given; with it off, V is returned as is."""
    import r2omni_amd as ro
    from oracle.quant import normalized_fwht

    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    dev = torch.device("cuda:0")
    b, hq, hkv, t, qdt, tdt, had, shared = CASES[case]
    gen = torch.Generator().manual_seed(30 + case)
    q = torch.randn(b, hq, t, 128, generator=gen).to(qdt).to(dev)
    k = torch.randn(b, hkv, t, 128, generator=gen).to(qdt).to(dev)
    v = (torch.randn(b, hkv, t, 128, generator=gen) * 3).to(qdt).to(dev)
    pos = torch.randint(0, 8000, (3, b, t), generator=gen).double()
    ang = pos[..., None] * (1.0 / (1e6 ** (torch.arange(0, 128, 2, dtype=torch.float64) / 128)))
    ang = torch.cat([ang, ang], dim=-1)
    cos, sin = ang.cos().to(tdt).to(dev), ang.sin().to(tdt).to(dev)
    sections = (16, 24, 24)
    q2, k2 = ro.qwen_qk_mrope(q, k, cos, sin, sections, apply_hadamard=had)
    vbuf = torch.full_like(v, 7.0)
    q3, k3, v3 = ro.qwen_qk_mrope(q, k, cos, sin, sections, apply_hadamard=had, value=v,
                                  output=(torch.empty_like(q), torch.empty_like(k), vbuf))
    torch.cuda.synchronize()
    assert torch.equal(q3.view(torch.int16), q2.view(torch.int16))
    assert torch.equal(k3.view(torch.int16), k2.view(torch.int16))
    assert v3.data_ptr() == vbuf.data_ptr()
    rows = _np32(v).reshape(-1, 128)
    if had:
        assert _exact_where_normal(v3.reshape(-1, 128), normalized_fwht(rows), qdt)
    else:
        assert torch.equal(v3, v)
        _, _, same = ro.qwen_qk_mrope(q, k, cos, sin, sections, value=v)
        assert same is v
    with pytest.raises(ValueError, match="value"):
        ro.qwen_qk_mrope(q, k, cos, sin, sections, apply_hadamard=had, value=v[:, :, :, :64])


@pytest.mark.parametrize("case", range(len(NORM_CASES)))
def test_qwen3_qkv_norm_rope_folds_the_v_hadamard(case):
    """qwen3_qk_norm_rope(value=V): Q and K bit-identical to the two-tensor call; with the Hadamard
    on, V is its FWHT (bit-exact to the reference's stage order) written into the caller's buffer;
    with it off, V is copied unchanged into that buffer."""
    import r2omni_amd as ro
    from oracle.quant import normalized_fwht
    from test_oracle_rope import _rope_tables_1d

    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    dev = torch.device("cuda:0")
    b, hq, hkv, t, dt, had, shared = NORM_CASES[case]
    gen = torch.Generator().manual_seed(40 + case)
    q = (torch.randn(b, hq, t, 128, generator=gen) * 3).to(dt).to(dev)
    k = (torch.randn(b, hkv, t, 128, generator=gen) * 3).to(dt).to(dev)
    v = (torch.randn(b, hkv, t, 128, generator=gen) * 3).to(dt).to(dev)
    wq, wk = (torch.rand(128, generator=gen) * 2).to(dt).to(dev), (torch.rand(128, generator=gen) * 2).to(dt).to(dev)
    cos, sin = _rope_tables_1d(1 if shared else b, t, gen, dt)
    cos, sin = cos.to(dev), sin.to(dev)
    q2, k2 = ro.qwen3_qk_norm_rope(q, k, wq, wk, cos, sin, eps=1e-6, apply_hadamard=had)
    vbuf = torch.full_like(v, 5.0)
    q3, k3, v3 = ro.qwen3_qk_norm_rope(q, k, wq, wk, cos, sin, eps=1e-6, apply_hadamard=had, value=v,
                                       output=(torch.empty_like(q), torch.empty_like(k), vbuf))
    torch.cuda.synchronize()
    assert torch.equal(q3.view(torch.int16), q2.view(torch.int16))
    assert torch.equal(k3.view(torch.int16), k2.view(torch.int16))
    assert v3.data_ptr() == vbuf.data_ptr()
    if had:
        assert _exact_where_normal(v3.reshape(-1, 128), normalized_fwht(_np32(v).reshape(-1, 128)), dt)
    else:
        assert torch.equal(v3, v)
    with pytest.raises(ValueError, match="one tensor per input"):
        ro.qwen3_qk_norm_rope(q, k, wq, wk, cos, sin, value=v, output=(q2, k2))


@pytest.mark.parametrize("norm", [False, True])
def test_rejected_call_leaves_the_value_buffer_untouched(norm):
    """Every output is checked before the launch or the V copy: a bad Q output raises and the
    caller's V buffer keeps its contents (apply_hadamard=False copies V into it only on success)."""
    import r2omni_amd as ro

    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    dev = torch.device("cuda:0")
    q = torch.randn(1, 4, 1, 128, device=dev).to(torch.bfloat16)
    k = torch.randn(1, 2, 1, 128, device=dev).to(torch.bfloat16)
    v = torch.randn(1, 2, 1, 128, device=dev).to(torch.bfloat16)
    vbuf = torch.full_like(v, 3.0)
    bad = (torch.empty(1, 4, 1, 64, device=dev, dtype=torch.bfloat16), torch.empty_like(k), vbuf)
    with pytest.raises(ValueError):
        if norm:
            w = torch.ones(128, device=dev, dtype=torch.bfloat16)
            cs = torch.zeros(1, 1, 128, device=dev, dtype=torch.bfloat16)
            ro.qwen3_qk_norm_rope(q, k, w, w, cs, cs, value=v, output=bad)
        else:
            cs = torch.zeros(3, 1, 1, 128, device=dev, dtype=torch.float32)
            ro.qwen_qk_mrope(q, k, cs, cs, (16, 24, 24), value=v, output=bad)
    torch.cuda.synchronize()
    assert torch.equal(vbuf, torch.full_like(v, 3.0))
