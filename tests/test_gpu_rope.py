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
        if had:  # FWHT summation order differs: at most one output ulp
            np.testing.assert_allclose(_np32(got), want, rtol=2 ** -7, atol=1e-6)
        else:    # same fp32 operations in the same order: bit-exact
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
