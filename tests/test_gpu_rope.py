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
