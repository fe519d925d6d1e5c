"""Pin the mRoPE oracle with closed forms (no reference fixture exists for the Triton kernel)."""
import numpy as np
import pytest
import torch

from oracle.quant import normalized_fwht
from oracle.rope import qwen_mrope

SECTIONS = (16, 24, 24)  # Qwen2.5-Omni mrope_section


def _tables(b, t, rng, duplicated=True):
    """Standard RoPE tables for 3 position axes: cos/sin [3, B, T, 128], halves duplicated."""
    inv = 1.0 / (1e6 ** (np.arange(0, 128, 2) / 128))
    pos = rng.integers(0, 5000, size=(3, b, t)).astype(np.float64)
    ang = pos[..., None] * inv  # [3, B, T, 64]
    if duplicated:
        ang = np.concatenate([ang, ang], axis=-1)
    else:
        ang = np.concatenate([ang, ang + rng.standard_normal(ang.shape)], axis=-1)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def test_identity_tables_return_the_input():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((2, 3, 4, 128)).astype(np.float32)
    ones, zeros = np.ones((3, 2, 4, 128), np.float32), np.zeros((3, 2, 4, 128), np.float32)
    np.testing.assert_array_equal(qwen_mrope(x, ones, zeros, SECTIONS, hadamard=False, dtype="float32"), x)
    np.testing.assert_allclose(qwen_mrope(x, ones, zeros, SECTIONS, hadamard=True, dtype="float32"),
                               normalized_fwht(x), atol=1e-6)


def test_pairs_rotate_as_complex_products():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((1, 2, 3, 128)).astype(np.float32)
    cos, sin = _tables(1, 3, rng)
    out = qwen_mrope(x, cos, sin, SECTIONS, hadamard=False, dtype="float32").astype(np.float64)
    d = np.arange(64)
    axis = np.where(d < 16, 0, np.where(d < 40, 1, 2))
    c = np.stack([cos[axis, 0, t, d] for t in range(3)]).astype(np.float64)  # [T, 64]
    s = np.stack([sin[axis, 0, t, d] for t in range(3)]).astype(np.float64)
    z = (x[..., :64].astype(np.float64) + 1j * x[..., 64:].astype(np.float64)) * (c + 1j * s)
    np.testing.assert_allclose(out[..., :64], z.real, atol=1e-5)
    np.testing.assert_allclose(out[..., 64:], z.imag, atol=1e-5)
    # the rotation preserves every pair's norm
    np.testing.assert_allclose(out[..., :64] ** 2 + out[..., 64:] ** 2,
                               x[..., :64].astype(np.float64) ** 2 + x[..., 64:].astype(np.float64) ** 2, rtol=1e-5)


def test_sections_pick_axes_like_the_split_concatenate_formulation():
    # transformers' apply_multimodal_rotary_pos_emb: split the tables along the last dim by the
    # sections repeated twice and take chunk i from axis i % 3 (restated here independently).
    rng = np.random.default_rng(2)
    x = rng.standard_normal((2, 1, 2, 128)).astype(np.float32)
    cos, sin = _tables(2, 2, rng, duplicated=False)
    tc, ts = torch.from_numpy(cos), torch.from_numpy(sin)
    split = list(SECTIONS) * 2
    c = torch.cat([m[i % 3] for i, m in enumerate(tc.split(split, dim=-1))], dim=-1)[:, None]
    s = torch.cat([m[i % 3] for i, m in enumerate(ts.split(split, dim=-1))], dim=-1)[:, None]
    tx = torch.from_numpy(x)
    rot = torch.cat((-tx[..., 64:], tx[..., :64]), dim=-1)
    want = (tx * c + rot * s).numpy()
    got = qwen_mrope(x, cos, sin, SECTIONS, hadamard=False, dtype="float32")
    np.testing.assert_allclose(got, want, atol=1e-6)


# ----------------------------------------------------------- Qwen3 RMSNorm + RoPE branch
def _ulp_steps(a: np.ndarray, b: np.ndarray, dtype: str) -> np.ndarray:
    """Distance in representable steps of ``dtype`` between two arrays of ``dtype`` values."""
    if dtype == "bfloat16":
        from oracle.quant import f32_to_bf16_bits

        ia, ib = f32_to_bf16_bits(a).astype(np.int64), f32_to_bf16_bits(b).astype(np.int64)
    else:
        ia = a.astype(np.float16).view(np.uint16).astype(np.int64)
        ib = b.astype(np.float16).view(np.uint16).astype(np.int64)
    mono = lambda i: np.where(i & 0x8000, -(i & 0x7FFF), i)  # noqa: E731  sign-magnitude -> ordered
    return np.abs(mono(ia) - mono(ib))


def _rope_tables_1d(b, t, gen, dt):
    inv = 1.0 / (1e6 ** (torch.arange(0, 128, 2, dtype=torch.float64) / 128))
    pos = torch.randint(0, 40000, (b, t), generator=gen).double()
    ang = pos[..., None] * inv
    ang = torch.cat([ang, ang], dim=-1)
    return ang.cos().to(dt), ang.sin().to(dt)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("hadamard", [False, True])
def test_qwen3_norm_rope_matches_the_transformers_ops_on_cpu(dt, hadamard):
    """The oracle against transformers' own Qwen3RMSNorm and apply_rotary_pos_emb (and the
    normalised FWHT) evaluated by torch on the CPU in the model dtype."""
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm, apply_rotary_pos_emb
    from oracle.rope import qwen3_norm_rope

    gen = torch.Generator().manual_seed(5)
    q = (torch.randn(2, 4, 3, 128, generator=gen) * 3).to(dt)
    k = (torch.randn(2, 2, 3, 128, generator=gen) * 3).to(dt)
    qn, kn = Qwen3RMSNorm(128, eps=1e-6).to(dt), Qwen3RMSNorm(128, eps=1e-6).to(dt)
    with torch.no_grad():
        qn.weight.copy_((torch.rand(128, generator=gen) * 2).to(dt))
        kn.weight.copy_((torch.rand(128, generator=gen) * 2).to(dt))
        cos, sin = _rope_tables_1d(2, 3, gen, dt)
        want_q, want_k = apply_rotary_pos_emb(qn(q.transpose(1, 2)).transpose(1, 2),
                                              kn(k.transpose(1, 2)).transpose(1, 2), cos, sin)
        if hadamard:  # the CPU branch of the reference: normalized_fwht(q).to(q.dtype)
            want_q = torch.from_numpy(normalized_fwht(want_q.float().numpy())).to(dt)
            want_k = torch.from_numpy(normalized_fwht(want_k.float().numpy())).to(dt)
    name = "bfloat16" if dt == torch.bfloat16 else "float16"
    f = lambda t: t.float().numpy()  # noqa: E731
    for x, w, want in ((q, qn.weight, want_q), (k, kn.weight, want_k)):
        got = qwen3_norm_rope(f(x), f(w.detach()), f(cos), f(sin), eps=1e-6, hadamard=hadamard, dtype=name)
        steps = _ulp_steps(got, f(want), name)
        # torch sums the squares in another order: a last-bit change of the variance may move the
        # normalised value's rounding by one step, rarely (two after the RoPE sum, in fp16)
        assert steps.max() <= 2 and (steps == 0).mean() >= 0.995, (steps.max(), (steps == 0).mean())


def test_qwen3_norm_rope_unit_weight_zero_angle_is_a_plain_rms_norm():
    from oracle.rope import qwen3_norm_rope

    rng = np.random.default_rng(7)
    x = rng.standard_normal((1, 2, 2, 128)).astype(np.float32)
    ones, zeros = np.ones((1, 2, 128), np.float32), np.zeros((1, 2, 128), np.float32)
    got = qwen3_norm_rope(x, np.ones(128, np.float32), ones, zeros, eps=0.0, hadamard=False, dtype="float32")
    want = x / np.sqrt((x.astype(np.float64) ** 2).mean(-1, keepdims=True))
    np.testing.assert_allclose(got, want, rtol=1e-6)
    np.testing.assert_allclose((got.astype(np.float64) ** 2).mean(-1), 1.0, rtol=1e-6)
