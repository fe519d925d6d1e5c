"""Pin the mRoPE oracle with closed forms (no reference fixture exists for the Triton kernel)."""
import numpy as np
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
