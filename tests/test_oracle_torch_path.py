"""The torch-CPU restatement (oracle/torch_path.py, the CPU baseline) equals the numpy oracle bit for
bit: every dequantised pool and the attention output, for every cache variant, before and after a
flush with a partial K superblock tail.  The numpy oracle itself is pinned by the reference's own
golden fixtures (test_oracle_golden.py)."""
import numpy as np
import pytest
import torch

from oracle import torch_path
from oracle.attention import mixed_reference
from oracle.cache import append_token, build_cache, pool_kv
from oracle.quant import bf16_bits_to_f32, f32_to_bf16_bits


def _bf16(x):
    return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(x, np.float32)))


@pytest.mark.parametrize("variant,sb,group,gen", [("int4k", 32, 32, "int2"), ("int4k", 128, 128, "int2"),
                                                  ("int2k", 32, 64, "int2"), ("bf16k", 32, 32, "int2"),
                                                  ("matched", 32, 32, "int2"), ("int4k", 32, 32, "int4"),
                                                  ("int2k", 128, 128, "int4")])
def test_torch_path_equals_numpy_oracle(variant, sb, group, gen):
    rng = np.random.default_rng(5)
    h, pages = 2, 23
    hist = pages * 32 + 16  # a partial last page: the K arena ends inside a superblock
    key = _bf16(rng.standard_normal((h, hist, 128)) * np.where(np.arange(128) % 37 == 0, 8.0, 1.0))
    value = _bf16(rng.standard_normal((h, hist, 128)))
    offsets = np.arange(pages + 1) * 32
    lengths = np.array([32] * pages + [16])
    classes = rng.choice([1, 2, 5], size=pages + 1, p=(0.2, 0.5, 0.3))
    oc = build_cache(key, value, offsets, lengths, classes, dtype="bfloat16", page_size=32, superblock=sb,
                     group=group, variant=variant, gen_values=gen)
    q = _bf16(rng.standard_normal((1, 8, 128)))
    steps = 60 if variant == "bf16k" else 140  # v_fourq_k_bf16 refuses a flush
    for step in range(steps):
        append_token(oc, _bf16(rng.standard_normal((h, 128))), _bf16(rng.standard_normal((h, 128))),
                     global_index=hist + step, logical_position=hist + step)
        if step in (steps // 2, steps - 1):
            tc = torch_path.from_oracle(oc)
            got, want = torch_path.pool_kv(tc), pool_kv(oc)
            assert len(got) == len(want)
            for (gk, gv), (wk, wv) in zip(got, want):
                np.testing.assert_array_equal(gk.numpy(), wk)
                np.testing.assert_array_equal(gv.numpy(), wv)
            np.testing.assert_array_equal(torch_path.mixed_reference(q, tc), mixed_reference(q, oc))
    assert oc.flushed_tokens == (0 if variant == "bf16k" else 128)


def test_torch_path_dequantises_on_every_call():
    """The cache holds packed codes only: the dequantised pools are new tensors on each call."""
    rng = np.random.default_rng(6)
    key = _bf16(rng.standard_normal((1, 64, 128)))
    oc = build_cache(key, key, np.array([0, 32]), np.array([32, 32]), np.array([2, 5]), dtype="bfloat16")
    tc = torch_path.from_oracle(oc)
    a, b = torch_path.pool_kv(tc), torch_path.pool_kv(tc)
    assert all(x[0].data_ptr() != y[0].data_ptr() for x, y in zip(a, b))
    assert tc.k_packed.dtype == torch.uint8 and tc.v2_packed.dtype == torch.uint8
