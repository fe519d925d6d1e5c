"""Load the golden fixtures written by tests/golden/make_golden.py (data only)."""
import glob
import os

import numpy as np

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _all_names():
    return sorted(os.path.splitext(os.path.basename(p))[0] for p in glob.glob(os.path.join(HERE, "*.npz")))


def _keys(name):
    return set(np.load(os.path.join(HERE, name + ".npz"), allow_pickle=False).files)


def fixture_names():
    """Fixtures of the compact INT4-K cache (v_fourq_k_int4_compact) with INT2 generated values."""
    return [n for n in _all_names() if not {"variant", "gen_values"} & _keys(n)]


def gen_int4_fixture_names():
    """Fixtures of the compact INT4-K cache with INT4 generated values (generated_value_precision="int4")."""
    return [n for n in _all_names() if "gen_values" in _keys(n)]


def variant_fixture_names():
    """Fixtures of the BF16-K caches (matched-FP and v_fourq_k_bf16)."""
    return [n for n in _all_names() if "variant" in _keys(n)]


def load(name):
    return dict(np.load(os.path.join(HERE, name + ".npz"), allow_pickle=False))


def as_f32(arr, dtype):
    """Fixture tensors of dtype bfloat16 are stored as uint16 bit patterns."""
    from oracle.quant import bf16_bits_to_f32

    if "bfloat16" in str(dtype):
        return bf16_bits_to_f32(arr)
    return np.asarray(arr).astype(np.float32)
