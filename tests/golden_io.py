"""Load the golden fixtures written by tests/golden/make_golden.py (data only)."""
import glob
import os

import numpy as np

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def fixture_names():
    return sorted(os.path.splitext(os.path.basename(p))[0] for p in glob.glob(os.path.join(HERE, "*.npz")))


def load(name):
    return dict(np.load(os.path.join(HERE, name + ".npz"), allow_pickle=False))


def as_f32(arr, dtype):
    """Fixture tensors of dtype bfloat16 are stored as uint16 bit patterns."""
    from oracle.quant import bf16_bits_to_f32

    if "bfloat16" in str(dtype):
        return bf16_bits_to_f32(arr)
    return np.asarray(arr).astype(np.float32)
