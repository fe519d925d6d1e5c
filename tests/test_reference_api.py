"""normalized_fwht of the package (int2_reference.py:18-31) on the CPU: the oracle's stage order
bit for bit, the fp32 result dtype, any power-of-two width, and the reference's error."""
import numpy as np
import pytest
import torch

from oracle.quant import normalized_fwht as oracle_fwht


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("width", [1, 2, 64, 128, 256])
def test_normalized_fwht_matches_oracle(dtype, width):
    from r2omni_amd import normalized_fwht

    x = (torch.randn(3, 5, width, generator=torch.Generator().manual_seed(width)) * 3).to(dtype)
    got = normalized_fwht(x)
    assert got.dtype == torch.float32 and got.shape == x.shape
    np.testing.assert_array_equal(got.numpy(), oracle_fwht(x.float().numpy()))


def test_normalized_fwht_is_an_involution_and_rejects_bad_widths():
    from r2omni_amd import normalized_fwht

    x = torch.randn(4, 128, dtype=torch.float64).float()
    np.testing.assert_allclose(normalized_fwht(normalized_fwht(x)).numpy(), x.numpy(), atol=2e-6)
    e0 = torch.zeros(128)
    e0[0] = 1
    np.testing.assert_allclose(normalized_fwht(e0).numpy(), np.full(128, 128 ** -0.5), rtol=1e-7)
    with pytest.raises(ValueError, match="power of two"):
        normalized_fwht(torch.zeros(2, 96))
