"""The e4m3-pair split reconstructs bf16 rows exactly (the property the exact
FP8 prefill GEMMs rely on), with every scaled value inside the e4m3 range."""
import numpy as np
import torch

from fp8pair_ref import fp8pair_join, fp8pair_split, wide_rows


def test_split_reconstructs_bf16_rows_exactly():
    x = wide_rows(64, 512, seed=1)
    hi, lo, sa, sl = fp8pair_split(x)
    np.testing.assert_array_equal(fp8pair_join(hi, lo, sa, sl), x.double().numpy())


def test_scale_is_the_smallest_that_fits_448():
    x = wide_rows(16, 256, seed=2)
    _, _, sa, _ = fp8pair_split(x)
    amax = x.float().reshape(16, 8, 32).abs().amax(-1).double()
    e = sa.double() - 127
    nz = amax > 0
    assert torch.all(amax[nz] / torch.pow(2.0, e[nz]) <= 448.0)
    assert torch.all(amax[nz] / torch.pow(2.0, e[nz] - 1) > 448.0)


def test_no_nan_codes():
    hi, lo, _, _ = fp8pair_split(wide_rows(8, 256, seed=3))
    for t in (hi, lo):
        assert not torch.any((t & 0x7F) == 0x7F)
