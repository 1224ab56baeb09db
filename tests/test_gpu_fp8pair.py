"""The device split (xtu_fp8pair_quant) equals the CPU restatement byte for
byte and reconstructs the rows exactly."""
import numpy as np
import pytest
import torch

from fp8pair_ref import fp8pair_join, fp8pair_split, wide_rows
from xtu_moe_amd import _lib
from xtu_moe_amd.layer import _p

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,K", [(1, 128), (37, 2048), (300, 7168)])
def test_device_split_matches_restatement(M, K):
    x = wide_rows(M, K, seed=M)
    dev = torch.device("cuda")
    xd = x.to(dev)
    hi = torch.empty((M, K), dtype=torch.uint8, device=dev)
    lo = torch.empty_like(hi)
    sa = torch.empty((M, K // 32), dtype=torch.uint8, device=dev)
    sl = torch.empty_like(sa)
    _lib.call("xtu_fp8pair_quant", _p(xd), M, K, _p(hi), _p(lo), _p(sa), _p(sl), 0)
    torch.cuda.synchronize()
    rh, rl, rsa, rsl = fp8pair_split(x)
    for got, ref in ((hi, rh), (lo, rl), (sa, rsa), (sl, rsl)):
        np.testing.assert_array_equal(got.cpu().numpy(), ref.numpy())
    np.testing.assert_array_equal(fp8pair_join(hi.cpu(), lo.cpu(), sa.cpu(), sl.cpu()),
                                  x.double().numpy())
