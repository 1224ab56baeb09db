"""Weighted unpermute (xtu_combine) against a float64 restatement of the
reference's per-token ordered sum (moe_v2.hpp:920-930): pairs in top-k order,
pairs sent to the trash bucket or with zero weight skipped, shared rows added
with weight 1.  Top-k widths with and without a compile-time shape, small and
larger batches."""
import numpy as np
import pytest
import torch

from helpers import random_routing
from xtu_moe_amd import layer as L

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T,K,E,NS,H", [(7, 1, 8, 0, 256), (33, 3, 16, 1, 512), (64, 4, 32, 0, 1024),
                                        (50, 8, 64, 1, 2048), (40, 10, 512, 2, 768),
                                        (9, 11, 40, 1, 128), (300, 8, 64, 1, 1280),
                                        (257, 2, 8, 0, 256)])
@pytest.mark.parametrize("drop_zero", [False, True])
@pytest.mark.parametrize("out_bf16", [False, True])
def test_combine_matches_ordered_sum(T, K, E, NS, H, drop_zero, out_bf16):
    ids, wts = random_routing(T, K, E, seed=T * K + H, invalid_frac=0.1, zero_frac=0.1)
    dev = torch.device("cuda")
    seg = L.segmentation(T, K, E, NS, 128, dev)
    seg.run(torch.from_numpy(ids).cuda(), torch.from_numpy(wts).cuda(), None, drop_zero)
    g = torch.Generator(device=dev).manual_seed(T + K)
    y = torch.randn((max(seg.A, 1), H), generator=g, device=dev)
    out = torch.empty((T, H), dtype=torch.bfloat16 if out_bf16 else torch.float32, device=dev)
    wt = torch.from_numpy(wts).cuda()
    L.combine(seg, y, wt, out)
    torch.cuda.synchronize()
    inv = seg.inv.cpu().numpy()[: seg.A]
    trash = int(seg.seg_start[E + NS].item())
    yn = y.cpu().numpy().astype(np.float64)
    ref = np.zeros((T, H))
    for t in range(T):
        for k in range(K):
            pos, w = inv[t * K + k], float(wts[t, k])
            if pos < trash and w != 0.0:
                ref[t] += w * yn[pos]
        for s in range(NS):
            ref[t] += yn[inv[T * K + t * NS + s]]
    got = out.float().cpu().numpy()
    if out_bf16:
        np.testing.assert_allclose(got, ref, rtol=1e-2, atol=1e-2)
    else:
        np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)
    # a token whose pairs were all dropped and that has no shared row is exactly 0
    dropped = [t for t in range(T) if NS == 0 and all(
        inv[t * K + k] >= trash or wts[t, k] == 0.0 for k in range(K))]
    for t in dropped:
        assert not got[t].any()
