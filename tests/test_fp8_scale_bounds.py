"""The FP8 prefill kernel choice (CPU): the 32x32x64 kernel carries its
accumulators in units of the current block scale and rescales by
s(kb-1)/s(kb), so it is taken only for scales that are finite, positive and
within 2^32 of each other; the choice is made when the weights are built
(so a graph captured later takes the kernel eager calls take), and the host
store's answer for slot planes agrees with the resident weights'."""
import math

import torch

from helpers import make_dense_layer
from xtu_moe_amd import formats as F
from xtu_moe_amd.host_store import HostExpertStore
from xtu_moe_amd.layer import FP8_RATIO_MAX, ExpertWeights, fp8_block_scales_bounded


def test_bound_semantics():
    s = torch.full((2, 3, 4), 0.01)
    assert fp8_block_scales_bounded(s)
    for bad in (0.0, -0.01, math.inf, math.nan):
        t = s.clone()
        t[1, 2, 3] = bad
        assert not fp8_block_scales_bounded(t), bad
    t = s.clone()
    t[0, 0, 0] = 0.01 * FP8_RATIO_MAX              # max/min exactly 2^32: taken
    assert fp8_block_scales_bounded(t)
    t[0, 0, 0] = 0.01 * FP8_RATIO_MAX * 2          # beyond: not taken
    assert not fp8_block_scales_bounded(t)
    # the bound spans every tensor given
    assert not fp8_block_scales_bounded(s, s * FP8_RATIO_MAX * 4)


def test_decided_at_build_and_host_store_agrees():
    d = make_dense_layer(F.FMT_FP8, 3, 256, 128, seed=4)
    W = ExpertWeights.from_dense(F.FMT_FP8, d["w13"], d["s13"], d["w2"], d["s2"], device="cpu")
    assert W._fp8_pos is True
    assert HostExpertStore.from_weights(W, pin=False).fp8_scales_bounded()
    d["s13"][2, 1, 0] = 0.0
    W2 = ExpertWeights.from_dense(F.FMT_FP8, d["w13"], d["s13"], d["w2"], d["s2"], device="cpu")
    assert W2._fp8_pos is False
    assert not HostExpertStore.from_weights(W2, pin=False).fp8_scales_bounded()
    # slot planes decide nothing themselves
    slots = ExpertWeights(F.FMT_FP8, 256, 128, 3, 0, W.w13.clone(), W.s13.clone(), W.w2.clone(),
                          W.s2.clone(), mutable=True)
    assert slots._fp8_pos is None
