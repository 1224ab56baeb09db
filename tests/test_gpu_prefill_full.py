"""DeepSeek-V3 FP8 layer at its full prefill size (H=7168, I=2048, 256 routed
+ 1 shared experts, T=8192 tokens, grouped sigmoid top-8): properties that
hold at any size, and sampled tokens against the oracle.

* Token permutation: each output row is reduced in a fixed order that does
  not depend on the row's position in its M tile or on the other tokens, so
  permuting the batch permutes the output bit for bit.
* Sampled tokens: the oracle's dequantised-fp32 layer for a set of tokens
  that routes to every expert (a greedy cover, with the last rows of eight
  experts' buckets; plus the first, a middle and the last token; only their
  experts, at full H and I); the layer's bf16 output
  within max-abs 2e-2 (plus half a bf16 ulp of the value) and rel-L2 5e-3.
  The FP8 prefill GEMM is exact up to fp32 rounding (e4m3 weights against
  exact e4m3 activation pairs on the scaled fp8 MFMA, fp32 accumulation, the
  block scales applied by accumulator rescaling); what remains is the bf16
  rounding of act before down and of the output, so the comparison is made
  on the bf16 outputs the layer returns and the fp32 rel-L2 is held to the
  same 5e-3.
"""
import numpy as np
import pytest
import torch

from helpers import REL_L2, check_close, cover_tokens, rel_l2, sampled_oracle
from xtu_moe_amd import formats as F
from xtu_moe_amd.layer import moe_forward, route
from xtu_moe_amd.synthetic import synth_layer

pytestmark = pytest.mark.gpu

H, I, E, NS, K, T = 7168, 2048, 256, 1, 8, 8192


@pytest.fixture(scope="module")
def layer():
    dev = torch.device("cuda")
    W = synth_layer(F.FMT_FP8, E, NS, H, I, seed=3, device=dev)
    g = torch.Generator(device=dev).manual_seed(11)
    x = torch.randn((T, H), generator=g, device=dev).to(torch.bfloat16)
    logits = torch.randn((T, E), generator=g, device=dev)
    wts, ids = route(logits, top_k=K, scoring="sigmoid", n_group=8, topk_group=4,
                     routed_scaling_factor=2.5)
    out = moe_forward(x, ids, wts, W, out_dtype=torch.float32)
    torch.cuda.synchronize()
    yield W, x, ids, wts, out
    del W
    torch.cuda.empty_cache()


def test_token_permutation_is_bitwise_equivariant(layer):
    W, x, ids, wts, out = layer
    perm = torch.randperm(T, generator=torch.Generator().manual_seed(5)).to(x.device)
    out_p = moe_forward(x[perm].contiguous(), ids[perm].contiguous(), wts[perm].contiguous(), W,
                        out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(out_p, out[perm])


def test_sampled_tokens_match_oracle(layer):
    """Tokens that together route to every one of the 256 experts (a greedy
    cover, with the last token of eight experts' buckets, whose pairs sit in
    partial M tiles), plus the first, a middle and the last token."""
    W, x, ids, wts, out = layer
    toks, covered = cover_tokens(ids.cpu().numpy(), E, seed=7)
    assert len(covered) == E   # every routed expert (the shared one is in every token)
    toks = sorted(set(toks) | {0, T // 2 + 17, T - 1})
    ref = sampled_oracle(F.FMT_FP8, W, x, ids, wts, toks)
    got = out[toks]
    check_close(got.to(torch.bfloat16).float().cpu().numpy(), ref, bf16_out=True,
                what="ds-v3 fp8 T=8192 sample (bf16 output)")
    assert rel_l2(got.cpu().numpy(), ref) <= REL_L2
