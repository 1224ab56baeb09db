"""The HIP layer against the reference engine's golden outputs (fixtures of
tests/golden, written by the compiled reference xiaotu-moe CPU engine): every
weight format on the decode and the grouped-GEMM paths, the INT8 ALIGN path
and the tiny Mixtral-style configuration."""
import numpy as np
import pytest
import torch

from helpers import MAX_ABS, REL_L2, rel_l2
from golden.make_golden import act_args
from test_golden import CASES, load_case
from xtu_moe_amd.layer import ExpertWeights, moe_forward

pytestmark = pytest.mark.gpu


def _run(name, path):
    c, d, f = load_case(name)
    dev = torch.device("cuda")
    t = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a))
    w13, w2 = t(d["w13"]), t(d["w2"])
    if c["fmt"] == 0:   # bf16 bits -> bf16 tensors
        w13, w2 = w13.view(torch.bfloat16), w2.view(torch.bfloat16)
    W = ExpertWeights.from_dense(c["fmt"], w13, t(d["s13"]), w2, t(d["s2"]), t(d["gs13"]),
                                 t(d["gs2"]), n_shared=c["NS"], device=dev)
    x = torch.from_numpy(f["x_bits"].astype(np.int16)).view(torch.bfloat16).to(dev)
    a = act_args(c)
    out = moe_forward(x, torch.from_numpy(f["ids"]).to(dev), torch.from_numpy(f["wts"]).to(dev),
                      W, swiglu_limit=a["limit"], swiglu_alpha=a["alpha"], swiglu_beta=a["beta"],
                      path=path, int8=bool(c.get("int8")), out_dtype=torch.float32)
    torch.cuda.synchronize()
    return out.cpu().numpy(), f["out"]


@pytest.mark.parametrize("name", sorted(n for n in CASES if not CASES[n].get("int8")))
@pytest.mark.parametrize("path", ["decode", "gemm"])
def test_layer_matches_reference_engine(name, path):
    if path == "decode" and CASES[name]["T"] > 16:
        pytest.skip("decode path takes at most 16 tokens")
    out, ref = _run(name, path)
    assert rel_l2(out, ref) <= REL_L2, (name, path)
    assert np.max(np.abs(out - ref)) <= MAX_ABS, (name, path)


@pytest.mark.parametrize("name", sorted(n for n in CASES if CASES[n].get("int8")))
def test_int8_layer_matches_reference_engine(name):
    out, ref = _run(name, "gemm")
    assert rel_l2(out, ref) <= REL_L2, name
    assert np.max(np.abs(out - ref)) <= MAX_ABS, name
