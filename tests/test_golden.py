"""Golden fixtures written by the reference xiaotu-moe CPU engine
(tests/golden/make_golden.py): the oracle reproduces the engine's outputs
within the parity bar, for every weight format, the INT8 ALIGN path and the
tiny Mixtral-style configuration.  Weights are regenerated from each
fixture's recipe and checked against its digest first."""
import os

import numpy as np
import pytest

import oracle
from golden.make_golden import CASES, weights_digest
from helpers import MAX_ABS, REL_L2, dense_to_numpy, make_dense_layer, rel_l2

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load_case(name):
    c = CASES[name]
    f = np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False)
    d = dense_to_numpy(c["fmt"], make_dense_layer(c["fmt"], c["E"] + c["NS"], c["H"], c["I"],
                                                  seed=c["seed"]))
    assert weights_digest(d) == str(f["digest"]), f"{name}: weight recipe drifted"
    return c, d, f


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_matches_reference_engine_fixture(name):
    c, d, f = load_case(name)
    args = (f["x_bits"], f["ids"], f["wts"], c["E"], c["NS"], c["H"], c["I"])
    if c.get("int8"):
        out = oracle.moe_layer_i8(*args, d["w13"], d["s13"], d["w2"], d["s2"], limit=c["limit"])
    else:
        out = oracle.moe_layer(c["fmt"], *args, d["w13"], d["s13"], d["w2"], d["s2"], d["gs13"],
                               d["gs2"], limit=c["limit"])
    ref = f["out"]
    assert rel_l2(out, ref) <= REL_L2, name
    assert np.max(np.abs(out - ref)) <= MAX_ABS, name
