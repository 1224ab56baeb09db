"""Golden fixtures written by the reference xiaotu-moe CPU engine
(tests/golden/make_golden.py): the oracle reproduces the engine's outputs
within the parity bar, for every weight format, the INT8 ALIGN path and the
tiny Mixtral-style configuration.  Weights are regenerated from each
fixture's recipe and checked against its digest first."""
import os

import numpy as np
import pytest

import oracle
from golden.make_golden import CASES, act_args, weights_digest
from helpers import MAX_ABS, REL_L2, dense_to_numpy, make_dense_layer, rel_l2

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load_case(name):
    c = CASES[name]
    f = np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False)
    d = dense_to_numpy(c["fmt"], make_dense_layer(c["fmt"], c["E"] + c["NS"], c["H"], c["I"],
                                                  seed=c["seed"], std=c.get("std", 0.02)))
    assert weights_digest(d) == str(f["digest"]), f"{name}: weight recipe drifted"
    return c, d, f


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_matches_reference_engine_fixture(name):
    c, d, f = load_case(name)
    args = (f["x_bits"], f["ids"], f["wts"], c["E"], c["NS"], c["H"], c["I"])
    if c.get("int8"):
        out = oracle.moe_layer_i8(*args, d["w13"], d["s13"], d["w2"], d["s2"], **act_args(c))
    else:
        out = oracle.moe_layer(c["fmt"], *args, d["w13"], d["s13"], d["w2"], d["s2"], d["gs13"],
                               d["gs2"], **act_args(c))
    ref = f["out"]
    assert rel_l2(out, ref) <= REL_L2, name
    assert np.max(np.abs(out - ref)) <= MAX_ABS, name


@pytest.mark.parametrize("name", sorted(n for n in CASES if "alpha" in CASES[n]))
def test_activation_fixtures_pin_alpha_and_beta(name):
    """The SwiGLU-OAI fixtures fail the bar for an oracle that drops alpha or
    beta: they pin both terms, not just the clamp."""
    c, d, f = load_case(name)
    args = (f["x_bits"], f["ids"], f["wts"], c["E"], c["NS"], c["H"], c["I"])
    fn = oracle.moe_layer_i8 if c.get("int8") else (
        lambda *a, **k: oracle.moe_layer(c["fmt"], *a[:7], a[7], a[8], a[9], a[10], d["gs13"],
                                         d["gs2"], **k))
    for wrong in (dict(alpha=1.0, beta=c["beta"]), dict(alpha=c["alpha"], beta=0.0)):
        out = fn(*args, d["w13"], d["s13"], d["w2"], d["s2"], limit=c["limit"], **wrong)
        assert rel_l2(out, f["out"]) > 10 * REL_L2, (name, wrong)


def test_offset_guard_fixture_is_past_the_guard():
    """In small_mxfp4_int8_g2 every gate/up and down tile of the reference
    engine fails its offset guard cmin + emin - 128 >= -24 (so the engine
    took its fp32 path there), while the INT8 restatement, which scales each
    row in fp32 after an int32 sum that cannot overflow (|ACC| <= K/32 *
    48768 * 8), stays within the layer bar of it (the fixture test above)
    and its accumulators stay exact."""
    c, d, f = load_case("small_mxfp4_int8_g2")
    x = oracle.bf16_bits_to_f32(f["x_bits"])
    cmin = min(oracle.i8_quant_row(row)[1] for row in x)
    emin13 = int(d["s13"].min())
    assert cmin + emin13 - 128 < -24
    # down: the activation rows the engine quantises are bf16(act) of the
    # routed pairs; their exponents are smaller still
    ids, wts = f["ids"], f["wts"]
    E, NS, H, I = c["E"], c["NS"], c["H"], c["I"]
    w13 = d["w13"]
    deq = oracle.e2m1_table()[np.stack([w13 & 15, w13 >> 4], -1).reshape(E + NS, 2 * I, H)]
    deq = deq * oracle.e8m0_table()[np.repeat(d["s13"], 32, axis=-1)]
    crows = []
    for t in range(c["T"]):
        for e in [int(i) for i, w in zip(ids[t], wts[t]) if 0 <= i < E and w != 0] + [E]:
            g = deq[e, :I] @ x[t]
            u = deq[e, I:] @ x[t]
            act = g / (1 + np.exp(-g)) * u
            crows.append(oracle.i8_quant_row(act.astype(np.float32))[1])
    assert max(crows) + int(d["s2"].min()) - 128 < -24
    # the restatement takes the fp32 path on these rows as the engine did:
    # agreement far inside the ~2e-2 that the INT8 rounding alone would leave
    args = (f["x_bits"], f["ids"], f["wts"], E, NS, H, I)
    out = oracle.moe_layer_i8(*args, d["w13"], d["s13"], d["w2"], d["s2"], **act_args(c))
    assert rel_l2(out, f["out"]) < 1e-5
    # the accumulators of the INT8 restatement equal the int64 closed form
    acc, _, dmax = oracle.i8_gemm(x, d["w13"][0], d["s13"][0])
    assert dmax <= 3 and np.abs(acc).max() < 2 ** 31
