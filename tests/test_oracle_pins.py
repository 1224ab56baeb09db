"""Pins of the oracle (CPU restatement of the reference's algorithm) against
closed forms, brute force and textbook routines -- each check is independent
of the oracle's own code, so a dropped term, a wrong sign or index, or a
transposed operand in the restatement fails here.

Codecs: exhaustive against the OCP definitions and torch's float8 decoding.
expf / sigmoid: against float64 libm.  Routers: against a sort-based brute
force.  Segmentation: against numpy's stable argsort.  Expert math: against a
float64 dense computation from the codec tables, and (where the reference
engine is built) against the reference xiaotu-moe CPU engine itself.  INT8
ALIGN: accumulators against an int64 closed form."""
import math

import numpy as np
import pytest
import torch

import oracle
from helpers import MAX_ABS, REL_L2, dense_to_numpy, make_dense_layer, random_routing, rel_l2
from xtu_moe_amd import formats as F


# ----------------------------------------------------------------------- codecs
def test_e2m1_table_closed_form():
    # OCP MX e2m1: sign, 2 exponent bits (bias 1), 1 mantissa bit; e=0 subnormal
    want = []
    for c in range(16):
        s = -1.0 if c & 8 else 1.0
        e, m = (c >> 1) & 3, c & 1
        want.append(s * (0.5 * m if e == 0 else (1.0 + 0.5 * m) * 2.0 ** (e - 1)))
    np.testing.assert_array_equal(oracle.e2m1_table(), np.array(want, np.float32))
    np.testing.assert_array_equal(np.array(F.E2M1_VALUES, np.float32), np.array(want, np.float32))


def test_e8m0_table_exhaustive():
    t = oracle.e8m0_table()
    for b in range(255):
        assert t[b] == np.float32(math.ldexp(1.0, b - 127)), b
    assert np.isinf(t[255])


def test_e4m3_table_exhaustive_vs_torch():
    t = oracle.e4m3_table()
    ref = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    finite = np.isfinite(ref)
    np.testing.assert_array_equal(t[finite], ref[finite])
    # e4m3fn has no infinities; 0x7F / 0xFF are NaN and never produced by the quantiser
    assert not finite[[0x7F, 0xFF]].any()


def test_bf16_rounding_vs_torch():
    rng = np.random.default_rng(0)
    f = np.concatenate([rng.standard_normal(10000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 10000),
                        np.array([0.0, -0.0, np.inf, -np.inf, 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8,
                                  3.3895314e38], np.float32)]).astype(np.float32)
    ours = oracle.f32_to_bf16_bits(f)
    ref = torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, ref)


# ------------------------------------------------------------ exp and sigmoid
def test_expf_within_two_ulp_of_libm():
    x = np.concatenate([np.linspace(-87.0, 88.0, 20001), [0.0, -1e-30, 1e-30, 1.0, -1.0]]).astype(np.float32)
    got = oracle.expf(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert np.max(np.abs(got - ref) / ulp) <= 2.0
    assert oracle.expf(np.array([0.0], np.float32))[0] == 1.0
    assert oracle.expf(np.array([-200.0], np.float32))[0] == 0.0
    assert np.isinf(oracle.expf(np.array([100.0], np.float32))[0])


def test_sigmoid_and_silu_gate():
    L = oracle.lib()
    for v in np.linspace(-30, 30, 601).astype(np.float32):
        want = 1.0 / (1.0 + math.exp(-float(v)))
        assert abs(L.xo_sigmoid(float(v)) - want) <= 2.5 * np.spacing(np.float32(want))
    # act = g' * sigmoid(alpha g') * (u' + beta), gate clamped above, up both sides
    for g, u, lim, a, b in [(1.5, -2.0, 0.0, 1.0, 0.0), (9.0, 8.0, 7.0, 1.0, 0.0),
                            (-3.0, -9.0, 7.0, 1.702, 1.0), (0.25, 0.5, 0.0, 1.0, 1.0)]:
        gp = min(g, lim) if lim > 0 else g
        up = min(max(u, -lim), lim) if lim > 0 else u
        want = gp / (1.0 + math.exp(-a * gp)) * (up + b)
        assert abs(L.xo_silu_gate(g, u, lim, a, b) - want) <= 1e-5 * max(1.0, abs(want))


# ---------------------------------------------------------------------- routing
def _brute_topk(score, K, allowed=None):
    idx = [e for e in range(len(score)) if allowed is None or allowed[e]]
    return sorted(idx, key=lambda e: (-float(score[e]), e))[:K]


@pytest.mark.parametrize("T,E,K", [(5, 8, 2), (7, 64, 6), (4, 512, 10)])
@pytest.mark.parametrize("renorm", [True, False])
def test_softmax_topk_brute_force(T, E, K, renorm):
    rng = np.random.default_rng(E + K)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    lg[0, : E // 2] = np.round(lg[0, : E // 2])   # exact ties -> lower index first
    ids, wts = oracle.route_softmax_topk(lg, K, renormalize=renorm)
    for t in range(T):
        want = _brute_topk(lg[t], K)
        assert list(ids[t]) == want
        p = np.exp(lg[t].astype(np.float64) - lg[t].max())
        den = p[want].sum() if renorm else p.sum()
        np.testing.assert_allclose(wts[t], p[want] / den, rtol=2e-6, atol=1e-8)


@pytest.mark.parametrize("with_bias", [False, True])
def test_grouped_sigmoid_brute_force(with_bias):
    rng = np.random.default_rng(3)
    T, E, G, TG, K, scale = 9, 256, 8, 4, 8, 2.5
    lg = rng.standard_normal((T, E)).astype(np.float32)
    lg[1] = np.round(lg[1] * 2) / 2
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32) if with_bias else None
    ids, wts = oracle.route_grouped_sigmoid(lg, bias, G, TG, K, scale)
    gsz = E // G
    for t in range(T):
        s = 1.0 / (1.0 + np.exp(-lg[t].astype(np.float64)))
        sel = s + (0 if bias is None else bias.astype(np.float64))
        # fp32 selection scores as the router forms them (sigmoid in fp32, + bias in fp32)
        sel32 = (oracle.lib() and np.array([oracle.lib().xo_sigmoid(float(v)) for v in lg[t]], np.float32))
        sel32 = sel32 + (np.float32(0) if bias is None else bias)
        gscore = [sum(sorted(sel32[g * gsz:(g + 1) * gsz], reverse=True)[:2]) for g in range(G)]
        groups = sorted(range(G), key=lambda g: (-float(np.float32(gscore[g])), g))[:TG]
        allowed = np.zeros(E, bool)
        for g in groups:
            allowed[g * gsz:(g + 1) * gsz] = True
        want = _brute_topk(sel32, K, allowed)
        assert list(ids[t]) == want
        np.testing.assert_allclose(wts[t], s[want] / s[want].sum() * scale, rtol=2e-6)
        assert abs(float(sel[want[0]]) - float(sel32[want[0]])) < 1e-6


# ----------------------------------------------------------------- segmentation
@pytest.mark.parametrize("T,K,E,NS", [(0, 4, 16, 1), (1, 8, 256, 1), (37, 3, 20, 2), (300, 8, 64, 0)])
@pytest.mark.parametrize("drop_zero", [False, True])
def test_segment_vs_stable_argsort(T, K, E, NS, drop_zero):
    ids, wts = random_routing(T, K, E, seed=T + 1, invalid_frac=0.1, zero_frac=0.1)
    r = oracle.segment(ids, wts, E, NS, drop_zero)
    flat_ids = ids.reshape(-1)
    flat_w = wts.reshape(-1)
    bucket = np.where((flat_ids < 0) | (flat_ids >= E), E + NS, flat_ids)
    if drop_zero:
        bucket = np.where(flat_w == 0.0, E + NS, bucket)
    shared = np.array([E + s for t in range(T) for s in range(NS)], np.int64)
    bucket = np.concatenate([bucket, shared]).astype(np.int64)
    tok = np.concatenate([np.repeat(np.arange(T), K), np.repeat(np.arange(T), NS)])
    w = np.concatenate([flat_w, np.ones(T * NS, np.float32)])
    order = np.argsort(bucket, kind="stable")
    np.testing.assert_array_equal(r["sorted_pair"], order)
    np.testing.assert_array_equal(r["sorted_tok"], tok[order])
    np.testing.assert_array_equal(r["sorted_wts"], w[order])
    inv = np.empty_like(order)
    inv[order] = np.arange(len(order))
    np.testing.assert_array_equal(r["inv"], inv)
    counts = np.bincount(bucket, minlength=E + NS + 1)
    np.testing.assert_array_equal(r["seg_start"], np.concatenate([[0], np.cumsum(counts)]))


# ------------------------------------------------------------------ expert math
def _dense_f64_layer(fmt, d, x_bits, ids, wts, E, NS, H, I, limit=0.0):
    """Independent float64 restatement from the codec tables (no oracle code)."""
    def deq(w, s, gs):
        if fmt == F.FMT_BF16:
            return oracle.bf16_bits_to_f32(w).astype(np.float64)
        return F.dequantize(fmt, *(torch.as_tensor(v) if v is not None else None
                                   for v in (w, s, gs))).double().numpy()

    W13 = deq(d["w13"], d["s13"], d["gs13"])
    W2 = deq(d["w2"], d["s2"], d["gs2"])
    x = oracle.bf16_bits_to_f32(x_bits).astype(np.float64)
    T, K = ids.shape
    out = np.zeros((T, H))
    for t in range(T):
        routed = [(int(ids[t, k]), float(wts[t, k])) for k in range(K)
                  if 0 <= ids[t, k] < E and wts[t, k] != 0.0]   # invalid ids are ignored
        for e, wgt in routed + [(E + s, 1.0) for s in range(NS)]:
            gu = W13[e] @ x[t]
            g, u = gu[:I], gu[I:]
            if limit > 0:
                g = np.minimum(g, limit)
                u = np.clip(u, -limit, limit)
            act = g / (1.0 + np.exp(-g)) * u
            act = oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(act.astype(np.float32))).astype(np.float64)
            out[t] += wgt * (W2[e] @ act)
    return out


FMTS = [F.FMT_BF16, F.FMT_FP8, F.FMT_MXFP4, F.FMT_NVFP4, F.FMT_INT4]


@pytest.mark.parametrize("fmt", FMTS)
def test_oracle_layer_vs_float64_dense(fmt):
    E, NS, H, I, T, K = 6, 1, 256, 128, 7, 2
    d = dense_to_numpy(fmt, make_dense_layer(fmt, E + NS, H, I, seed=fmt + 10))
    ids, wts = random_routing(T, K, E, seed=2, invalid_frac=0.15, zero_frac=0.1)
    x = oracle.f32_to_bf16_bits(np.random.default_rng(4).standard_normal((T, H)).astype(np.float32))
    got = oracle.moe_layer(fmt, x, ids, wts, E, NS, H, I, d["w13"], d["s13"], d["w2"], d["s2"],
                           d["gs13"], d["gs2"], limit=4.0)
    ref = _dense_f64_layer(fmt, d, x, ids, wts, E, NS, H, I, limit=4.0)
    # the only rounding the two share is act -> bf16; a near-tie can flip one bf16 ulp
    assert rel_l2(got, ref) < 1e-3
    assert np.max(np.abs(got - ref)) < 2e-3


@pytest.mark.skipif(not oracle.ref_available(), reason="reference engine build not available")
@pytest.mark.parametrize("fmt", FMTS)
def test_oracle_layer_vs_reference_engine(fmt):
    """The compiled reference xiaotu-moe engine (MOE_V2::forward_many) on the
    same checkpoint-layout weights: the oracle sits within the parity bar."""
    E, NS, H, I, T, K = 6, 0, 256, 256, 9, 3
    d = dense_to_numpy(fmt, make_dense_layer(fmt, E, H, I, seed=fmt + 20))
    ids, wts = random_routing(T, K, E, seed=5)
    x = oracle.f32_to_bf16_bits(np.random.default_rng(6).standard_normal((T, H)).astype(np.float32))
    got = oracle.moe_layer(fmt, x, ids, wts, E, NS, H, I, d["w13"], d["s13"], d["w2"], d["s2"],
                           d["gs13"], d["gs2"])
    eng = oracle.RefEngine(fmt, E, K, H, I, d["w13"], d["s13"], d["w2"], d["s2"], d["gs13"], d["gs2"])
    ref = eng.forward(x, ids, wts)
    eng.close()
    assert rel_l2(got, ref) <= REL_L2
    assert np.max(np.abs(got - ref)) <= MAX_ABS


# ------------------------------------------------------------------ INT8 ALIGN
def test_i8_quant_row_closed_form():
    rng = np.random.default_rng(8)
    for scale in (1e-3, 0.7, 3.0, 1e4):
        a = (rng.standard_normal(512) * scale).astype(np.float32)
        a8, crow = oracle.i8_quant_row(a)
        m = np.float32(np.abs(a).max())
        bits = int(m.view(np.uint32))
        ef, mant = (bits >> 23) & 255, bits & 0x7FFFFF
        want_crow = max(-120, min(120, (ef - 127) - 6 + (1 if mant > 0x7E0000 else 0)))
        assert crow == want_crow
        want = np.clip(np.rint(a.astype(np.float64) * 2.0 ** -crow), -127, 127).astype(np.int8)
        np.testing.assert_array_equal(a8, want)


def test_i8_gemm_accumulators_closed_form():
    """ACC[m][n] = sum_g D_g * 2^(b_g - emin_n), D_g = sum a8 * (2 e2m1) in int64."""
    rng = np.random.default_rng(9)
    M, N, K = 5, 32, 256
    a = rng.standard_normal((M, K)).astype(np.float32)
    codes = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    s = rng.integers(120, 124, (N, K // 32), dtype=np.uint8)   # spread <= 3
    acc, c, dmax = oracle.i8_gemm(a, codes, s)
    assert dmax <= 3
    w4 = np.empty((N, K), np.int64)
    e2m1 = np.array(F.E2M1_VALUES)
    w4[:, 0::2] = (2 * e2m1[codes & 15]).astype(np.int64)
    w4[:, 1::2] = (2 * e2m1[codes >> 4]).astype(np.int64)
    for m in range(M):
        a8, crow = oracle.i8_quant_row(a[m])
        a8 = a8.astype(np.int64)
        for n in range(N):
            emin = int(s[n].min())
            tot = 0
            for g in range(K // 32):
                D = int(np.dot(a8[g * 32:(g + 1) * 32], w4[n, g * 32:(g + 1) * 32]))
                tot += D << (int(s[n, g]) - emin)
            assert acc[m, n] == tot
            want_c = float(tot) * 2.0 ** (emin - 128) * 2.0 ** crow
            assert abs(c[m, n] - want_c) <= 1e-6 * max(1.0, abs(want_c))


# --------------------------------------------------------------------- formats
@pytest.mark.parametrize("fmt", FMTS)
def test_pack_unpack_round_trip(fmt):
    E, N, K = 3, 128, 384
    w = torch.randn((E, N, K)) * 0.02
    q, s, gs = F.quantize(fmt, w)
    p = F.pack_weight(fmt, q)
    assert p.shape == (E, N * F.row_bytes(fmt, K))
    back = F.unpack_weight(fmt, p, N, K)
    assert torch.equal(back.view(torch.uint8) if fmt == F.FMT_BF16 else back,
                       q.view(torch.uint8) if fmt == F.FMT_BF16 else q)
    if s is not None:
        ps = F.pack_scales(fmt, s, N, K)
        assert torch.equal(F.unpack_scales(fmt, ps, N, K), s)


@pytest.mark.parametrize("fmt", [F.FMT_FP8, F.FMT_MXFP4, F.FMT_NVFP4])
def test_quantiser_error_bounds(fmt):
    w = torch.randn((2, 256, 512)) * 0.02
    q, s, gs = F.quantize(fmt, w)
    back = F.dequantize(fmt, q, s, gs)
    rel = float((back - w).norm() / w.norm())
    assert rel < {F.FMT_FP8: 0.04, F.FMT_MXFP4: 0.2, F.FMT_NVFP4: 0.15}[fmt]


def _i8_marked_layer(seed=70):
    """MXFP4 layer with three weight rows spread beyond 3 e8m0 steps: gate row 5
    of expert 1 (5 steps), up row 9 of expert 2 (4), down row 7 of expert 3 (6)."""
    E, H, I = 4, 256, 256
    d = dense_to_numpy(F.FMT_MXFP4, make_dense_layer(F.FMT_MXFP4, E, H, I, seed=seed))
    s13, s2 = d["s13"].copy(), d["s2"].copy()
    for plane, e, row, spread in ((s13, 1, 5, 5), (s13, 2, I + 9, 4), (s2, 3, 7, 6)):
        m = int(plane[e, row].min())
        plane[e, row, 0], plane[e, row, 1] = m + spread, m
    d["s13"], d["s2"] = s13, s2
    return d, E, H, I


def _deq_row(w, s, n):
    """float64 dequantised MXFP4 row n of one expert ([N][K/2] codes, [N][K/32] e8m0)."""
    e2m1 = np.array(F.E2M1_VALUES, np.float64)
    v = np.empty(w.shape[1] * 2)
    v[0::2], v[1::2] = e2m1[w[n] & 15], e2m1[w[n] >> 4]
    return v * np.repeat(2.0 ** (s[n].astype(np.float64) - 127), 32)


def _silu_bf16(g, u):
    act = np.array([oracle.lib().xo_silu_gate(float(a), float(b), 0.0, 1.0, 0.0)
                    for a, b in zip(g, u)], np.float32)
    return oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(act))


def test_i8_marked_rows_take_the_fp32_path():
    """A token routed to one expert with weight 1: the layer's columns equal
    the integer path (oracle.i8_gemm, pinned by its closed form above) except
    the marked rows' columns, which equal the fp32 dot of the bf16 operand with
    the dequantised row (float64 here) -- gate/up (expert 1, gate row 5) and
    down (expert 3, row 7).  Without the fallback the integer path would use
    the wrapped int8 weights and miss."""
    d, E, H, I = _i8_marked_layer()
    rng = np.random.default_rng(71)
    x = oracle.f32_to_bf16_bits(rng.standard_normal((2, H)).astype(np.float32))
    ids = np.array([[1], [3]], np.int32)
    wts = np.ones((2, 1), np.float32)
    got = oracle.moe_layer_i8(x, ids, wts, E, 0, H, I, d["w13"], d["s13"], d["w2"], d["s2"])
    for t, e in ((0, 1), (1, 3)):
        xf = oracle.bf16_bits_to_f32(x[t])
        _, gu, _ = oracle.i8_gemm(xf[None, :], d["w13"][e], d["s13"][e])
        gu = gu[0].astype(np.float64)
        marked13 = [i for i in range(I)
                    if np.ptp(d["s13"][e][i]) > 3 or np.ptp(d["s13"][e][I + i]) > 3]
        for i in marked13:
            gu[i] = np.dot(xf.astype(np.float64), _deq_row(d["w13"][e], d["s13"][e], i))
            gu[I + i] = np.dot(xf.astype(np.float64), _deq_row(d["w13"][e], d["s13"][e], I + i))
        act = _silu_bf16(gu[:I].astype(np.float32), gu[I:].astype(np.float32))
        _, y, _ = oracle.i8_gemm(act[None, :], d["w2"][e], d["s2"][e])
        y = y[0].astype(np.float64)
        marked2 = [h for h in range(H) if np.ptp(d["s2"][e][h]) > 3]
        for h in marked2:
            y[h] = np.dot(act.astype(np.float64), _deq_row(d["w2"][e], d["s2"][e], h))
        assert marked13 or marked2
        np.testing.assert_allclose(got[t], y, rtol=1e-5, atol=1e-7)
        # the wrapped integer weights would miss the marked columns
        _, ywrap, _ = oracle.i8_gemm(act[None, :], d["w2"][e], d["s2"][e])
        for h in marked2:
            assert abs(ywrap[0, h] - y[h]) > 0.1 * abs(y[h]) + 1e-3


@pytest.mark.skipif(not oracle.ref_available("avx512_vnni"),
                    reason="reference engine VNNI build not available")
def test_i8_marked_rows_vs_reference_engine():
    """The reference engine with the ALIGN gate on routes the tiles holding
    the marked rows to its fp32 path (its tiles are per CPU thread slice, so
    which unmarked columns share that path depends on the thread count).  The
    oracle's per-column choice is no further from the engine than the integer
    path itself is from the fp32 layer."""
    d, E, H, I = _i8_marked_layer()
    rng = np.random.default_rng(72)
    T, K = 8, 2
    x = oracle.f32_to_bf16_bits(rng.standard_normal((T, H)).astype(np.float32))
    ids, wts = random_routing(T, K, E, seed=73)
    got = oracle.moe_layer_i8(x, ids, wts, E, 0, H, I, d["w13"], d["s13"], d["w2"], d["s2"])
    f32 = oracle.moe_layer(F.FMT_MXFP4, x, ids, wts, E, 0, H, I, d["w13"], d["s13"], d["w2"],
                           d["s2"])
    L = oracle.ref_lib("avx512_vnni")
    eng = oracle.RefEngine(F.FMT_MXFP4, E, K, H, I, d["w13"], d["s13"], d["w2"], d["s2"],
                           isa="avx512_vnni")
    L.xref_set_int8(1, 1 << 30)
    try:
        ref = eng.forward(x, ids.astype(np.uint32), wts)
    finally:
        L.xref_set_int8(0, 0)
        eng.close()
    assert rel_l2(got, ref) <= rel_l2(got, f32)
    assert rel_l2(ref, f32) < 0.1   # the engine did not run wrapped weights either
