"""Pins of the activation-triple restatement (tests/tri_ref.py) on the CPU:
the e2m3 / e2m1 value tables against the OCP definitions written out, the
round-to-nearest-even against a brute-force search over every code (ties to
the even code), the scale exponent against a search over exponents, the byte
layout against its inverse, and the reconstruction error against its bound
2^(e-9)."""
import numpy as np
import torch

from fp8pair_ref import wide_rows
from tri_ref import (e2m1_value, e2m3_value, rne_e2m1, rne_e2m3, tri_exponent, tri_join,
                     tri_split, tri_unpack)

E2M3_POS = [m / 8 for m in range(8)] + [1 + m / 8 for m in range(8)] + \
    [2 + m / 4 for m in range(8)] + [4 + m / 2 for m in range(8)]
E2M1_POS = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]


def test_value_tables():
    assert list(e2m3_value(np.arange(32))) == E2M3_POS
    assert list(e2m3_value(np.arange(32) | 0x20)) == [-v for v in E2M3_POS]
    assert list(e2m1_value(np.arange(8))) == E2M1_POS
    assert list(e2m1_value(np.arange(8) | 0x8)) == [-v for v in E2M1_POS]


def _brute(y, values, sign_bit):
    """IEEE conversion by search: the representable magnitude nearest |y|,
    ties to the even code, and the sign bit of y copied (-0 for a negative
    value that rounds to zero)."""
    codes = np.arange(len(values))
    d = np.abs(np.abs(y)[:, None] - values[None, :])
    best = d.min(1, keepdims=True)
    cand = np.where(d == best, codes[None, :], 1 << 20)
    even = np.where((cand & 1) == 0, cand, 1 << 20)
    pick = np.where(even.min(1) < (1 << 20), even.min(1), cand.min(1))
    return pick | np.where(np.signbit(y), sign_bit, 0)


def test_rne_e2m3_brute_force():
    y = np.concatenate([np.arange(-7.5 * 4096, 7.5 * 4096 + 1) / 4096.0, [-0.0]])
    c, q = rne_e2m3(y)
    want = _brute(y, np.array(E2M3_POS), 0x20)
    assert np.array_equal(c, want)
    assert np.array_equal(q, e2m3_value(c)) and np.array_equal(np.signbit(q), np.signbit(y))
    # ties resolve to the even code
    for t in (0.0625, 1.0625, 1.9375, 2.125, 3.875, 4.25, 7.25):
        ct, _ = rne_e2m3(np.array([t]))
        assert ct[0] % 2 == 0, t


def test_rne_e2m1_brute_force():
    y = np.concatenate([np.arange(-4 * 4096, 4 * 4096 + 1) / 4096.0, [-0.0]])
    c, q = rne_e2m1(y)
    want = _brute(y, np.array(E2M1_POS[:7]), 0x8)
    assert np.array_equal(c, want)
    assert np.array_equal(q, e2m1_value(c))


def test_exponent_is_smallest():
    rng = np.random.default_rng(0)
    amax = np.concatenate([
        (rng.random(2000) * 2.0 ** rng.integers(-120, 120, 2000)).astype(np.float32),
        np.float32(7.5) * np.exp2(np.arange(-100, 100)).astype(np.float32),
        np.nextafter(np.float32(7.5) * np.exp2(np.arange(-100, 100)).astype(np.float32),
                     np.float32(np.inf)),
    ]).astype(np.float32)
    # bf16 values only (what the split sees)
    amax = torch.from_numpy(amax).to(torch.bfloat16).float().numpy()
    e = tri_exponent(amax)
    for a, ee in zip(amax.astype(np.float64), e):
        assert a <= 7.5 * 2.0 ** ee
        assert ee == -127 or a > 7.5 * 2.0 ** (ee - 1)


def _rows():
    g = torch.Generator().manual_seed(3)
    a = torch.randn((64, 1024), generator=g).to(torch.bfloat16)
    b = wide_rows(48, 1024, seed=4)
    c = torch.zeros((4, 1024), dtype=torch.bfloat16)
    c[0, :32] = 3.0e38                      # near the bf16 maximum
    c[1, 32:64] = 1.0e-37                   # scale bytes below 4 / 8: pieces 2, 3 zero
    c[2, 64:96] = torch.linspace(-7.5, 7.5, 32)
    c[3, 96:128] = -0.0
    return torch.cat([a, b, c])


def test_layout_round_trip_and_error_bound():
    x = _rows()
    M, K = x.shape
    q, sq, codes = tri_split(x)
    assert q.shape == (M, 2 * K) and sq.shape == (M, K // 32)
    for got, want in zip(tri_unpack(q, K), codes):
        assert np.array_equal(got, want)
    xr = tri_join(q, sq, K)
    xf = x.float().numpy().astype(np.float64)
    err = np.abs(xr - xf).reshape(M, K // 32, 32)
    e = sq.astype(np.float64) - 127
    ok = sq >= 8
    bound = np.exp2(e - 9)
    assert np.all(err.max(-1)[ok] <= bound[ok])
    amax = np.abs(xf).reshape(M, K // 32, 32).max(-1)
    assert np.all(err.max(-1)[ok] <= 2.0 ** -10.9 * amax[ok] + 0.0)
    # N(0,1) rows: rms error ~1e-4 of the values (bf16 rounding itself is ~1.7e-3)
    n = xf[:64]
    rel = np.sqrt(((xr[:64] - n) ** 2).mean() / (n ** 2).mean())
    assert rel < 2e-4, rel
    # a plausible packing mistake (pieces 2 and 3 swapped) is caught
    bad = tri_join(np.concatenate([q.reshape(M, -1, 64)[:, :, :24], q.reshape(M, -1, 64)[:, :, 48:],
                                   q.reshape(M, -1, 64)[:, :, 24:48]], -1).reshape(M, 2 * K),
                   sq, K)
    assert np.abs(bad - xf).max() > 1e-3


def test_first_two_pieces_error_bound():
    """The MXFP4 prefill's "duo" activations are the triples' first two
    pieces: x ~= 2^e (p1 + p2/16), |error| <= 2^(e-6) (half an e2m3 step of
    the second piece, scaled), rms ~7.5e-4 of the values for N(0,1) rows --
    inside the layer's 5e-3 bar with a wide margin; dropping the second
    piece (a plausible indexing mistake) misses the bound."""
    x = _rows()
    M, K = x.shape
    q, sq, (c1, c2, c3) = tri_split(x)
    e = sq.astype(np.float64) - 127
    v1, v2 = e2m3_value(c1), e2m3_value(c2)
    two = np.exp2(e)[..., None] * (v1 + np.where((sq >= 4)[..., None], v2, 0.0) / 16)
    xf = x.float().numpy().astype(np.float64).reshape(M, K // 32, 32)
    err = np.abs(two - xf).max(-1)
    ok = sq >= 8
    assert np.all(err[ok] <= np.exp2(e - 6)[ok])
    n = xf[:64]
    rel = np.sqrt(((two[:64] - n) ** 2).mean() / (n ** 2).mean())
    assert 2e-4 < rel < 1.5e-3, rel
    one = np.exp2(e)[..., None] * v1
    assert not np.all(np.abs(one - xf).max(-1)[ok] <= np.exp2(e - 6)[ok])
