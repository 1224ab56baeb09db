"""CPU restatement of the activation-triple split of bf16 rows (the activation
format of the MXFP4 prefill GEMMs on the double-rate fp6 / fp4 MFMA): per row
and 32-k block, with e the smallest exponent such that max|x| <= 7.5 * 2^e,

    x ~= 2^e * (p1 + p2 / 16 + p3 / 256),

p1 = RNE e2m3 of x / 2^e, p2 = RNE e2m3 of 16x the remainder, p3 = RNE e2m1
of 16x the next remainder (IEEE conversions: the sign is copied, so a
negative value rounding to zero is -0, and each remainder is taken from the
piece's decoded value, -0 included); the e8m0 byte is e + 127 and a piece whose scale
byte (e + 127 - 4, e + 127 - 8) would be negative is zero.  Layout of one
row: [K/64 steps][2 halves][p1 24 B | p2 24 B | p3 16 B], codes packed
little-endian (code j of p1 / p2 at bits 6j..6j+5, of p3 at bits 4j..4j+3).
Test infrastructure only."""
import numpy as np
import torch

E2M3_MAX = 7.5


def e2m3_value(code):
    """OCP FP6 E2M3 (bias 1, no inf / nan): code -> value."""
    code = np.asarray(code, dtype=np.int64)
    s = np.where(code & 0x20, -1.0, 1.0)
    E, m = (code >> 3) & 3, code & 7
    mag = np.where(E == 0, m / 8.0, (1.0 + m / 8.0) * np.exp2(E - 1.0))
    return s * mag


def e2m1_value(code):
    """OCP FP4 E2M1 (bias 1): code -> value."""
    code = np.asarray(code, dtype=np.int64)
    s = np.where(code & 0x8, -1.0, 1.0)
    E, m = (code >> 1) & 3, code & 1
    mag = np.where(E == 0, m / 2.0, (1.0 + m / 2.0) * np.exp2(E - 1.0))
    return s * mag


def rne_e2m3(y):
    """IEEE conversion to e2m3 (|y| <= 7.5): the magnitude rounded to nearest
    even on the grid (step 1/8 below 2, 1/4 below 4, 1/2 up to 7.5), the sign
    copied (a negative value rounding to zero gives -0); (code, value)."""
    y = np.asarray(y, dtype=np.float64)
    a = np.abs(y)
    inv = np.where(a < 2, 8.0, np.where(a < 4, 4.0, 2.0))
    n = np.rint(a * inv)
    c = np.where(inv == 8.0, n, np.where(inv == 4.0, n + 8, n + 16)).astype(np.int64)
    c = c | np.where(np.signbit(y), 0x20, 0)
    return c, e2m3_value(c)


def rne_e2m1(y):
    """IEEE conversion to e2m1 (|y| <= 4): magnitude rounded to nearest even
    (step 1/2 below 2, 1 below 4, 2 at 4), sign copied; (code, value)."""
    y = np.asarray(y, dtype=np.float64)
    a = np.abs(y)
    inv = np.where(a < 2, 2.0, np.where(a < 4, 1.0, 0.5))
    n = np.rint(a * inv)
    c = np.where(inv == 2.0, n, np.where(inv == 1.0, n + 2, n + 4)).astype(np.int64)
    c = c | np.where(np.signbit(y), 0x8, 0)
    return c, e2m1_value(c)


def tri_exponent(amax):
    """Smallest e with amax <= 7.5 * 2^e, from the fp32 bits (zero and
    subnormal blocks -127), clamped to [-127, 127]."""
    bits = np.asarray(amax, dtype=np.float32).view(np.int32).astype(np.int64)
    ex, frac = (bits >> 23) & 0xFF, bits & 0x7FFFFF
    e = ex - 127 - 2 + (frac > 0x700000)
    return np.clip(np.where(ex == 0, -127, e), -127, 127)


def tri_split(x: torch.Tensor):
    """x: bf16 [M, K] (K % 64 == 0) -> (q uint8 [M, 2K], sq uint8 [M, K/32],
    codes: (c1, c2, c3) int64 [M, K/32, 32])."""
    M, K = x.shape
    xf = x.float().numpy().reshape(M, K // 32, 32)
    amax = np.abs(xf).max(-1)
    e = tri_exponent(amax)
    s = e + 127
    y = np.ldexp(xf.astype(np.float64), (-e)[..., None])
    c1, q1 = rne_e2m3(y)
    y2 = (y - q1) * 16.0
    c2, q2 = rne_e2m3(y2)
    c3, _ = rne_e2m1((y2 - q2) * 16.0)
    c2 = np.where((s >= 4)[..., None], c2, 0)
    c3 = np.where((s >= 8)[..., None], c3, 0)
    nb = K // 32
    out = np.zeros((M, nb, 64), dtype=np.uint8)
    for piece, off in ((c1, 0), (c2, 24)):
        g = piece.reshape(M, nb, 8, 4)
        v = g[..., 0] | (g[..., 1] << 6) | (g[..., 2] << 12) | (g[..., 3] << 18)
        b = np.stack([v & 0xFF, (v >> 8) & 0xFF, (v >> 16) & 0xFF], -1).reshape(M, nb, 24)
        out[:, :, off:off + 24] = b
    p3 = c3.reshape(M, nb, 16, 2)
    out[:, :, 48:64] = p3[..., 0] | (p3[..., 1] << 4)
    # blocks 2j, 2j + 1 are the halves of step j's 128-byte line
    return (out.reshape(M, 2 * K), s.astype(np.uint8), (c1, c2, c3))


def tri_unpack(q: np.ndarray, K: int):
    """Inverse of the byte layout: q uint8 [M, 2K] -> codes (c1, c2, c3)."""
    M = q.shape[0]
    nb = K // 32
    b = np.asarray(q, dtype=np.int64).reshape(M, nb, 64)
    cs = []
    for off in (0, 24):
        t = b[:, :, off:off + 24].reshape(M, nb, 8, 3)
        v = t[..., 0] | (t[..., 1] << 8) | (t[..., 2] << 16)
        cs.append(np.stack([(v >> (6 * i)) & 0x3F for i in range(4)], -1).reshape(M, nb, 32))
    t = b[:, :, 48:64]
    cs.append(np.stack([t & 0xF, t >> 4], -1).reshape(M, nb, 32))
    return tuple(cs)


def tri_join(q: np.ndarray, sq: np.ndarray, K: int) -> np.ndarray:
    """float64 2^(s-127) * (p1 + p2 / 16 + p3 / 256) [M, K]."""
    c1, c2, c3 = tri_unpack(q, K)
    v = e2m3_value(c1) + e2m3_value(c2) / 16.0 + e2m1_value(c3) / 256.0
    M = q.shape[0]
    return np.ldexp(v, (np.asarray(sq, dtype=np.int64) - 127)[..., None]).reshape(M, K)
