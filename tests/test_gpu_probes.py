"""Device builtins the kernels rely on, checked in bounds against host expectations:
scaled fp4/fp8 converters (nibble order, scale handling), MFMA operand and result
lane layouts, and the fixed-sequence exp/sigmoid (bit-exact vs the oracle)."""
import numpy as np
import pytest
import torch

import oracle
from probes import probe_lib as _lib
from xtu_moe_amd.layer import _p, _stream

pytestmark = pytest.mark.gpu

E2M1 = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6], np.float32)


def _bf16_pair(words: np.ndarray):
    w = words.astype(np.uint32)
    lo = ((w & 0xFFFF) << 16).view(np.float32)
    hi = (w & 0xFFFF0000).view(np.float32)
    return lo, hi


@pytest.mark.parametrize("variant", ["xtu_probe_fp4", "xtu_probe_fp4_mul"])
def test_fp4_converter_power_of_two_scales(variant):
    scales = np.array([1.0, 2.0 ** -3, 2.0 ** 5, 2.0 ** -9, 2.0 ** 20], np.float32)
    s_d = torch.from_numpy(scales).cuda()
    out = torch.empty(len(scales) * 256, dtype=torch.int32, device="cuda")
    _lib.call(variant, _p(s_d), len(scales), _p(out), _stream())
    torch.cuda.synchronize()
    words = out.cpu().numpy().view(np.uint32).reshape(len(scales), 256)
    b = np.arange(256)
    for i, s in enumerate(scales):
        lo, hi = _bf16_pair(words[i])
        np.testing.assert_array_equal(lo, E2M1[b & 15] * s)
        np.testing.assert_array_equal(hi, E2M1[b >> 4] * s)


def test_fp4_mul_converter_e4m3_scales():
    # NVFP4: e4m3 scale values (not powers of two); products are exact in bf16
    t = oracle.e4m3_table()
    scales = t[[0x38, 0x3b, 0x45, 0x2d, 0x51, 0x01]].astype(np.float32)
    s_d = torch.from_numpy(scales).cuda()
    out = torch.empty(len(scales) * 256, dtype=torch.int32, device="cuda")
    _lib.call("xtu_probe_fp4_mul", _p(s_d), len(scales), _p(out), _stream())
    torch.cuda.synchronize()
    words = out.cpu().numpy().view(np.uint32).reshape(len(scales), 256)
    b = np.arange(256)
    for i, s in enumerate(scales):
        lo, hi = _bf16_pair(words[i])
        np.testing.assert_array_equal(lo, (E2M1[b & 15] * s).astype(np.float32))
        np.testing.assert_array_equal(hi, (E2M1[b >> 4] * s).astype(np.float32))


def test_fp8_converter_all_bytes():
    out = torch.empty(256, dtype=torch.int32, device="cuda")
    _lib.call("xtu_probe_fp8", _p(out), _stream())
    torch.cuda.synchronize()
    lo, _ = _bf16_pair(out.cpu().numpy().view(np.uint32))
    ref = oracle.e4m3_table()
    ok = np.array([b not in (0x7F, 0xFF) for b in range(256)])
    np.testing.assert_array_equal(lo[ok], ref[ok])


def _bf16_small_ints(shape, rng):
    v = rng.integers(-8, 9, size=shape).astype(np.float32)
    return v, oracle.f32_to_bf16_bits(v)


@pytest.mark.parametrize("which,shape_a,shape_b", [(0, (16, 32), (32, 16)), (1, (32, 16), (16, 32))])
def test_mfma_bf16_layouts(which, shape_a, shape_b):
    rng = np.random.default_rng(which)
    a, ab = _bf16_small_ints(shape_a, rng)
    b, bb = _bf16_small_ints(shape_b, rng)
    A = torch.from_numpy(ab.view(np.int16)).cuda()
    B = torch.from_numpy(bb.view(np.int16)).cuda()
    C = torch.zeros((shape_a[0], shape_b[1]), dtype=torch.float32, device="cuda")
    _lib.call("xtu_probe_mfma", which, _p(A), _p(B), _p(C), _stream())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(C.cpu().numpy(), a @ b)


def test_mfma_i8_layout():
    rng = np.random.default_rng(7)
    a = rng.integers(-127, 128, size=(32, 32)).astype(np.int8)
    b = rng.integers(-96, 97, size=(32, 32)).astype(np.int8)
    A = torch.from_numpy(a).cuda()
    B = torch.from_numpy(b).cuda()
    C = torch.zeros((32, 32), dtype=torch.int32, device="cuda")
    _lib.call("xtu_probe_mfma", 2, _p(A), _p(B), _p(C), _stream())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(C.cpu().numpy(), a.astype(np.int64) @ b.astype(np.int64))


def test_exp_sigmoid_bit_exact():
    rng = np.random.default_rng(3)
    x = np.concatenate([np.linspace(-90, 90, 20001, dtype=np.float32),
                        rng.standard_normal(20000).astype(np.float32) * 4,
                        np.array([0.0, -0.0, 1e-30, -1e-30, 88.4, -86.9, 87.0, -87.0], np.float32)])
    xd = torch.from_numpy(x).cuda()
    e = torch.empty_like(xd)
    s = torch.empty_like(xd)
    _lib.call("xtu_probe_exp", _p(xd), x.size, _p(e), _p(s), _stream())
    torch.cuda.synchronize()
    L = oracle.lib()
    ref_e = np.array([L.xo_expf(float(v)) for v in x], np.float32)
    ref_s = np.array([L.xo_sigmoid(float(v)) for v in x], np.float32)
    np.testing.assert_array_equal(e.cpu().numpy().view(np.uint32), ref_e.view(np.uint32))
    np.testing.assert_array_equal(s.cpu().numpy().view(np.uint32), ref_s.view(np.uint32))


def test_scaled_mfma_fp8_a_fp4_b_layout():
    """v_mfma_scale_f32_16x16x128_f8f6f4 with an e4m3 A and an e2m1 B, the
    layout the 16x16x128 exact-pair kernel relies on (MXFP4 and FP8 prefill
    at shapes the 32x32x64 kernels do not take): A lane 16q + r is row r with
    bytes 0..15 = k 16q.. and bytes 16..31 = k 64 + 16q..; B lane 16g + c is
    column c with nibble j (low nibble first) = k 32g + j -- one P16 MXFP4
    chunk; the scale byte of row r (column c) for the 32-k block b comes from
    lane 16b + r (16b + c).  Values are chosen so every sum is exact in fp32."""
    rng = np.random.default_rng(11)
    # e4m3 codes with exponent field 5..9 (|v| in [2^-2, 2^2 * 1.875]), random sign
    a_codes = (rng.integers(5, 10, (16, 128)) << 3 | rng.integers(0, 8, (16, 128))
               | (rng.integers(0, 2, (16, 128)) << 7)).astype(np.uint8)
    b_codes = rng.integers(0, 16, (16, 128)).astype(np.uint8)    # [col][k] e2m1 nibbles
    sa = rng.integers(126, 129, (16, 4)).astype(np.uint8)        # [row][block]
    sb = rng.integers(126, 129, (16, 4)).astype(np.uint8)        # [col][block]
    A = np.zeros((64, 32), np.uint8)
    B = np.zeros((64, 32), np.uint8)
    la, lb = np.zeros(64, np.uint8), np.zeros(64, np.uint8)
    for q in range(4):
        for r in range(16):
            lane = 16 * q + r
            A[lane, :16] = a_codes[r, 16 * q:16 * q + 16]
            A[lane, 16:] = a_codes[r, 64 + 16 * q:64 + 16 * q + 16]
            nib = b_codes[r, 32 * q:32 * q + 32]
            B[lane, :16] = nib[0::2] | (nib[1::2] << 4)
            la[lane], lb[lane] = sa[r, q], sb[r, q]
    dev = "cuda"
    tA = torch.from_numpy(A.view(np.int32).copy()).to(dev)
    tB = torch.from_numpy(B.view(np.int32).copy()).to(dev)
    tsa, tsb = torch.from_numpy(la).to(dev), torch.from_numpy(lb).to(dev)
    C = torch.zeros(64 * 4, dtype=torch.float32, device=dev)
    _lib.call("xtu_probe_mfma_scaled_fp4b", _p(tA), _p(tB), _p(tsa), _p(tsb), _p(C), _stream())
    torch.cuda.synchronize()
    c = C.cpu().numpy().reshape(64, 4)
    got = np.zeros((16, 16))
    for lane in range(64):
        for i in range(4):
            got[4 * (lane // 16) + i, lane % 16] = c[lane, i]
    av = oracle.e4m3_table().astype(np.float64)[a_codes] * np.repeat(2.0 ** (sa - 127.0), 32, 1)
    bv = E2M1.astype(np.float64)[b_codes] * np.repeat(2.0 ** (sb - 127.0), 32, 1)
    np.testing.assert_array_equal(got, av @ bv.T)
