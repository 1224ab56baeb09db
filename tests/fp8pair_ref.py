"""CPU restatement of the exact e4m3-pair split of bf16 rows (the activation
format of the exact FP8 prefill GEMMs): per row and 32-k block,
x = hi * 2^(sa-127) + lo * 2^(sl-127), sa the smallest scale that puts the
block maximum at <= 448, hi = RNE e4m3 of x / 2^(sa-127), lo = e4m3 of 16x the
remainder, sl = sa - 4."""
import numpy as np
import torch


def fp8pair_split(x: torch.Tensor):
    """x: bf16 [M, K] (K % 32 == 0) -> hi, lo uint8 [M, K]; sa, sl uint8 [M, K/32]."""
    M, K = x.shape
    xf = x.float().reshape(M, K // 32, 32)
    amax = xf.abs().amax(-1)
    bits = amax.view(torch.int32)
    ex = (bits >> 23) & 0xFF
    frac = bits & 0x7FFFFF
    e = ex - 127 - 8 + (frac > 0x600000).to(torch.int32)
    e = torch.where(ex == 0, torch.full_like(e, -127), e).clamp(-127, 127)
    xs = torch.ldexp(xf.double(), (-e).double().unsqueeze(-1)).float()
    hi = xs.to(torch.float8_e4m3fn)
    r = (xs - hi.float()) * 16.0
    lo = r.to(torch.float8_e4m3fn)
    sa = (e + 127).to(torch.uint8)
    sl = (e + 127 - 4).clamp(min=0).to(torch.uint8)
    return (hi.view(torch.uint8).reshape(M, K), lo.view(torch.uint8).reshape(M, K), sa, sl)


def fp8pair_join(hi, lo, sa, sl) -> np.ndarray:
    """float64 hi * 2^(sa-127) + lo * 2^(sl-127)."""
    M, K = hi.shape
    h = torch.as_tensor(hi).view(torch.float8_e4m3fn).double().reshape(M, K // 32, 32)
    l = torch.as_tensor(lo).view(torch.float8_e4m3fn).double().reshape(M, K // 32, 32)
    sa = torch.as_tensor(sa).to(torch.float64) - 127
    sl = torch.as_tensor(sl).to(torch.float64) - 127
    v = torch.ldexp(h, sa.unsqueeze(-1)) + torch.ldexp(l, sl.unsqueeze(-1))
    return v.reshape(M, K).numpy()


def wide_rows(M, K, seed=0):
    """bf16 rows with N(0,1) values, blocks scaled over a wide range, zero
    blocks, isolated large values and negative zeros; no value is below 2^-13
    of its block's maximum (below 2^-13.8 the split may drop the last bit:
    hi is subnormal there)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((M, K), generator=g)
    scale = torch.pow(2.0, torch.randint(-40, 40, (M, K // 32), generator=g).float())
    x = (x.reshape(M, K // 32, 32) * scale.unsqueeze(-1)).reshape(M, K)
    if K >= 64:
        x[0, :32] = 0.0
        x[0, 32:64] = -0.0
    if M >= 2:
        x[1, 5] = 1.0e4
    if M >= 3 and K >= 96:
        x[2, 64:96] = torch.linspace(-3.0, 3.0, 32)
    xb = x.reshape(M, K // 32, 32)
    amax = xb.abs().amax(-1, keepdim=True)
    small = (xb.abs() < amax * 2.0 ** -13) & (xb != 0)
    xb[small] = torch.copysign(amax.expand_as(xb)[small] * 2.0 ** -13, xb[small])
    return xb.reshape(M, K).to(torch.bfloat16)
