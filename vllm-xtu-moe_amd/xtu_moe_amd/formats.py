"""Expert-weight formats: quantisers for synthetic data and the P16 packing.

Checkpoint ("dense") layouts follow the reference engine
(xiaotu_moe/csrc/moe/moe_v2.hpp:454-470, moe_v2_packed4_w4a8.inc:1966-1976,
moe_v2_fp8.hpp:1-11):

* MXFP4: codes [E][N][K/2] u8 (low nibble = even k), e8m0 [E][N][K/32] u8;
* NVFP4: codes as MXFP4, e4m3 [E][N][K/16] u8, fp32 global scale [E];
* FP8:   e4m3 [E][N][K] u8, fp32 block scales [E][N/128][K/128];
* BF16:  [E][N][K] bf16.

The device layout is P16: per expert, [N/16][K/SB][4][16][16 bytes] where a
16-byte chunk holds 32 fp4 codes, 16 fp8 codes or 8 bf16 values of one row,
so a wave64 loading 16 bytes per lane reads one contiguous KiB
(lane = 16 * chunk + row).  fp4 scales follow the same (panel, super-block,
chunk, row) order; fp8 block scales keep their dense layout.

The quantisers are the build's own (OCP MX rule for MXFP4, amax/448 blocks for
FP8, two-level amax scaling for NVFP4); the codes they produce are the test
and benchmark inputs, not a parity subject.
"""
from __future__ import annotations

import torch

FMT_BF16, FMT_FP8, FMT_MXFP4, FMT_NVFP4, FMT_INT4 = 0, 1, 2, 3, 4
FMT_NAMES = {FMT_BF16: "bf16", FMT_FP8: "fp8", FMT_MXFP4: "mxfp4", FMT_NVFP4: "nvfp4",
             FMT_INT4: "int4"}
# INT4 / WNA16 (the engine's MOE_WNA16): nibble codes (low nibble = even k),
# value = code - 8, times an fp32 scale per (row, group of INT4_GROUP k);
# computed by the host engine
INT4_GROUPS = (32, 64, 128)
INT4_GROUP = 128

E2M1_VALUES = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
               -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0)


def fmt_of(name) -> int:
    if isinstance(name, int):
        return name
    inv = {v: k for k, v in FMT_NAMES.items()}
    return inv[str(name).lower()]


# ------------------------------------------------------------------ quantisers
def _e2m1_codes(v: torch.Tensor) -> torch.Tensor:
    """Round-to-nearest-even onto the e2m1 grid, saturating at +-6 -> 4-bit codes."""
    a = v.abs()
    mag = ((a > 0.25).to(torch.uint8) + (a >= 0.75).to(torch.uint8) + (a > 1.25).to(torch.uint8)
           + (a >= 1.75).to(torch.uint8) + (a > 2.5).to(torch.uint8) + (a >= 3.5).to(torch.uint8)
           + (a > 5.0).to(torch.uint8))
    sign = ((v < 0) & (mag > 0)).to(torch.uint8) << 3
    return mag | sign


def _pack_nibbles(codes: torch.Tensor) -> torch.Tensor:
    return codes[..., 0::2] | (codes[..., 1::2] << 4)


def quantize_mxfp4(w: torch.Tensor):
    """w [..., N, K] float -> (codes [..., N, K/2] u8, e8m0 [..., N, K/32] u8)."""
    *lead, N, K = w.shape
    wb = w.float().reshape(*lead, N, K // 32, 32)
    amax = wb.abs().amax(-1)
    e = torch.floor(torch.log2(amax.clamp_min(2.0 ** -126))) - 2.0
    e = torch.where(amax > 0, e, torch.full_like(e, -127.0)).clamp(-127.0, 127.0)
    scale = torch.exp2(e)
    codes = _e2m1_codes(wb / scale[..., None]).reshape(*lead, N, K)
    return _pack_nibbles(codes).contiguous(), (e + 127.0).to(torch.uint8).contiguous()


def quantize_nvfp4(w: torch.Tensor):
    """w [E, N, K] -> (codes [E,N,K/2] u8, e4m3 scale bytes [E,N,K/16] u8, gs [E] fp32)."""
    E, N, K = w.shape
    wf = w.float()
    amax_t = wf.abs().reshape(E, -1).amax(-1)
    gs = (amax_t / (448.0 * 6.0)).clamp_min(1e-30)
    wb = wf.reshape(E, N, K // 16, 16)
    sblk = (wb.abs().amax(-1) / 6.0) / gs[:, None, None]
    s8 = sblk.clamp(max=448.0).to(torch.float8_e4m3fn)
    sq = s8.float() * gs[:, None, None]
    v = torch.where(sq[..., None] > 0, wb / sq[..., None].clamp_min(1e-30), torch.zeros_like(wb))
    codes = _e2m1_codes(v).reshape(E, N, K)
    return _pack_nibbles(codes).contiguous(), s8.view(torch.uint8).contiguous(), gs.float().contiguous()


def quantize_fp8_block(w: torch.Tensor):
    """w [..., N, K] -> (e4m3 codes [..., N, K] u8, fp32 scales [..., N/128, K/128])."""
    *lead, N, K = w.shape
    wb = w.float().reshape(*lead, N // 128, 128, K // 128, 128)
    amax = wb.abs().amax(dim=(-3, -1))
    s = torch.where(amax > 0, amax / 448.0, torch.ones_like(amax))
    q = (wb / s[..., :, None, :, None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return q.view(torch.uint8).reshape(*lead, N, K).contiguous(), s.float().contiguous()


def quantize_int4(w: torch.Tensor, group: int = INT4_GROUP):
    """w [..., N, K] -> (codes [..., N, K/2] u8 (value = code - 8), fp32 scales
    [..., N, K/group]): symmetric, the group maximum at +-7 steps."""
    *lead, N, K = w.shape
    wb = w.float().reshape(*lead, N, K // group, group)
    amax = wb.abs().amax(-1)
    s = torch.where(amax > 0, amax / 7.0, torch.ones_like(amax))
    q = torch.round(wb / s[..., None]).clamp(-8, 7).to(torch.int16) + 8
    codes = q.to(torch.uint8).reshape(*lead, N, K)
    return _pack_nibbles(codes).contiguous(), s.float().contiguous()


def quantize(fmt: int, w: torch.Tensor):
    """Dense checkpoint tensors (w, s, gs) of `w` [E, N, K] in format `fmt`."""
    if fmt == FMT_INT4:
        c, s = quantize_int4(w)
        return c, s, None
    if fmt == FMT_MXFP4:
        c, s = quantize_mxfp4(w)
        return c, s, None
    if fmt == FMT_NVFP4:
        return quantize_nvfp4(w)
    if fmt == FMT_FP8:
        c, s = quantize_fp8_block(w)
        return c, s, None
    return w.to(torch.bfloat16).contiguous(), None, None


def quantize_w13(fmt: int, w13: torch.Tensor):
    """quantize() of a gate/up weight [E, 2I, H].  NVFP4 quantises the gate
    and up halves separately, each with its own second-level scale (gs
    [E, 2]: gate, up), as a checkpoint's w1 / w3 are; other formats are
    quantize() of the whole."""
    if fmt != FMT_NVFP4:
        return quantize(fmt, w13)
    I = w13.shape[1] // 2
    cg, sg, gg = quantize_nvfp4(w13[:, :I])
    cu, su, gu = quantize_nvfp4(w13[:, I:])
    return (torch.cat([cg, cu], 1).contiguous(), torch.cat([sg, su], 1).contiguous(),
            torch.stack([gg, gu], 1).contiguous())


# ---------------------------------------------------------------- dequantisers
def e4m3_table(device=None) -> torch.Tensor:
    return torch.arange(256, dtype=torch.uint8, device=device).view(torch.float8_e4m3fn).float()


def dequantize(fmt: int, w: torch.Tensor, s=None, gs=None) -> torch.Tensor:
    """Dense checkpoint tensors -> fp32 [E, N, K] (exact)."""
    if fmt == FMT_BF16:
        return w.float()
    if fmt == FMT_FP8:
        v = w.view(torch.float8_e4m3fn).float()
        E, N, K = v.shape
        return (v.reshape(E, N // 128, 128, K // 128, 128) * s[:, :, None, :, None]).reshape(E, N, K)
    vals = (tuple(float(c - 8) for c in range(16)) if fmt == FMT_INT4 else E2M1_VALUES)
    lut = torch.tensor(vals, dtype=torch.float32, device=w.device)
    lo, hi = lut[(w & 15).long()], lut[(w >> 4).long()]
    v = torch.stack([lo, hi], -1).reshape(*w.shape[:-1], w.shape[-1] * 2)
    if fmt == FMT_INT4:
        return v * s.float().repeat_interleave(v.shape[-1] // s.shape[-1], -1)
    if fmt == FMT_MXFP4:
        return v * torch.exp2(s.float() - 127.0).repeat_interleave(32, -1)
    sc = e4m3_table(w.device)[s.long()] * gs[:, None, None]
    return v * sc.repeat_interleave(16, -1)


# ---------------------------------------------------------------------- packing
def row_bytes(fmt: int, K: int) -> int:
    return {FMT_BF16: 2 * K, FMT_FP8: K, FMT_MXFP4: K // 2, FMT_NVFP4: K // 2,
            FMT_INT4: K // 2}[fmt]


def pack_weight(fmt: int, w: torch.Tensor) -> torch.Tensor:
    """Dense [E, N, K(packed)] -> P16 bytes [E, N*row_bytes] u8."""
    E, N = w.shape[0], w.shape[1]
    b = w.contiguous().view(torch.uint8).reshape(E, N, -1)
    RB = b.shape[-1]
    assert N % 16 == 0 and RB % 64 == 0, (N, RB)
    p = b.reshape(E, N // 16, 16, RB // 64, 4, 16).permute(0, 1, 3, 4, 2, 5)
    return p.contiguous().reshape(E, N * RB)


def unpack_weight(fmt: int, p: torch.Tensor, N: int, K: int) -> torch.Tensor:
    """P16 bytes -> dense checkpoint tensor (inverse of pack_weight)."""
    E = p.shape[0]
    RB = row_bytes(fmt, K)
    d = p.reshape(E, N // 16, RB // 64, 4, 16, 16).permute(0, 1, 4, 2, 3, 5).contiguous()
    d = d.reshape(E, N, RB)
    return d.view(torch.bfloat16) if fmt == FMT_BF16 else d


# fp4 scale groups: per 16-row panel, the scales of UG consecutive 128-k
# super-blocks are stored [4 chunk q][16 row r][16 bytes] (16 bytes = UG
# one-byte MXFP4 scales or UG two-byte NVFP4 scale pairs), so one 16-byte load
# hands the lane that reads chunk (q, r) the scales of UG super-blocks.  The
# last group of a panel is zero-padded.
SCALE_GROUP = {FMT_MXFP4: 16, FMT_NVFP4: 8}


def scale_groups(fmt: int, K: int) -> int:
    ug = SCALE_GROUP[fmt]
    return (K // 128 + ug - 1) // ug


def scale_bytes(fmt: int, N: int, K: int, group: int = INT4_GROUP) -> int:
    """Packed scale bytes of one [N, K] matrix (per expert)."""
    if fmt == FMT_INT4:
        return N * (K // group) * 4
    if fmt in SCALE_GROUP:
        return N // 16 * scale_groups(fmt, K) * 1024
    if fmt == FMT_FP8:
        return (N // 128) * (K // 128) * 4
    return 0


def pack_scales(fmt: int, s, N: int, K: int):
    """Dense scales -> packed scale groups (fp4) / unchanged (fp8) / None (bf16)."""
    if s is None or fmt == FMT_BF16:
        return None
    E = s.shape[0]
    if fmt == FMT_INT4:   # fp32 [E, N, K/group], kept in row order for the host engine
        g = int4_group_of(s, K)
        if s.dtype != torch.float32 or s.dim() != 3 or s.shape[1] != N:
            raise ValueError(f"INT4 scales must be fp32 [E, {N}, {K}/group], got {s.dtype} "
                             f"{tuple(s.shape)}")
        return s.contiguous().reshape(E, N * (K // g))
    if fmt == FMT_FP8:
        if s.dtype != torch.float32 or tuple(s.shape[1:]) != (N // 128, K // 128):
            raise ValueError(f"FP8 block scales must be fp32 [E, {N // 128}, {K // 128}], "
                             f"got {s.dtype} {tuple(s.shape)}")
        return s.contiguous().reshape(E, -1)
    gk = 32 if fmt == FMT_MXFP4 else 16
    if s.element_size() != 1 or tuple(s.shape[1:]) != (N, K // gk):
        raise ValueError(f"{FMT_NAMES[fmt]} scales must be one byte each [E, {N}, {K // gk}], "
                         f"got {s.dtype} {tuple(s.shape)}")
    ug, nsb = SCALE_GROUP[fmt], K // 128
    G = scale_groups(fmt, K)
    per = 4 if fmt == FMT_MXFP4 else 8          # scale bytes per (row, super-block)
    d = s.contiguous().view(torch.uint8).reshape(E, N // 16, 16, nsb, per)
    if G * ug != nsb:
        d = torch.nn.functional.pad(d, (0, 0, 0, G * ug - nsb))
    if fmt == FMT_MXFP4:   # [p][r][g][u][q] -> [p][g][q][r][u]
        d = d.reshape(E, N // 16, 16, G, ug, 4).permute(0, 1, 3, 5, 2, 4)
    else:                  # [p][r][g][u][q][h] -> [p][g][q][r][u][h]
        d = d.reshape(E, N // 16, 16, G, ug, 4, 2).permute(0, 1, 3, 5, 2, 4, 6)
    return d.contiguous().reshape(E, -1)


def int4_group_of(s, K: int) -> int:
    """The k per scale of INT4 scales [E, N, K/group] (32, 64 or 128)."""
    if s.dim() != 3 or s.shape[-1] == 0 or K % s.shape[-1]:
        raise ValueError(f"INT4 scales {tuple(s.shape)} do not split K={K} into groups")
    g = K // s.shape[-1]
    if g not in INT4_GROUPS:
        raise ValueError(f"INT4 group of {g} k is not supported (groups: {INT4_GROUPS})")
    return g


def unpack_scales(fmt: int, p, N: int, K: int):
    if p is None or fmt == FMT_BF16:
        return None
    E = p.shape[0]
    if fmt == FMT_INT4:
        return p.reshape(E, N, -1)
    if fmt == FMT_FP8:
        return p.reshape(E, N // 128, K // 128)
    ug, nsb = SCALE_GROUP[fmt], K // 128
    G = scale_groups(fmt, K)
    if fmt == FMT_MXFP4:   # [p][g][q][r][u] -> [p][r][g][u][q]
        d = p.reshape(E, N // 16, G, 4, 16, ug).permute(0, 1, 4, 2, 5, 3)
        d = d.reshape(E, N // 16, 16, G * ug, 4)[:, :, :, :nsb]
        return d.contiguous().reshape(E, N, K // 32)
    d = p.reshape(E, N // 16, G, 4, 16, ug, 2).permute(0, 1, 4, 2, 5, 3, 6)
    d = d.reshape(E, N // 16, 16, G * ug, 4, 2)[:, :, :, :nsb]
    return d.contiguous().reshape(E, N, K // 16)


def algorithmic_bytes(fmt: int, N: int, K: int) -> int:
    """Bytes a weight stream of one [N, K] matrix must read: codes plus one
    scale per scaling block (no layout padding)."""
    w = N * K * {FMT_BF16: 2.0, FMT_FP8: 1.0, FMT_MXFP4: 0.5, FMT_NVFP4: 0.5, FMT_INT4: 0.5}[fmt]
    s = {FMT_BF16: 0, FMT_FP8: (N // 128) * (K // 128) * 4, FMT_MXFP4: N * K // 32,
         FMT_NVFP4: N * K // 16 + 4, FMT_INT4: N * (K // INT4_GROUP) * 4}[fmt]
    return int(w + s)


def expert_bytes(fmt: int, H: int, I: int) -> int:
    """HBM bytes of one expert (w13 + s13 + w2 + s2, plus NVFP4's two global
    scales) in format `fmt`, as packed."""
    w = 3 * H * I * {FMT_BF16: 2.0, FMT_FP8: 1.0, FMT_MXFP4: 0.5, FMT_NVFP4: 0.5}[fmt]
    s = scale_bytes(fmt, 2 * I, H) + scale_bytes(fmt, H, I)
    if fmt == FMT_NVFP4:
        s += 8
    return int(w + s)


def bf16_bits(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.bfloat16).contiguous().view(torch.int16)
