"""Shared test helpers: seeded synthetic layers and the parity tolerance."""
from __future__ import annotations

import os
import types

import numpy as np
import torch

import oracle
from xtu_moe_amd import formats as F

# bf16 layer outputs vs the dequantized-fp32 oracle (the parity bar)
MAX_ABS = 2e-2
REL_L2 = 5e-3


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def check_close(out, ref, *, bf16_out: bool, what: str = ""):
    """fp32 outputs: max-abs <= 2e-2 and rel-L2 <= 5e-3.  bf16 outputs: the same
    rel-L2, and max-abs <= 2e-2 plus half a bf16 ulp of the reference value
    (the final rounding of the output itself)."""
    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(out - ref)
    slack = np.abs(ref) * 2.0 ** -8 if bf16_out else 0.0
    worst = float(np.max(err - slack)) if err.size else 0.0
    r = rel_l2(out, ref)
    assert worst <= MAX_ABS, f"{what}: max-abs excess {worst:.3e} > {MAX_ABS}"
    assert r <= REL_L2, f"{what}: rel-L2 {r:.3e} > {REL_L2}"
    return r


def make_dense_layer(fmt: int, E_total: int, H: int, I: int, seed: int = 0, std: float = 0.02,
                     split_gate_up: bool = False):
    """Dense checkpoint tensors (CPU torch) of E_total experts drawn N(0, std)
    and quantised; split_gate_up: NVFP4 gate and up halves quantised apart
    (gs13 [E, 2], the two scales differ), the up half drawn at 3 std."""
    g = torch.Generator().manual_seed(seed)
    w13 = torch.randn((E_total, 2 * I, H), generator=g) * std
    w2 = torch.randn((E_total, H, I), generator=g) * std
    if split_gate_up:
        w13[:, I:] *= 3.0
    w13q, s13, gs13 = (F.quantize_w13 if split_gate_up else F.quantize)(fmt, w13)
    w2q, s2, gs2 = F.quantize(fmt, w2)
    return dict(w13=w13q, s13=s13, gs13=gs13, w2=w2q, s2=s2, gs2=gs2)


def dense_to_numpy(fmt: int, d: dict) -> dict:
    out = {}
    for k, v in d.items():
        if v is None:
            out[k] = None
        elif fmt == F.FMT_BF16 and k in ("w13", "w2"):
            out[k] = v.contiguous().view(torch.int16).numpy().view(np.uint16)
        else:
            out[k] = v.contiguous().numpy()
    return out


def bf16_tensor_to_bits(x: torch.Tensor) -> np.ndarray:
    return x.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def oracle_layer(fmt, dn: dict, x_bits, ids, wts, E, NS, H, I, limit=0.0):
    return oracle.moe_layer(fmt, x_bits, ids, wts, E, NS, H, I, dn["w13"], dn["s13"], dn["w2"],
                            dn["s2"], dn["gs13"], dn["gs2"], limit=limit)


def random_routing(T, K, E, seed=0, invalid_frac=0.0, zero_frac=0.0):
    rng = np.random.default_rng(seed)
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32) if T else np.zeros((0, K), np.int32)
    wts = rng.random((T, K)).astype(np.float32) + 0.05
    if invalid_frac > 0:
        m = rng.random((T, K)) < invalid_frac
        ids[m] = rng.choice([-1, E, E + 3], size=int(m.sum()))
    if zero_frac > 0:
        m = rng.random((T, K)) < zero_frac
        wts[m] = 0.0
    return ids, wts


# ------------------------------------------------------------- INT4 (WNA16)
def int4_dense(E_, H_, I_, group, seed):
    """Dense INT4 checkpoint tensors (engine layout) of E_ experts."""
    g = torch.Generator().manual_seed(seed)
    w13 = torch.randn((E_, 2 * I_, H_), generator=g) * 0.05
    w2 = torch.randn((E_, H_, I_), generator=g) * 0.05
    a, b = F.quantize_int4(w13, group)
    c, e = F.quantize_int4(w2, group)
    return dict(w13=a, s13=b, w2=c, s2=e, gs13=None, gs2=None)


def gptq_pack(codes):
    """codes [E, N, K] (0..15) -> GPTQ int32 [E, K/8, N], nibble i of a word = k 8j+i."""
    c = codes.to(torch.int64).reshape(codes.shape[0], codes.shape[1], -1, 8)
    word = sum(c[..., i] << (4 * i) for i in range(8))
    word = torch.where(word >= 2 ** 31, word - 2 ** 32, word)
    return word.to(torch.int32).transpose(1, 2).contiguous()


def unpack_nibbles(b):
    """[..., K/2] bytes -> [..., K] codes, low nibble first."""
    return torch.stack([b & 15, b >> 4], -1).reshape(*b.shape[:-1], b.shape[-1] * 2)


def int4_layer(E_, H_, I_, seed):
    """A GPTQ-style INT4 layer object (int32 qweight / transposed scales /
    symmetric qzeros) and its dense tensors."""
    d = int4_dense(E_, H_, I_, 128, seed)
    d["s13"], d["s2"] = d["s13"].half().float(), d["s2"].half().float()   # GPTQ keeps fp16
    P = torch.nn.Parameter
    layer = types.SimpleNamespace(
        w13_qweight=P(gptq_pack(unpack_nibbles(d["w13"])), requires_grad=False),
        w2_qweight=P(gptq_pack(unpack_nibbles(d["w2"])), requires_grad=False),
        w13_scales=P(d["s13"].transpose(1, 2).half(), requires_grad=False),
        w2_scales=P(d["s2"].transpose(1, 2).half(), requires_grad=False),
        w13_qzeros=torch.full((E_, H_ // 128, 2 * I_ // 8), 0x77777777, dtype=torch.int32),
        top_k=3, renormalize=True, swiglu_limit=7.0)
    return d, layer


def cover_tokens(ids, E: int, n_last: int = 8, seed: int = 0):
    """Tokens of a batch that together route to every expert the batch uses
    (ids in [0, E)): for n_last random experts the last token routed to them
    (its pair sits in the expert's last, partial M tile), then a greedy cover
    (the token reaching the most experts not yet covered, lowest index on
    ties).  Returns (sorted tokens, the set of experts they cover)."""
    ids = np.asarray(ids)
    valid = (ids >= 0) & (ids < E)
    used = set(np.unique(ids[valid]).tolist())
    rng = np.random.default_rng(seed)
    chosen = []
    for e in rng.choice(sorted(used), size=min(n_last, len(used)), replace=False):
        chosen.append(int(np.nonzero((ids == e).any(1))[0].max()))
    covered = set(ids[chosen][valid[chosen]].tolist()) if chosen else set()
    while covered != used:
        left = np.array(sorted(used - covered))
        gain = (np.isin(ids, left) & valid).sum(1)
        t = int(np.argmax(gain))
        chosen.append(t)
        covered |= set(ids[t][valid[t]].tolist())
    return sorted(set(chosen)), covered


ORACLE_THREADS = min(16, os.cpu_count() or 1)


def sampled_oracle(fmt, W, x, ids, wts, toks, limit=0.0, int8=False, alpha=1.0, beta=0.0):
    """The oracle layer for the tokens `toks` of a batch on device weights W:
    only their experts (remapped to 0..U-1) and the shared experts, at full H
    and I, one token per call spread over host threads (the oracle's C entry
    points release the interpreter lock)."""
    from concurrent.futures import ThreadPoolExecutor

    from xtu_moe_amd.synthetic import dense_experts
    ids_s = ids[toks].cpu().numpy()
    wts_s = wts[toks].cpu().numpy()
    valid = (ids_s >= 0) & (ids_s < W.E)
    used = np.unique(ids_s[valid])
    remap = {int(e): i for i, e in enumerate(used)}
    cids = np.where(valid, np.vectorize(lambda e: remap.get(int(e), -1))(ids_s), -1)
    cids = cids.astype(np.int32)
    dn = dense_experts(W, list(used) + [W.E + s for s in range(W.n_shared)])
    xb = bf16_tensor_to_bits(x[toks])
    U, NS, H, I = len(used), W.n_shared, W.H, W.I

    def one(i):
        sl = slice(i, i + 1)
        if int8:
            return oracle.moe_layer_i8(xb[sl], cids[sl], wts_s[sl], U, NS, H, I, dn["w13"],
                                       dn["s13"], dn["w2"], dn["s2"], limit=limit, alpha=alpha,
                                       beta=beta)
        return oracle.moe_layer(fmt, xb[sl], cids[sl], wts_s[sl], U, NS, H, I, dn["w13"],
                                dn["s13"], dn["w2"], dn["s2"], dn["gs13"], dn["gs2"], limit=limit,
                                alpha=alpha, beta=beta)

    with ThreadPoolExecutor(max_workers=ORACLE_THREADS) as ex:
        rows = list(ex.map(one, range(len(toks))))
    return np.concatenate(rows, 0) if rows else np.zeros((0, H), np.float32)


def threaded_oracle(fmt, dn: dict, x_bits, ids, wts, E, NS, H, I, limit=0.0):
    """oracle_layer over dense numpy weights, one token per call spread over
    host threads (the weights are read in place, never copied)."""
    from concurrent.futures import ThreadPoolExecutor

    def one(t):
        sl = slice(t, t + 1)
        return oracle_layer(fmt, dn, x_bits[sl], ids[sl], wts[sl], E, NS, H, I, limit=limit)

    with ThreadPoolExecutor(max_workers=ORACLE_THREADS) as ex:
        rows = list(ex.map(one, range(len(ids))))
    return np.concatenate(rows, 0) if rows else np.zeros((0, H), np.float32)
